// Decode / spec-verify GEMV (kernel 1): y[j, r] = inverse[j] * sum_b dot(W[r, b], q8[j, b])
// for m <= 16 activation rows, every wire format, weights streamed once from HBM.
//
// Reference: kai_dual::mmvq_dual (vllm_gguf_plugin/native/kernels/kai_dual_mmvq.cuh:258-327)
// and its launcher (:329-397). Design for gfx950 instead of warp32 CTAs:
//   * one wave64 owns R consecutive output rows; its 64 lanes walk the row's units
//     (kai_units.h) so each load instruction covers contiguous wire bytes;
//   * every unit's activation slice (all m rows) is loaded once and reused for the
//     R weight rows, which keeps L1/L2 traffic per weight byte low as m grows;
//   * integer dots with v_dot4_i32_i8, fp32 scale/accumulate per block;
//   * per-row totals by a wave64 DPP/swizzle reduction, no LDS or barrier;
//   * merged-projection epilogue: x inverse[j], F32 or BF16, strided store.
// Four independent waves per 256-thread workgroup. IQ3_S copies its 2 KiB grid
// into LDS once per workgroup.
#pragma once

#include "kai_iq3s_grid.h"
#include "kai_launch.h"
#include "kai_units.h"

namespace kai {

// Each translation unit that instantiates the IQ3_S kernel owns a copy of the grid.
static __device__ const uint32_t iq3s_grid_global[512] = {KAI_IQ3S_GRID_VALUES};

constexpr int MMVQ_THREADS = 256;
constexpr int MMVQ_WAVES = MMVQ_THREADS / WAVE;

template <int TYPE>
__device__ __forceinline__ Unit<TYPE> make_unit(int sub, const uint32_t *grid) {
    if constexpr (TYPE == IQ3_S) return Unit<TYPE>(sub, grid);
    else return Unit<TYPE>(sub);
}

__device__ __forceinline__ void store_out(void *dst, bool bf16, int64_t index, float v) {
    if (bf16) static_cast<uint16_t *>(dst)[index] = float_to_bf16_bits(v);
    else static_cast<float *>(dst)[index] = v;
}

// Occupancy floor per activation-row count: enough waves in flight to cover HBM
// latency, leaving registers for R x M accumulators and the prefetched units.
template <int M> constexpr int mmvq_min_waves() { return M <= 2 ? 4 : 2; }

template <int TYPE, int M, int R, bool TWO_PASS>
__global__ __launch_bounds__(MMVQ_THREADS) __attribute__((amdgpu_waves_per_eu(mmvq_min_waves<M>(), 8)))
void mmvq_kernel(
    const uint8_t *__restrict__ weight, int64_t row_bytes, int nrows, int units_per_row,
    const block_q8_1 *__restrict__ y1, const block_q8_1 *__restrict__ y2, int y_row_blocks,
    const float *__restrict__ inverse, void *__restrict__ dst, int64_t stride_dst, int dst_bf16) {
    using U = Unit<TYPE>;
    constexpr int BYTES = block_bytes(TYPE);
    __shared__ uint32_t grid_lds[TYPE == IQ3_S ? 512 : 1];
    if constexpr (TYPE == IQ3_S) {
        for (int i = threadIdx.x; i < 512; i += MMVQ_THREADS) grid_lds[i] = iq3s_grid_global[i];
        __syncthreads();
    }
    const int wave = threadIdx.x / WAVE;
    const int lane = threadIdx.x % WAVE;
    const int row0 = (blockIdx.x * MMVQ_WAVES + wave) * R;
    if (row0 >= nrows) return;

    const U unit = make_unit<TYPE>(lane % U::PER_BLOCK, grid_lds);
    const uint8_t *rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rows[r] = weight + static_cast<int64_t>(min(row0 + r, nrows - 1)) * row_bytes;

    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < M; ++j) acc[r][j] = 0.0f;

    // Software pipeline over the weight stream: the next unit's wire bytes are
    // requested before the current unit is multiplied, so one unit per row of HBM
    // reads stays in flight behind the arithmetic (activation slices hit L1/L2).
    typename U::W next[R];
    if (lane < units_per_row) {
#pragma unroll
        for (int r = 0; r < R; ++r) unit.load_w(next[r], rows[r] + static_cast<int64_t>(lane / U::PER_BLOCK) * BYTES);
    }
    for (int u = lane; u < units_per_row; u += WAVE) {
        const int blk = u / U::PER_BLOCK;
        typename U::P w[R];
#pragma unroll
        for (int r = 0; r < R; ++r) w[r] = unit.prep(next[r]);
        if (u + WAVE < units_per_row) {
            const int64_t nb = static_cast<int64_t>((u + WAVE) / U::PER_BLOCK) * BYTES;
#pragma unroll
            for (int r = 0; r < R; ++r) unit.load_w(next[r], rows[r] + nb);
        }
#pragma unroll
        for (int j = 0; j < M; ++j) {
            typename U::A a;
            unit.load_a(a, y1 + static_cast<int64_t>(j) * y_row_blocks, blk);
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r][j] += unit.dot(w[r], a);
            if constexpr (TWO_PASS) {
                typename U::A a2;
                unit.load_a(a2, y2 + static_cast<int64_t>(j) * y_row_blocks, blk);
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r][j] += unit.dot(w[r], a2);
            }
        }
    }

    // Every lane ends with every total; lane (r*M + j) stores item (r, j).
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int j = 0; j < M; ++j) {
            const float total = wave_sum(acc[r][j]);
            if (lane == (r * M + j) % WAVE && row0 + r < nrows) {
                store_out(dst, dst_bf16 != 0, static_cast<int64_t>(j) * stride_dst + row0 + r, total * inverse[j]);
            }
        }
    }
}

// Rows per wave: more rows reuse each activation slice more often (fewer L1/L2
// bytes per weight byte) at the cost of registers.
template <int M> constexpr int rows_per_wave() { return M <= 2 ? 2 : M <= 8 ? 4 : 2; }

template <int TYPE, int M>
static void launch_m(const void *weight, int64_t n, int64_t k, const block_q8_1 *y1, const block_q8_1 *y2,
                     const float *inverse, void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream) {
    constexpr int R = rows_per_wave<M>();
    constexpr int QK = block_elems(TYPE);
    const int64_t blocks_per_row = k / QK;
    const int64_t row_bytes = blocks_per_row * block_bytes(TYPE);
    const int units = static_cast<int>(blocks_per_row * Unit<TYPE>::PER_BLOCK);
    const int64_t rows_per_group = int64_t(MMVQ_WAVES) * R;
    const dim3 grid(static_cast<unsigned>((n + rows_per_group - 1) / rows_per_group));
    const auto *w = static_cast<const uint8_t *>(weight);
    const int yrb = static_cast<int>(k / QK8_1);
    if (y2) {
        if constexpr (M <= 8) {
            mmvq_kernel<TYPE, M, R, true><<<grid, MMVQ_THREADS, 0, stream>>>(
                w, row_bytes, static_cast<int>(n), units, y1, y2, yrb, inverse, dst, stride_dst, dst_bf16 ? 1 : 0);
        } else {
            throw Error("Two-pass activations are supported for up to 8 rows");
        }
    } else {
        mmvq_kernel<TYPE, M, R, false><<<grid, MMVQ_THREADS, 0, stream>>>(
            w, row_bytes, static_cast<int>(n), units, y1, y2, yrb, inverse, dst, stride_dst, dst_bf16 ? 1 : 0);
    }
}

// Per-type entry used by launch_mmvq; one translation unit per type keeps builds parallel.
template <int TYPE>
void launch_mmvq_type(const void *weight, int64_t n, int64_t k, int64_t m, const block_q8_1 *y1,
                      const block_q8_1 *y2, const float *inverse, void *dst, bool dst_bf16, int64_t stride_dst,
                      hipStream_t stream) {
    switch (m) {
#define KAI_M(MM) case MM: launch_m<TYPE, MM>(weight, n, k, y1, y2, inverse, dst, dst_bf16, stride_dst, stream); break;
        KAI_M(1) KAI_M(2) KAI_M(3) KAI_M(4) KAI_M(5) KAI_M(6) KAI_M(7) KAI_M(8)
        KAI_M(9) KAI_M(10) KAI_M(11) KAI_M(12) KAI_M(13) KAI_M(14) KAI_M(15) KAI_M(16)
#undef KAI_M
        default: throw Error("GEMV supports 1..16 activation rows");
    }
}

}  // namespace kai
