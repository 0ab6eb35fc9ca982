// Small-M GEMM on fp16 MFMA (kernel "mfv"): multi-sequence decode with up to 16
// activation rows, Y[m, n] = inverse[m] * sum_k a[m, k] w[n, k] for the row-normalised
// Q8_1 activation a = d8 * q8 and the dequantised K-quant weight w (reference:
// kai_fused_mmq_run, vllm_gguf_plugin/native/kernels/current_ggml_direct.cu:1196-1265).
//
// The operands and their arithmetic are those of the prefill GEMM (kai_mmf.cuh): exact
// fp16 integer weights sc * q * 2^-P dequantised in registers, a16 = half(d8 * q8) and the
// min-term operands from prepare_mmf_kernel, one fp32 accumulator per superblock unit.
// What changes is the shape: at m <= 16 the weight stream is the cost (one MFMA per 512
// weights) and the activation is tiny, so
//   * a wave owns 16 weight rows; the four waves of a workgroup (64 rows) run the same
//     superblocks in step, one barrier per superblock;
//   * the activation of one superblock (16 rows x 256 fp16 plus the min-term pairs,
//     9 KiB) goes to LDS once per workgroup by global_load_lds, whole 128-byte lines;
//     16-byte chunk c of activation row r sits at chunk c ^ r, so the MFMA operand reads
//     (16 rows, one chunk each) hit distinct banks;
//   * weight bytes (a lane's header and two 16-byte code runs per superblock) go straight
//     into registers, MFV_AHEAD superblocks ahead, like the activation stages;
//   * each lane derives the constants of its own weight row; the MFMA takes the
//     activation as A and the weights as B, so a lane's accumulator column is its own
//     weight row and the per-superblock rescale multiplies by its own ratio;
//   * when 64-row workgroups alone would leave the chip idle, the superblocks are split
//     over KS workgroups (grid.y) that write fp32 partial sums, added in a fixed order by
//     mfv_reduce_kernel.
// Loads and LDS DMAs are issued by asm the compiler does not track; every wait is an
// explicit vmcnt (vector memory completes in order) tied to the registers it guards.
#pragma once

#include "kai_mmf.cuh"

namespace kai {

constexpr int MFV_AHEAD = 2;                  // superblocks requested ahead
constexpr int MFV_RING = MFV_AHEAD + 1;       // activation stages and weight slots
constexpr int MFV_ABYTES = 16 * 512;          // a16 of 16 rows x 256 values
constexpr int MFV_TBYTES = 16 * 64;           // min-term pairs of 16 rows
constexpr int MFV_STAGE = MFV_ABYTES + MFV_TBYTES;

// 4 bytes per lane from base + voff to LDS at lds + 4 * lane.
__device__ __forceinline__ void mfv_dma4(const void *base, uint32_t voff, uint32_t lds) {
    __asm__ volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(base), "s"(lds)
                     : "memory");
}
template <int N>
__device__ __forceinline__ void mfv_wait(u4_t (&w)[3]) {
    __asm__ volatile("s_waitcnt vmcnt(%3)" : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]) : "n"(N) : "memory");
}

template <int TYPE>
__global__ __launch_bounds__(256) void mfv_kernel(const uint8_t *weight, int64_t row_bytes, int n, int k,
                                                  const uint16_t *a16, const uint8_t *tmin,
                                                  const float *__restrict__ inverse, int m, void *__restrict__ dst,
                                                  int64_t stride_dst, int dst_bf16, float *__restrict__ partial) {
    using F = MmfW<TYPE>;
    constexpr int SBB = F::SBB, TROW = F::TROW;
    static_assert(TROW == 64, "min-term pairs of 64 bytes per row and superblock");
    __shared__ __align__(16) uint8_t stage[MFV_RING][MFV_STAGE];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    const int col = lane & 15, g = lane >> 4;
    const int nsb = k >> 8, ks = int(gridDim.y), kz = int(blockIdx.y);
    const int s0 = kz * nsb / ks, s1 = (kz + 1) * nsb / ks;  // workgroup-uniform, s0 < s1
    const int r0 = __builtin_amdgcn_readfirstlane(int(blockIdx.x) * 64 + 16 * wave);

    // This wave's 16 weight rows (rows past n read zeros: an empty range past the end).
    const __amdgpu_buffer_rsrc_t wres =
        mmf_rsrc(weight + int64_t(min(r0, n)) * row_bytes, uint32_t(max(0, min(16, n - r0))) * uint32_t(row_bytes));
    const uint32_t hoff = uint32_t(col) * uint32_t(row_bytes);

    // Activation DMA roles. a16: chunk q = (2 wave + i) 64 + lane of the 512 per stage,
    // row q / 32 at physical chunk q % 32 holding logical chunk (q % 32) ^ row. Min-term
    // pairs: dword q = 64 wave + lane of the 256, row q / 16. Rows past m repeat m - 1.
    uint32_t aoff[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int q = (2 * wave + i) * 64 + lane, r = q >> 5;
        aoff[i] = uint32_t(min(r, m - 1)) * uint32_t(k) * 2u + 16u * uint32_t((q & 31) ^ r);
    }
    const int tq = wave * 64 + lane;
    const uint32_t toff = uint32_t(min(tq >> 4, m - 1)) * uint32_t(nsb) * 64u + 4u * uint32_t(tq & 15);

    auto issue = [&](u4_t (&w)[3], int sb, int st) {
        const uint8_t *ab = reinterpret_cast<const uint8_t *>(a16) + size_t(sb) * 512;
        mmf_dma16(ab, aoff[0], lds_addr(&stage[st][(2 * wave) * 1024]));
        mmf_dma16(ab, aoff[1], lds_addr(&stage[st][(2 * wave + 1) * 1024]));
        mfv_dma4(tmin + size_t(sb) * 64, toff, lds_addr(&stage[st][MFV_ABYTES + wave * 256]));
        const uint32_t sw = uint32_t(sb) * SBB;
        w[0] = mmf_load16(wres, hoff, sw);                               // header
        w[1] = mmf_load16(wres, hoff + 16u + 16u * uint32_t(g), sw);     // codes [16g, +16) of qs
        w[2] = mmf_load16(wres, hoff + 80u + 16u * uint32_t(g), sw);     // codes [64 + 16g, +16)
    };
    constexpr int NOP = 6;  // vector-memory operations per superblock and wave

    v4f_t acc[2] = {v4f_t{0.0f, 0.0f, 0.0f, 0.0f}, v4f_t{0.0f, 0.0f, 0.0f, 0.0f}};  // two MFMA chains
    float unit = 1.0f;
    u4_t wr[MFV_RING][3];

    // Prologue: superblocks s0 .. s0 + AHEAD - 1 (clamped); s0's operands land first.
#pragma unroll
    for (int r = 0; r < MFV_AHEAD; ++r) issue(wr[r], min(s0 + r, s1 - 1), r);
    mfv_wait<(MFV_AHEAD - 1) * NOP>(wr[0]);
    __syncthreads();

    for (int sb0 = s0; sb0 < s1; sb0 += MFV_RING) {
#pragma unroll
        for (int r = 0; r < MFV_RING; ++r) {
            const int sb = sb0 + r;
            if (sb >= s1) break;  // uniform
            // Refill the slot and stage of superblock sb - 1 (every wave is past it).
            issue(wr[(r + MFV_AHEAD) % MFV_RING], min(sb + MFV_AHEAD, s1 - 1), (r + MFV_AHEAD) % MFV_RING);
            const uint8_t *as = stage[r];
            h8_t af[4][2];  // this superblock's activation operands, read before the VALU work
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    const int c = 8 * jj + 4 * b + g;
                    af[jj][b] = *reinterpret_cast<const h8_t *>(as + col * 512 + 16 * (c ^ col));
                }
            const h8_t tf = *reinterpret_cast<const h8_t *>(as + MFV_ABYTES + col * 64 + 16 * g);
            const u4_t hdr = wr[r][0];
            const MmfRow rw = F::row(hdr);
            const u2_t kc[2] = {F::consts(hdr, rw, 2 * (g >> 1)),          // block pair of steps 0-1
                                F::consts(hdr, rw, 2 * (2 + (g >> 1)))};   // steps 2-3
            const u4_t mw = F::min_pair(hdr, rw, g);
            const float ratio = unit * __builtin_amdgcn_rcpf(rw.unit);  // earlier superblocks into this unit
            acc[0] *= ratio;
            acc[1] *= ratio;
            unit = rw.unit;
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const u4_t &pq = wr[r][1 + (jj >> 1)];
                const u2_t cq = (jj & 1) ? u2_t{pq.z, pq.w} : u2_t{pq.x, pq.y};
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    const uint32_t kk = kc[jj >> 1][b];
                    const h8_t wf = b == 0 ? F::template frag<0>(cq, kk) : F::template frag<1>(cq, kk);
                    acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[jj][b], wf, acc[b], 0, 0, 0);
                }
            }
            acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(tf, __builtin_bit_cast(h8_t, mw), acc[0], 0, 0, 0);
            // Superblock sb + 1's operands have landed (only the last AHEAD - 1 superblocks'
            // requests stay in flight); the barrier publishes its activation stage and
            // lets the next refill overwrite this one.
            mfv_wait<(MFV_AHEAD - 1) * NOP>(wr[(r + 1) % MFV_RING]);
            __syncthreads();
        }
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no DMA lands after the workgroup ends
    const v4f_t acc_sum = (acc[0] + acc[1]) * unit;

    // D[4g + i][col]: activation row 4g + i, weight row r0 + col.
    const int c = r0 + col;
    if (c >= n) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = 4 * g + i;
        if (row >= m) continue;
        if (partial) {
            partial[(int64_t(kz) * m + row) * n + c] = acc_sum[i];
        } else {
            const float v = acc_sum[i] * inverse[row];
            const int64_t idx = int64_t(row) * stride_dst + c;
            if (dst_bf16) static_cast<uint16_t *>(dst)[idx] = float_to_bf16_bits(v);
            else static_cast<float *>(dst)[idx] = v;
        }
    }
}

// Sum of the KS partial products in split order, times inverse[m], stored F32 or BF16.
__global__ __launch_bounds__(256) void mfv_reduce_kernel(const float *__restrict__ partial, int ks, int m, int n,
                                                         const float *__restrict__ inverse, void *__restrict__ dst,
                                                         int64_t stride_dst, int dst_bf16) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= int64_t(m) * n) return;
    const int row = int(i / n), c = int(i % n);
    float s = partial[i];
    for (int z = 1; z < ks; ++z) s += partial[int64_t(z) * m * n + i];
    const float v = s * inverse[row];
    const int64_t idx = int64_t(row) * stride_dst + c;
    if (dst_bf16) static_cast<uint16_t *>(dst)[idx] = float_to_bf16_bits(v);
    else static_cast<float *>(dst)[idx] = v;
}

template <int TYPE>
void launch_mfv_type(const void *weight, int64_t n, int64_t k, int64_t m, const MmfAct &act, float *partial,
                     void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream) {
    if (!act.t32) throw Error("fp16-MFMA small-M GEMM: min-term operands were not prepared");
    const int ks = mfv_splits(n, k);
    if (ks > 1 && !partial) throw Error("fp16-MFMA small-M GEMM: no room for partial sums");
    const int64_t row_bytes = (k / 256) * MmfW<TYPE>::SBB;
    const dim3 grid(static_cast<unsigned>((n + 63) / 64), static_cast<unsigned>(ks));
    mfv_kernel<TYPE><<<grid, dim3(256), 0, stream>>>(static_cast<const uint8_t *>(weight), row_bytes,
                                                      static_cast<int>(n), static_cast<int>(k), act.a16, act.t32,
                                                      act.inverse, static_cast<int>(m), dst, stride_dst,
                                                      dst_bf16 ? 1 : 0, ks > 1 ? partial : nullptr);
    if (ks > 1) {
        const int64_t total = m * n;
        mfv_reduce_kernel<<<dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, stream>>>(
            partial, ks, static_cast<int>(m), static_cast<int>(n), act.inverse, dst, stride_dst, dst_bf16 ? 1 : 0);
    }
}

}  // namespace kai
