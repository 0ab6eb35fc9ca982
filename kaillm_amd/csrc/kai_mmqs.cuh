// Small-M batched GEMM (kernel 2) for 9..16 activation rows: multi-sequence decode. It
// streams every weight byte once.
//
// Y[m, n] = inverse[m] * sum over K of the GGML MMQ block arithmetic (kai_mmq.cuh, MMA
// flavour), i.e. the same per-block integer dots, scales and min terms as mmq_kernel.
//
// Design for gfx950:
//   * the preparation writes the activation as this kernel's LDS image (kai_launch.h,
//     MmqPlanes), so a workgroup stages its K chunk with direct global-to-LDS copies
//     (global_load_lds_dwordx4): no registers, no conversion, one barrier;
//   * a workgroup (WAVES waves) owns 16 * WAVES weight rows (16 per wave) and one chunk of
//     K steps (256 values each); each wave streams its rows' wire bytes from HBM into a
//     ring of DEPTH K steps of registers with no barrier and no branch in the loop: a
//     chunk is a whole number of ring turns (steps past the chunk read zero activation,
//     their weight loads are clamped to the chunk's last step), so every load and wait is
//     straight-line code;
//   * per 32-value block one v_mfma_i32_16x16x32_i8 (two for formats with per-16 scales),
//     the fp32 epilogue of the block's scales, min terms on v_mfma_f32_16x16x4f32;
//   * K is split into chunks when the rows alone leave the chip short of workgroups or a
//     whole row's activation would not fit the LDS; each chunk writes fp32 partial sums
//     [chunk][m][n] that mmqs_reduce_kernel adds in chunk order (deterministic), times
//     inverse, into the strided output.
#pragma once

#include <type_traits>

#include "kai_mmq.cuh"

namespace kai {

constexpr int MMQS_DEPTH = 2, MMQS_WAVES = 4;
constexpr int MMQS_LDS_BUDGET = 40 * 1024;  // per workgroup: four workgroups per CU
static_assert(MMQS_LDS_BUDGET <= 64 * 1024, "the launch does not raise the dynamic LDS limit");

template <int TYPE>
constexpr int mmqs_step_bytes() {  // one K step of 16 activation rows in LDS
    return mmq_buf_bytes<TYPE, 1>();
}

// One K step of one wave: 8 blocks x (1 or 2) int8 MFMAs against the staged activation at
// `base`, the block epilogue, and the min terms. Batched (MMA) arithmetic of the format.
// Each half step (4 blocks) runs in phases: operand reads and codes, then the MFMAs, then
// the epilogues, so every MFMA's latency is covered by the other blocks' work.
template <int TYPE>
__device__ __forceinline__ void mmqs_step(typename MmqW<TYPE>::Raw &w, const uint8_t *base, v4f_t &acc, int col,
                                          int oct, int aoct, const uint32_t *grid) {
    using W = MmqLoad<TYPE>;
    constexpr int MODE = W::template mode<true>();
    constexpr int MT = 16, NT = W::NTERM, HALF = 4;
    constexpr int D8_OFF = MT * 8 * 32, TA_OFF = D8_OFF + MT * 8 * 4;
    const float *d8s = reinterpret_cast<const float *>(base + D8_OFF);
    const v4i_t zero = {0, 0, 0, 0};
    const bool first = W::first_half(oct);
    W::fix(w);
#pragma unroll
    for (int h = 0; h < 8; h += HALF) {
        long aq[HALF], bq[HALF];
        float4 dv[HALF];
#pragma unroll
        for (int u = 0; u < HALF; ++u) {
            const int b = h + u;
            aq[u] = *reinterpret_cast<const long *>(base + (b * MT + col) * 32 + 8 * (aoct ^ ((col >> 2) & 3)));
            dv[u] = *reinterpret_cast<const float4 *>(d8s + b * MT + 4 * oct);
            bq[u] = static_cast<long>(W::template codes<true>(w, b, oct, grid));
        }
        v4i_t r1[HALF], r2[HALF];
#pragma unroll
        for (int u = 0; u < HALF; ++u) {
            if constexpr (MODE == MMQ_BLOCK) {
                r1[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aq[u], bq[u], zero, 0, 0, 0);
            } else {
                r1[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aq[u], first ? bq[u] : 0l, zero, 0, 0, 0);
                r2[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aq[u], first ? 0l : bq[u], zero, 0, 0, 0);
            }
        }
#pragma unroll
        for (int u = 0; u < HALF; ++u) {
            const int b = h + u;
            const float d8[4] = {dv[u].x, dv[u].y, dv[u].z, dv[u].w};
            if constexpr (MODE == MMQ_BLOCK) {
                const float sa = W::template scale<true>(w, b);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i] = fmaf(d8[i] * sa, static_cast<float>(r1[u][i]), acc[i]);
            } else if constexpr (MODE == MMQ_ISPLIT) {
                const float sa = W::template scale<true>(w, b);
                const int sl = W::iscale(w, 2 * b), sh = W::iscale(w, 2 * b + 1);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int x = __mul24(sl, r1[u][i]) + __mul24(sh, r2[u][i]);
                    acc[i] = fmaf(d8[i] * sa, static_cast<float>(x), acc[i]);
                }
            } else {
                const float fl = W::fscale(w, 2 * b), fh = W::fscale(w, 2 * b + 1);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float x = fmaf(fh, static_cast<float>(r2[u][i]), fl * static_cast<float>(r1[u][i]));
                    acc[i] = fmaf(d8[i], x, acc[i]);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // one half step's results live at a time
    }
    if constexpr (NT > 0) {
        const float *ta = reinterpret_cast<const float *>(base + TA_OFF);
#pragma unroll
        for (int j = 0; j < NT / 4; ++j)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ta[(4 * j + oct) * MT + col], W::template term<true>(w, j, oct),
                                                      acc, 0, 0, 0);
    }
}

// Coalesced weight stream. One K step of a wave's 16 rows is 16 runs of SB bytes (one per
// row); each run is read as U 16-byte units (unit c = bytes [16c, 16c + 16) of the run,
// the last one running into the next run, which is ignored), lane l taking units l, l + 64,
// ... so that a load instruction reads whole 16-byte pieces of a few contiguous runs. The
// units go into the wave's LDS transpose buffer (row r at r * SBP) from which each lane reads
// its MFMA operand fields. (Loading the fields straight from HBM puts 16 rows in every load
// instruction, and with superblocks of 210 bytes (Q6_K) that halves the achieved bandwidth.)
template <int TYPE>
struct MmqsStream {
    static constexpr int SB = MmqW<TYPE>::SB, U = (SB + 15) / 16, SBP = 16 * U;
    static constexpr int UPL = (16 * U + WAVE - 1) / WAVE;  // units per lane
};

// grid: x = blocks of 16 * WAVES weight rows, y = K chunks of `chunk` steps; the ring runs
// over `span` steps (chunk rounded up to a multiple of DEPTH; the padding reads zero
// activation). partial: [gridDim.y][m][n] fp32 when gridDim.y > 1, else the output is stored
// directly.
template <int TYPE, int DEPTH, int WAVES>
__global__ __launch_bounds__(WAVES * WAVE) void mmqs_kernel(
    const uint8_t *weight, int64_t row_bytes, int n, int k, const uint8_t *__restrict__ image, int m,
    const float *__restrict__ inverse, int chunk, int span, float *__restrict__ partial, void *__restrict__ dst,
    int64_t stride_dst, int dst_bf16) {
    constexpr int THREADS = WAVES * WAVE;
    // `weight` is not __restrict__: its loads must stay ordered by the compiler fences of the
    // ring below (loads through a restrict pointer are treated as invariant and move freely)
    using W = MmqLoad<TYPE>;
    constexpr int BUF = mmqs_step_bytes<TYPE>(), IMG = mmqs_image_step(mmq_layout(TYPE));
    constexpr int UNITS = BUF / 16;  // 16-byte units of one staged step
    extern __shared__ __align__(16) uint8_t kai_mmqs_lds[];
    __shared__ uint32_t grid_lds[TYPE == IQ3_S ? 512 : 1];

    const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
    const int col = lane % 16, oct = lane / 16;
    const int nb = k / QK8_1, steps = (k + MMQ_STEP - 1) / MMQ_STEP;
    const int s0 = blockIdx.y * chunk, own = min(chunk, steps - s0);  // this chunk's real steps
    const int nrow0 = (blockIdx.x * WAVES + wave) * 16;
    if constexpr (TYPE == IQ3_S) {
        for (int i = tid; i < 512; i += THREADS) grid_lds[i] = mmq_iq3s_grid[i];
    }

    // ---- the lane's units (row r = u / U, unit c = u % U of the wave's rows), as 32-bit byte
    // offsets into the matrix (the launcher checks that it is below 4 GiB), so every load is
    // the step's scalar base plus a fixed lane offset; a lane with no unit in a group re-reads
    // the wave's first unit into a spare slot. A wave whose last row's run can end inside a
    // unit (superblocks that are not whole units, or a short last step) clamps each unit start
    // to the matrix's last 16 bytes and moves the unit's LDS position back by as many bytes
    // (its bytes past the end do not exist and are never read), so no load leaves the matrix.
    // That wave runs its own copy of the loop, so the loop body has no branch.
    using S = MmqsStream<TYPE>;
    uint32_t ug[S::UPL];
    int uoff[S::UPL];
#pragma unroll
    for (int i = 0; i < S::UPL; ++i) {
        const int u = lane + WAVE * i, r = u / S::U, c = u % S::U;
        const bool real = u < 16 * S::U;
        ug[i] = real ? static_cast<uint32_t>(min(nrow0 + r, n - 1)) * static_cast<uint32_t>(row_bytes) + 16 * c
                     : static_cast<uint32_t>(min(nrow0, n - 1)) * static_cast<uint32_t>(row_bytes);
        uoff[i] = real ? r * S::SBP + 16 * c : 16 * S::SBP;
    }
    const bool careful = (S::SB % 16 != 0 || k % MMQ_STEP != 0) && nrow0 + 15 >= n - 1;  // uniform
    const uint32_t tail = static_cast<uint32_t>(int64_t(n) * row_bytes - 16);
    const int last = s0 + own - 1;  // the ring's run-ahead re-reads this (cached) step
    struct Slot {
        uint4 v[S::UPL];
        uint32_t back;  // careful: 4 bits per unit, the bytes its load start was moved back
    };
    Slot wr[DEPTH];
    auto wload = [&](Slot &w, int j, auto careful_tag) {
        const uint32_t soff = static_cast<uint32_t>(min(s0 + j, last)) * S::SB;
        if constexpr (decltype(careful_tag)::value) {
            w.back = 0;
#pragma unroll
            for (int i = 0; i < S::UPL; ++i) {
                const uint32_t g = ug[i] + soff, a = min(g, tail);
                w.v[i] = load_unaligned<uint4>(weight + a);
                w.back |= (g - a) << (4 * i);
            }
        } else {
            const uint8_t *base = weight + soff;
#pragma unroll
            for (int i = 0; i < S::UPL; ++i) w.v[i] = load_unaligned<uint4>(base + ug[i]);
        }
    };
    auto prologue = [&](auto careful_tag) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            wload(wr[d], d, careful_tag);
            __asm__ volatile("" ::: "memory");  // the loop's order: its waits then count the slots in flight
        }
    };
    if (careful) prologue(std::true_type{});
    else prologue(std::false_type{});

    // ---- the chunk's activation image -> LDS, 16 bytes a lane, a wave's 64 lanes filling
    // 1 KiB in lane order; the ring padding past the chunk is zeroed. Q4_0 takes its terms
    // from the image's second term array.
    const uint8_t *img = image + int64_t(s0) * IMG;
    const int units = span * UNITS;
    for (int u0 = wave * WAVE; u0 < units; u0 += THREADS) {
        const int u = u0 + lane, j = u / UNITS, o = (u % UNITS) * 16;
        if (u < units) {
            if (j < own) {
                const int src = TYPE == Q4_0 && o >= MMQS_CODE_BYTES + MMQS_D8_BYTES ? o + MMQS_D8_BYTES : o;
                __builtin_amdgcn_global_load_lds(
                    static_cast<const void *>(img + j * IMG + src),
                    (__attribute__((address_space(3))) uint8_t *)kai_mmqs_lds + u0 * 16,
                    16, 0, 0);
            } else {
                *reinterpret_cast<uint4 *>(kai_mmqs_lds + u * 16) = make_uint4(0, 0, 0, 0);
            }
        }
    }
    __syncthreads();

    // ---- stream the weights: DEPTH steps in flight, straight-line loads and waits
    const int aoct = W::act_pos(oct) / 8;
    lds_u8 *tb = (lds_u8 *)kai_mmqs_lds + span * BUF + wave * (16 * S::SBP + 16);
    auto run = [&](auto careful_tag) {
        v4f_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int j0 = 0; j0 < span; j0 += DEPTH) {
#pragma unroll
            for (int d = 0; d < DEPTH; ++d) {
                const Slot &w = wr[d];
#pragma unroll
                for (int i = 0; i < S::UPL; ++i) {
                    if constexpr (decltype(careful_tag)::value)
                        store_unaligned(tb + uoff[i] - int((w.back >> (4 * i)) & 15u), w.v[i]);
                    else
                        store16(tb + uoff[i], w.v[i]);
                }
                typename W::Raw raw;
                W::load(raw, tb + col * S::SBP, oct, min(8, nb - 8 * min(s0 + j0 + d, last)));
                mmqs_step<TYPE>(raw, kai_mmqs_lds + (j0 + d) * BUF, acc, col, oct, aoct, grid_lds);
                wload(wr[d], j0 + d + DEPTH, careful_tag);
                // keep the refill here and each step's work in its own section: without these
                // fences the loads are sunk to their use and the next slot's decode is hoisted
                // into this one, and the waits drain the ring every step
                __asm__ volatile("" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        return acc;
    };
    const v4f_t acc = careful ? run(std::true_type{}) : run(std::false_type{});

    // ---- store: rows 4*oct + i of weight row nrow0 + col
    const int c = nrow0 + col;
    if (c >= n) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = 4 * oct + i;
        if (row >= m) continue;
        if (gridDim.y > 1) {
            partial[(int64_t(blockIdx.y) * m + row) * n + c] = acc[i];
        } else {
            const float v = acc[i] * inverse[row];
            const int64_t idx = int64_t(row) * stride_dst + c;
            if (dst_bf16) static_cast<uint16_t *>(dst)[idx] = float_to_bf16_bits(v);
            else static_cast<float *>(dst)[idx] = v;
        }
    }
}

// out[row][c] = inverse[row] * sum over chunks (in order) of partial[chunk][row][c].
static __global__ __launch_bounds__(256) void mmqs_reduce_kernel(const float *__restrict__ partial, int chunks, int m,
                                                          int n, const float *__restrict__ inverse,
                                                          void *__restrict__ dst, int64_t stride_dst, int dst_bf16) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= int64_t(m) * n) return;
    const int row = static_cast<int>(i / n), c = static_cast<int>(i % n);
    float s = partial[i];
    for (int g = 1; g < chunks; ++g) s += partial[int64_t(g) * m * n + i];
    const float v = s * inverse[row];
    const int64_t idx = int64_t(row) * stride_dst + c;
    if (dst_bf16) static_cast<uint16_t *>(dst)[idx] = float_to_bf16_bits(v);
    else static_cast<float *>(dst)[idx] = v;
}

// Launch shape: K chunk (steps staged per workgroup) and chunk count. The staged chunk and
// the waves' transpose buffers fit MMQS_LDS_BUDGET, and K is cut into more chunks while the
// workgroups would not fill the chip. The plan depends only on the type and shape, so the
// scratch query and the launch agree on every device.
struct MmqsPlan {
    int chunk, chunks, span;
    size_t lds;
};
template <int TYPE>
constexpr size_t mmqs_stream_lds() {  // per wave: 16 rows and a spare unit
    return size_t(MMQS_WAVES) * (16 * MmqsStream<TYPE>::SBP + 16);
}
template <int TYPE>
inline MmqsPlan mmqs_plan(int64_t n, int64_t k) {
    constexpr int64_t WANT = 1024;  // workgroups that fill 256 CUs four deep
    constexpr int BUF = mmqs_step_bytes<TYPE>();
    constexpr int MAX_SPAN = int((MMQS_LDS_BUDGET - mmqs_stream_lds<TYPE>()) / BUF) / MMQS_DEPTH * MMQS_DEPTH;
    static_assert(MAX_SPAN >= MMQS_DEPTH, "the LDS budget must hold one ring turn of activation");
    const int steps = static_cast<int>(mmqs_steps(k));
    const int64_t blocks = (n + 16 * MMQS_WAVES - 1) / (16 * MMQS_WAVES);
    int chunks = (steps + MAX_SPAN - 1) / MAX_SPAN;
    while (blocks * chunks < WANT && (steps + chunks) / (chunks + 1) >= 2) ++chunks;
    MmqsPlan p;
    p.chunk = (steps + chunks - 1) / chunks;
    p.chunks = (steps + p.chunk - 1) / p.chunk;
    p.span = (p.chunk + MMQS_DEPTH - 1) / MMQS_DEPTH * MMQS_DEPTH;
    p.lds = size_t(p.span) * BUF + mmqs_stream_lds<TYPE>();
    return p;
}

// Partial-sum bytes of an m-row product with this matrix on the small-M GEMM (0 when its
// plan has one chunk).
template <int TYPE>
inline size_t mmqs_partial_bytes(int64_t m, int64_t n, int64_t k) {
    if (m < 1 || m > MMQS_MAX_ROWS) return 0;
    const MmqsPlan p = mmqs_plan<TYPE>(n, k);
    return p.chunks > 1 ? size_t(p.chunks) * size_t(m) * size_t(n) * sizeof(float) : 0;
}

// image: the layout's small-M image (kai_launch.h) of the m activation rows.
template <int TYPE>
void launch_mmqs(const void *weight, int64_t n, int64_t k, int64_t m, const uint8_t *image, const float *inverse,
                 float *partial, size_t partial_bytes, void *dst, bool dst_bf16, int64_t stride_dst,
                 hipStream_t stream) {
    if (m < 1 || m > MMQS_MAX_ROWS) throw Error("The small-M GEMM takes 1..16 activation rows");
    const MmqsPlan p = mmqs_plan<TYPE>(n, k);
    const size_t need = p.chunks > 1 ? size_t(p.chunks) * size_t(m) * size_t(n) * sizeof(float) : 0;
    if (need > partial_bytes || (need && !partial)) throw Error("Scratch too small for the small-M GEMM's partial sums");
    const int64_t row_bytes = (k / block_elems(TYPE)) * block_bytes(TYPE);
    if (n * row_bytes >= (int64_t(1) << 32)) throw Error("The small-M GEMM takes matrices below 4 GiB");
    const size_t lds = p.lds;
    auto kernel = mmqs_kernel<TYPE, MMQS_DEPTH, MMQS_WAVES>;  // within the default 64 KiB of dynamic LDS
    const dim3 grid(static_cast<unsigned>((n + 16 * MMQS_WAVES - 1) / (16 * MMQS_WAVES)), static_cast<unsigned>(p.chunks));
    kernel<<<grid, MMQS_WAVES * WAVE, lds, stream>>>(static_cast<const uint8_t *>(weight), row_bytes,
                                                     static_cast<int>(n), static_cast<int>(k), image,
                                                     static_cast<int>(m), inverse, p.chunk, p.span, partial, dst,
                                                     stride_dst, dst_bf16 ? 1 : 0);
    if (p.chunks > 1) {
        const int64_t total = m * n;
        mmqs_reduce_kernel<<<static_cast<unsigned>((total + 255) / 256), 256, 0, stream>>>(
            partial, p.chunks, static_cast<int>(m), static_cast<int>(n), inverse, dst, stride_dst, dst_bf16 ? 1 : 0);
    }
}

}  // namespace kai
