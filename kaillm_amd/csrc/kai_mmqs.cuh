// Small-M batched GEMM (kernel 2) for 9..16 activation rows: multi-sequence decode. It
// streams every weight byte once.
//
// Y[m, n] = inverse[m] * sum over K of the GGML MMQ block arithmetic (kai_mmq.cuh, MMA
// flavour), i.e. the same per-block integer dots, scales and min terms as mmq_kernel.
//
// Design for gfx950. At 16 rows the whole product is a few tens of K steps per SIMD, so a
// wave's start-up (its first weight loads from HBM) costs as much as its work unless each
// wave starts once; the kernel is therefore persistent and stream-K balanced:
//   * one workgroup of mmqs_waves waves per CU (at most MMQS_MAX_GRID); K is cut into as few chunks as
//     the LDS holds (usually one), and each chunk's workgroups stage its activation once,
//     from the LDS image the preparation wrote (kai_launch.h, MmqPlanes), with direct
//     global-to-LDS copies (global_load_lds_dwordx4): no registers, one barrier;
//   * a chunk's work is the row-major sequence of (16-row set, K step) pairs; its waves take
//     equal contiguous runs of it (at least MMQS_MIN_RUN steps), so every SIMD gets the same
//     number of steps whatever the shape; runs are dealt to the chunk's workgroups in turn, so
//     a chunk with fewer runs than waves still reaches every CU. A run crosses row sets: the
//     wave's ring of DEPTH steps of weight loads runs on
//     across them, and at the end of each piece of a row set the wave stores its sums;
//   * weights stream as contiguous 16-byte units per row into the wave's LDS transpose
//     buffer (MmqsStream), from which each lane reads its MFMA operand fields;
//   * per 32-value block one v_mfma_i32_16x16x32_i8 (two for formats with per-16 scales),
//     the fp32 epilogue of the block's scales, min terms on v_mfma_f32_16x16x4f32;
//   * each piece of a row set goes to fp32 partial sums [chunk][row set][piece][16][16]
//     that mmqs_reduce_kernel adds in chunk and piece order (deterministic), times inverse,
//     into the output.
#pragma once

#include <type_traits>

#include "kai_mmq.cuh"

namespace kai {

constexpr int MMQS_DEPTH = 2;
// Waves per workgroup: 16, and 12 for IQ3_S. Measured on MI355X at 16 rows (whole calls), 12
// against 16 waves: IQ3_S 5120x17408 36.70 -> 34.11 us, Q2_K 31.48 -> 31.28, Q6_K 5120x17408
// 32.22 -> 32.11, but Q6_K 5120x6144 19.53 -> 20.62.
template <int TYPE> constexpr int mmqs_waves() { return TYPE == IQ3_S ? 12 : 16; }
// Workgroups: one per CU of the device, at most MMQS_MAX_GRID (an MI355X's 256 CUs). The
// partial-sum scratch is sized for MMQS_MAX_GRID workgroups, which bounds it for any device:
// fewer workgroups take longer runs and so cut every row set into fewer pieces.
constexpr int MMQS_MAX_GRID = 256;
constexpr int MMQS_LDS_BUDGET = 160 * 1024;  // the CU's LDS
constexpr int MMQS_MIN_RUN = 4;             // K steps a wave takes at least (when it has work)

template <int TYPE>
constexpr int mmqs_step_bytes() {  // one K step of 16 activation rows in LDS
    return mmq_buf_bytes<TYPE, 1>();
}

// One K step of one wave: 8 blocks x (1 or 2) int8 MFMAs against the staged activation at
// `base`, the block epilogue, and the min terms. Batched (MMA) arithmetic of the format.
// Each group of HALF blocks runs in phases: operand reads and codes, then the MFMAs, then
// the epilogues, so every MFMA's latency is covered by the other blocks' work.
// The weight fields come from the wave's transpose buffer row `wp` (the lane's row, octet
// oct; nvalid blocks of the step inside the row): all at once, or per block for formats
// whose blocks are independent (LAZY), which keeps them out of the registers until used.
// EXACT: the exact weight products of mmq_kernel's EXACT form (the legacy MMQ's arithmetic).
template <int TYPE, bool EXACT>
__device__ __forceinline__ void mmqs_step(const lds_u8 *wp, int nvalid, const uint8_t *base, v4f_t &acc, int col,
                                          int oct, int aoct, const uint32_t *grid) {
    using W = MmqLoad<TYPE>;
    constexpr bool BATCHED = !EXACT;
    constexpr int MODE = W::template mode<BATCHED>();
    constexpr bool LAZY = LazyLoad<MmqW<TYPE>>::value;
    // blocks per phase: their MFMA results, operands and scales are live at once
    constexpr int MT = 16, NT = W::NTERM, HALF = MODE == MMQ_BLOCK ? 4 : 2;
    constexpr int D8_OFF = MT * 8 * 32, TA_OFF = D8_OFF + MT * 8 * 4;
    const float *d8s = reinterpret_cast<const float *>(base + D8_OFF);
    const v4i_t zero = {0, 0, 0, 0};
    const bool first = W::first_half(oct);
    typename W::Raw w;
    if constexpr (!LAZY) {
        W::load(w, wp, oct, nvalid);
        W::fix(w);
    }
    // ISPLIT: one float scale for the whole step (the superblock's d), applied once at the end
    // to the step's sum of d8 * (integer block dot); the blocks then need no scale product.
    v4f_t sacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int h = 0; h < 8; h += HALF) {
        long aq[HALF], bq[HALF];
        float4 dv[HALF];
#pragma unroll
        for (int u = 0; u < HALF; ++u) {
            const int b = h + u;
            if constexpr (LAZY) W::load_block(w, wp, oct, nvalid, b);
            aq[u] = *reinterpret_cast<const long *>(base + (b * MT + col) * 32 + 8 * (aoct ^ ((col >> 2) & 3)));
            dv[u] = *reinterpret_cast<const float4 *>(d8s + b * MT + 4 * oct);
            bq[u] = static_cast<long>(W::template codes<BATCHED>(w, b, oct, grid));
        }
        v4i_t r1[HALF], r2[HALF];
#pragma unroll
        for (int u = 0; u < HALF; ++u) {
            if constexpr (MODE == MMQ_BLOCK) {
                r1[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aq[u], bq[u], zero, 0, 0, 0);
            } else if constexpr (MODE == MMQ_ISPLIT) {  // first half and whole block
                r1[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aq[u], first ? bq[u] : 0l, zero, 0, 0, 0);
                r2[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aq[u], bq[u], zero, 0, 0, 0);
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
                const float sa = W::template scale<BATCHED>(w, b);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i] = fmaf(d8[i] * sa, static_cast<float>(r1[u][i]), acc[i]);
            } else if constexpr (MODE == MMQ_ISPLIT) {
                // sl * C_lo + sh * C_hi = (sl - sh) * C_lo + sh * C (exact 24-bit integers)
                const int sl = W::iscale(w, 2 * b), sh = W::iscale(w, 2 * b + 1);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int x = __mul24(sl - sh, r1[u][i]) + __mul24(sh, r2[u][i]);
                    sacc[i] = fmaf(d8[i], static_cast<float>(x), sacc[i]);
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
        __builtin_amdgcn_sched_barrier(0);  // one phase's results live at a time
    }
    if constexpr (MODE == MMQ_ISPLIT) {
        const float sa = W::template scale<BATCHED>(w, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = fmaf(sa, sacc[i], acc[i]);
    }
    if constexpr (NT > 0) {
        const float *ta = reinterpret_cast<const float *>(base + TA_OFF);
#pragma unroll
        for (int j = 0; j < NT / 4; ++j)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ta[(4 * j + oct) * MT + col], W::template term<BATCHED>(w, j, oct),
                                                      acc, 0, 0, 0);
    }
}

// Weights: the coalesced stream of kai_mmq_formats.h (MmqsStream), 16 rows per wave.

// The work split of a launch (host and device agree on it).
struct MmqsSplit {
    int chunks, chunk;  // K chunks of `chunk` steps (the last may be shorter)
    int wgs;            // workgroups per chunk
    int waves;          // waves per chunk that take work
    int qmax;           // pieces a row set has at most in one chunk
};
// Steps of chunk c; its positions per row set (rounded up to even: an odd chunk gets a zero
// step); and the run of its waves (even). With both even every piece of a row set starts at
// an even position and has an even length, so the loop runs whole ring turns (DEPTH 2).
__host__ __device__ inline int mmqs_chunk_steps(const MmqsSplit &p, int steps, int c) {
    return min(p.chunk, steps - c * p.chunk);
}
__host__ __device__ inline int mmqs_positions(int sc) { return sc + (sc & 1); }
__host__ __device__ inline int mmqs_run(const MmqsSplit &p, int rowsets, int sc) {
    const int run = (rowsets * mmqs_positions(sc) + p.waves - 1) / p.waves;
    return run + (run & 1);
}

// grid: chunks * wgs workgroups of WAVES waves; workgroup b works on chunk b / wgs.
template <int TYPE, int DEPTH, int WAVES, bool EXACT = false>
__global__ __launch_bounds__(WAVES * WAVE) void mmqs_kernel(
    const uint8_t *weight, int64_t row_bytes, int n, int k, const uint8_t *__restrict__ image, int m,
    const float *__restrict__ inverse, MmqsSplit split, float *__restrict__ partial, void *__restrict__ dst,
    int64_t stride_dst, int dst_bf16) {
    constexpr int THREADS = WAVES * WAVE;
    // `weight` is not __restrict__: its loads must stay ordered by the compiler fences of the
    // ring below (loads through a restrict pointer are treated as invariant and move freely)
    using W = MmqLoad<TYPE>;
    using S = MmqsStream<TYPE>;
    constexpr int BUF = mmqs_step_bytes<TYPE>(), IMG = mmqs_image_step(mmq_layout(TYPE));
    constexpr int UNITS = BUF / 16;  // 16-byte units of one staged step
    extern __shared__ __align__(16) uint8_t kai_mmqs_lds[];
    __shared__ uint32_t grid_lds[TYPE == IQ3_S ? 512 : 1];

    const int tid = threadIdx.x, lane = tid % WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);  // uniform: the run's control is scalar
    const int col = lane % 16, oct = lane / 16;
    const int nb = k / QK8_1, steps = (k + MMQ_STEP - 1) / MMQ_STEP;
    const int chunk_id = blockIdx.x / split.wgs;
    const int s0 = chunk_id * split.chunk, sc = mmqs_chunk_steps(split, steps, chunk_id);
    const int rowsets = (n + 15) / 16;
    // this wave's run [t0, t1) of the chunk's (row set, step) sequence. Runs are dealt to the
    // chunk's workgroups in turn (run w to wave w / wgs of workgroup w % wgs), so that when a
    // chunk has fewer runs than waves every workgroup, and so every CU, still gets a share.
    const int w = wave * split.wgs + blockIdx.x % split.wgs;
    const int sce = mmqs_positions(sc), run = mmqs_run(split, rowsets, sc), total = rowsets * sce;
    const int t0 = w < split.waves ? min(w * run, total) : total, t1 = w < split.waves ? min(t0 + run, total) : total;
    if constexpr (TYPE == IQ3_S) {
        for (int i = tid; i < 512; i += THREADS) grid_lds[i] = mmq_iq3s_grid[i];
    }

    // ---- the lane's units (row r = u / U, unit c = u % U of a row set), as 32-bit byte
    // offsets into the matrix (the launcher checks that it is below 4 GiB), so every load is
    // a scalar base (row set, step) plus a fixed lane offset; a lane with no unit in a group
    // re-reads the row set's first unit into a spare slot. A wave whose run reaches the last
    // row set, when its rows or runs can end inside a unit (rows not a multiple of 16,
    // superblocks that are not whole units, a short last step), clamps each unit start to the
    // matrix's last 16 bytes and moves the unit's LDS position back by as many bytes (0 for a
    // unit wholly past the end, whose rows are never stored), so no load leaves the matrix.
    // That wave runs its own copy of the loop, so the loop body has no branch for it.
    uint32_t ug[S::UPL];
    int uoff[S::UPL];
#pragma unroll
    for (int i = 0; i < S::UPL; ++i) {
        const int u = lane + WAVE * i, r = u / S::U, c = u % S::U;
        const bool real = u < 16 * S::U;
        ug[i] = real ? static_cast<uint32_t>(r) * static_cast<uint32_t>(row_bytes) + 16 * c : 0u;
        uoff[i] = real ? r * S::SBP + 16 * c : 16 * S::SBP;
    }
    const bool ragged = n % 16 != 0 || S::SB % 16 != 0 || k % MMQ_STEP != 0;
    const bool careful = ragged && t1 > t0 && (t1 - 1) / sce == rowsets - 1;  // uniform
    const uint32_t tail = static_cast<uint32_t>(int64_t(n) * row_bytes - 16);
    const uint32_t set_bytes = 16u * static_cast<uint32_t>(row_bytes);
    struct Slot {
        uint4 v[S::UPL];
        uint32_t back;  // careful: 4 bits per unit, the bytes its load start was moved back
    };
    Slot wr[DEPTH];
    // The next position to load (row set lr, position lj); the ring's run-ahead past the
    // run's end repeats its last position, and a chunk's zero step re-reads its last step.
    int lt = t0, lr = t1 > t0 ? t0 / sce : 0, lj = t1 > t0 ? t0 % sce : 0;
    auto wload = [&](Slot &sl, auto careful_tag) {
        const uint32_t lbase = static_cast<uint32_t>(lr) * set_bytes + static_cast<uint32_t>(s0 + min(lj, sc - 1)) * S::SB;
        if constexpr (decltype(careful_tag)::value) {
            sl.back = 0;
#pragma unroll
            for (int i = 0; i < S::UPL; ++i) {
                const uint32_t g = ug[i] + lbase, a = min(g, tail), back = g - a;
                sl.v[i] = load_unaligned<uint4>(weight + a);
                sl.back |= (back < 16u ? back : 0u) << (4 * i);
            }
        } else {
            const uint8_t *b = weight + lbase;
#pragma unroll
            for (int i = 0; i < S::UPL; ++i) sl.v[i] = load_unaligned<uint4>(b + ug[i]);
        }
        // advance (scalar selects: a branch here would split the loop body)
        const int adv = lt < t1 - 1 ? 1 : 0;
        lt += adv;
        lj += adv;
        const int wrap = lj == sce ? 1 : 0;
        lj = wrap ? 0 : lj;
        lr += wrap;
    };
    auto prologue = [&](auto careful_tag) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            wload(wr[d], careful_tag);
            __asm__ volatile("" ::: "memory");  // the loop's order: its waits then count the slots in flight
        }
    };
    // the clamped form for every wave (it clamps nothing where the fast form is safe), so the
    // ring enters either copy of the loop from one code path
    if (t1 > t0) prologue(std::true_type{});

    // ---- the chunk's activation image -> LDS, 16 bytes a lane, a wave's 64 lanes filling
    // 1 KiB in lane order. Q4_0 takes its terms from the image's second term array.
    const uint8_t *img = image + int64_t(s0) * IMG;
    const int units = sc * UNITS;
    for (int u0 = wave * WAVE; u0 < units; u0 += THREADS) {
        const int u = u0 + lane, j = u / UNITS, o = (u % UNITS) * 16;
        if (u < units) {
            const int src = TYPE == Q4_0 && o >= MMQS_CODE_BYTES + MMQS_D8_BYTES ? o + MMQS_D8_BYTES : o;
            __builtin_amdgcn_global_load_lds(static_cast<const void *>(img + j * IMG + src),
                                             (__attribute__((address_space(3))) uint8_t *)kai_mmqs_lds + u0 * 16,
                                             16, 0, 0);
        }
    }
    if (sce > sc) {  // the zero step of an odd chunk
        for (int u = tid; u < UNITS; u += THREADS) store16((lds_u8 *)kai_mmqs_lds + (units + u) * 16, make_uint4(0, 0, 0, 0));
    }
    __syncthreads();
    if (t1 <= t0) return;

    // ---- the run: DEPTH steps in flight, straight-line loads and waits; a piece of a row
    // set ends at its last step or the run's, and is stored there
    const int aoct = W::act_pos(oct) / 8;
    const int buf_off = mmqs_positions(split.chunk) * BUF;  // the transpose buffers follow the largest chunk
    lds_u8 *tb = (lds_u8 *)kai_mmqs_lds + buf_off + wave * (16 * S::SBP + 16);
    // piece q of row set r is this wave's index minus that of the wave holding the set's
    // first step; it goes to partial [chunk][row set][q] as [16 activation rows][16 columns]
    // fp32 (rows past m are zero), so that the reduction reads and writes whole rows
    auto store = [&](const v4f_t &acc, int r) {
        const int q = w - (r * sce) / run;
        float *p = partial + (((int64_t(chunk_id) * rowsets + r) * split.qmax + q) * 16 + 4 * oct) * 16 + col;
#pragma unroll
        for (int i = 0; i < 4; ++i) p[16 * i] = acc[i];
    };
    auto loop = [&](auto careful_tag) {
#pragma unroll 1
        for (int pa = t0; pa < t1;) {  // one piece of a row set: positions [pa, pb), both even
            const int r = pa / sce, pb = min(t1, (r + 1) * sce);
            v4f_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
            for (int j = pa - r * sce; j < pb - r * sce; j += DEPTH) {
#pragma unroll
                for (int d = 0; d < DEPTH; ++d) {
                    const Slot &sl = wr[d];
#pragma unroll
                    for (int i = 0; i < S::UPL; ++i) {
                        if constexpr (decltype(careful_tag)::value)
                            store_unaligned(tb + uoff[i] - int((sl.back >> (4 * i)) & 15u), sl.v[i]);
                        else
                            store16(tb + uoff[i], sl.v[i]);
                    }
                    mmqs_step<TYPE, EXACT>(tb + col * S::SBP, min(8, nb - 8 * (s0 + min(j + d, sc - 1))),
                                    kai_mmqs_lds + (j + d) * BUF, acc, col, oct, aoct, grid_lds);
                    wload(wr[d], careful_tag);
                    // keep the refill here and each step's work in its own section: without
                    // these fences the loads are sunk to their use and the next slot's decode
                    // is hoisted into this one, and the waits drain the ring every step
                    __asm__ volatile("" ::: "memory");
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            store(acc, r);
            pa = pb;
        }
    };
    // Q8_0 and Q4_0 (whose raw fields are many small pieces) run every wave on the clamped
    // copy: two copies of their loop do not fit the 128 registers without spilling
    if constexpr (LazyLoad<MmqW<TYPE>>::value) {
        loop(std::true_type{});
    } else {
        if (careful) loop(std::true_type{});
        else loop(std::false_type{});
    }
}

// out[row][c] = inverse[row] * sum over chunks, then pieces (in order), of the partial sums
// of c's row set. One workgroup per row set: thread t adds output (row t / 16, column
// 16 r + t % 16), so each piece's 16 x 16 sums are one contiguous KiB read by one load and the
// piece counts are uniform. (Combining the pieces in the GEMM itself needs an agent-scope
// release and acquire, which on MI355X write back and invalidate the XCD's L2: per wave and
// piece they made the GEMM six times slower; once per workgroup after its run, with per-row-set
// piece counters in the scratch, the call took 24 to 39 % longer than with this launch at 9
// and 16 rows on 5120 x 17408 and 5120 x 6144.)
static __global__ __launch_bounds__(256) void mmqs_reduce_kernel(const float *__restrict__ partial, MmqsSplit split,
                                                                  int steps, int m, int n,
                                                                  const float *__restrict__ inverse,
                                                                  void *__restrict__ dst, int64_t stride_dst,
                                                                  int dst_bf16) {
    const int r = blockIdx.x, row = threadIdx.x / 16, c = 16 * r + threadIdx.x % 16;
    const int rowsets = (n + 15) / 16;
    auto pieces = [&](int ch, const float *&p) {
        const int sc = mmqs_chunk_steps(split, steps, ch), sce = mmqs_positions(sc), run = mmqs_run(split, rowsets, sc);
        p = partial + (int64_t(ch) * rowsets + r) * split.qmax * 256 + threadIdx.x;
        return (r * sce + sce - 1) / run - (r * sce) / run + 1;
    };
    float s = 0.0f;
    constexpr int MC = 4, MQ = 4;
    if (split.chunks <= MC && split.qmax <= MQ) {  // every load in flight at once, then the same sums
        float t[MC][MQ];
        int np[MC];
#pragma unroll
        for (int ch = 0; ch < MC; ++ch) {
            const float *p = partial;
            np[ch] = ch < split.chunks ? pieces(ch, p) : 0;
#pragma unroll
            for (int q = 0; q < MQ; ++q) t[ch][q] = q < np[ch] ? p[q * 256] : 0.0f;
        }
#pragma unroll
        for (int ch = 0; ch < MC; ++ch)
#pragma unroll
            for (int q = 0; q < MQ; ++q)
                if (q < np[ch]) s += t[ch][q];
    } else {
        for (int ch = 0; ch < split.chunks; ++ch) {
            const float *p;
            const int np = pieces(ch, p);
            for (int q = 0; q < np; ++q) s += p[q * 256];
        }
    }
    if (row >= m || c >= n) return;  // rows past m hold zeros; columns past n are not stored
    const float v = s * inverse[row];
    const int64_t idx = int64_t(row) * stride_dst + c;
    if (dst_bf16) static_cast<uint16_t *>(dst)[idx] = float_to_bf16_bits(v);
    else static_cast<float *>(dst)[idx] = v;
}

// The split: K in as few chunks as the LDS holds (the staged chunk plus the waves' transpose
// buffers), `grid` workgroups shared by the chunks, and runs of at least MMQS_MIN_RUN steps.
// It depends only on the type, the shape and the grid.
template <int TYPE>
constexpr size_t mmqs_stream_lds() {  // per workgroup: 16 rows and a spare unit per wave
    return size_t(mmqs_waves<TYPE>()) * (16 * MmqsStream<TYPE>::SBP + 16);
}
template <int TYPE>
inline MmqsSplit mmqs_split(int64_t n, int64_t k, int grid) {
    constexpr int BUF = mmqs_step_bytes<TYPE>();
    constexpr int MAX_CHUNK =  // even, so that an odd chunk's zero step fits too
        int((MMQS_LDS_BUDGET - mmqs_stream_lds<TYPE>() - (TYPE == IQ3_S ? 2048 : 0)) / BUF) / 2 * 2;
    static_assert(MAX_CHUNK >= 2, "the LDS must hold two K steps of activation");
    const int steps = static_cast<int>(mmqs_steps(k)), rowsets = static_cast<int>((n + 15) / 16);
    MmqsSplit p;
    p.chunks = (steps + MAX_CHUNK - 1) / MAX_CHUNK;
    p.chunk = (steps + p.chunks - 1) / p.chunks;
    p.chunks = (steps + p.chunk - 1) / p.chunk;
    p.wgs = std::max(1, grid / p.chunks);
    const int64_t work = int64_t(rowsets) * mmqs_positions(p.chunk);  // the largest chunk's
    p.waves = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(int64_t(p.wgs) * mmqs_waves<TYPE>(),
                                                                         work / MMQS_MIN_RUN)));
    p.qmax = 1;
    for (int c = 0; c < p.chunks; ++c) {
        const int sc = mmqs_chunk_steps(p, steps, c), run = mmqs_run(p, rowsets, sc);
        p.qmax = std::max(p.qmax, (mmqs_positions(sc) + run - 1) / run + 1);
    }
    return p;
}
template <int TYPE>
inline size_t mmqs_lds_bytes(const MmqsSplit &p) {
    return size_t(mmqs_positions(p.chunk)) * mmqs_step_bytes<TYPE>() + mmqs_stream_lds<TYPE>();
}

// Partial-sum bytes of a split (chunk, row set, piece, 16 x 16 fp32).
inline size_t mmqs_split_bytes(const MmqsSplit &p, int64_t n) {
    return size_t(p.chunks) * size_t((n + 15) / 16) * size_t(p.qmax) * 256 * sizeof(float);
}
// Partial-sum bytes of an m-row product with this matrix on the small-M GEMM, on any device
// (the split of MMQS_MAX_GRID workgroups bounds every smaller grid's).
template <int TYPE>
inline size_t mmqs_partial_bytes(int64_t m, int64_t n, int64_t k) {
    if (m < 1 || m > MMQS_MAX_ROWS) return 0;
    return mmqs_split_bytes(mmqs_split<TYPE>(n, k, MMQS_MAX_GRID), n);
}

// image: the layout's small-M image (kai_launch.h) of the m activation rows. EXACT: the
// exact weight products (mmqs_step).
template <int TYPE, bool EXACT = false>
void launch_mmqs(const void *weight, int64_t n, int64_t k, int64_t m, const uint8_t *image, const float *inverse,
                 float *partial, size_t partial_bytes, void *dst, bool dst_bf16, int64_t stride_dst,
                 hipStream_t stream) {
    if (m < 1 || m > MMQS_MAX_ROWS) throw Error("The small-M GEMM takes 1..16 activation rows");
    if (n < 1 || k < MMQ_STEP / 8) throw Error("Invalid small-M GEMM shape");
    const MmqsSplit p = mmqs_split<TYPE>(n, k, std::min(device_cu_count(), MMQS_MAX_GRID));
    const size_t need = mmqs_split_bytes(p, n);
    if (need > partial_bytes || !partial) throw Error("Scratch too small for the small-M GEMM's partial sums");
    const int64_t row_bytes = (k / block_elems(TYPE)) * block_bytes(TYPE);
    if (n * row_bytes >= (int64_t(1) << 32)) throw Error("The small-M GEMM takes matrices below 4 GiB");
    const size_t lds = mmqs_lds_bytes<TYPE>(p);
    auto kernel = mmqs_kernel<TYPE, MMQS_DEPTH, mmqs_waves<TYPE>(), EXACT>;
    static DeviceFlags lds_raised;
    raise_dynamic_lds(reinterpret_cast<const void *>(kernel), MMQS_LDS_BUDGET - (TYPE == IQ3_S ? 2048 : 0), lds_raised,
                      "Cannot raise the small-M GEMM's dynamic LDS limit");
    kernel<<<dim3(static_cast<unsigned>(p.chunks * p.wgs)), mmqs_waves<TYPE>() * WAVE, lds, stream>>>(
        static_cast<const uint8_t *>(weight), row_bytes, static_cast<int>(n), static_cast<int>(k), image,
        static_cast<int>(m), inverse, p, partial, dst, stride_dst, dst_bf16 ? 1 : 0);
    mmqs_reduce_kernel<<<static_cast<unsigned>((n + 15) / 16), 256, 0, stream>>>(
        partial, p, static_cast<int>(mmqs_steps(k)), static_cast<int>(m), static_cast<int>(n), inverse, dst,
        stride_dst, dst_bf16 ? 1 : 0);
}

}  // namespace kai
