// Decode / spec-verify GEMV (kernel 1): y[j, r] = inverse[j] * sum_b dot(W[r, b], q8[j, b])
// for m <= 16 activation rows, every wire format, weights streamed once from HBM.
//
// Reference: kai_dual::mmvq_dual (vllm_gguf_plugin/native/kernels/kai_dual_mmvq.cuh:258-327)
// and its launcher (:329-397). Design for gfx950 instead of warp32 CTAs:
//   * a wave64 works on 64/G rows at once, one group of G lanes per row (G = 16..64,
//     wider for long rows, pick_group), and on RS such row sets one after the other
//     (gemv_row_sets);
//     the lanes of a group walk the row's ~32-byte units (kai_units.h) in order, so
//     each load instruction reads contiguous runs of G units of wire bytes;
//   * a ring of DEPTH units per lane of wire bytes is kept in flight (1 for superblock
//     formats with one row set, else 2): unit t + DEPTH is requested before unit t is
//     multiplied (a shallow ring keeps more waves resident);
//   * the activation (all m rows of Q8_1 blocks, byte for byte) is staged in LDS once
//     per workgroup together with the exact code sums of every 16-value half, so the
//     loop issues no vector-memory load other than the weight stream (vmcnt retires in
//     issue order, so any other global load in the loop would wait for the whole ring);
//   * integer dots with v_dot4_i32_i8, fp32 scale/accumulate per block;
//   * per-row totals by a DPP/swizzle reduction inside each lane group, no barrier;
//   * merged-projection epilogue: x inverse[j], F32 or BF16, strided store.
#pragma once

#include <type_traits>

#include "kai_iq3s_grid.h"
#include "kai_launch.h"
#include "kai_units.h"

namespace kai {

// Each translation unit that instantiates the IQ3_S kernel owns a copy of the grid.
static __device__ const uint32_t iq3s_grid_global[512] = {KAI_IQ3S_GRID_VALUES};

constexpr int MMVQ_LDS_BUDGET = 160 * 1024;

template <int TYPE>
__device__ __forceinline__ Unit<TYPE> make_unit(int sub, const uint32_t *grid) {
    if constexpr (TYPE == IQ3_S) return Unit<TYPE>(sub, grid);
    else return Unit<TYPE>(sub);
}

__device__ __forceinline__ void store_out(void *dst, bool bf16, int64_t index, float v) {
    if (bf16) static_cast<uint16_t *>(dst)[index] = float_to_bf16_bits(v);
    else static_cast<float *>(dst)[index] = v;
}

// Sum over the G lanes of each lane group (lanes Gg..Gg+G-1); every lane gets its group's sum.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    v += dpp_f32<DPP_QUAD_1032>(v);
    v += dpp_f32<DPP_QUAD_2301>(v);
    v += dpp_f32<DPP_ROW_HALF_MIRROR>(v);
    if constexpr (G >= 16) v += dpp_f32<DPP_ROW_MIRROR>(v);
    if constexpr (G >= 32) v += __shfl_xor(v, 16, WAVE);
    if constexpr (G >= 64) v += __shfl_xor(v, 32, WAVE);
    return v;
}

// LDS bytes of the staged activation: per pass and row, nb Q8_1 blocks (36 bytes) and
// nb packed half sums (4 bytes).
inline size_t mmvq_act_lds_bytes(int64_t m, int64_t k, bool two_pass) {
    return size_t(two_pass ? 2 : 1) * size_t(m) * size_t(k / QK8_1) * 40;
}

// Coalesced weight stream for Q6_K (210-byte superblocks of four units whose fields are many
// small pieces) on long rows at one activation row. One step of a wave covers 16 superblocks
// (WAVE / G rows, G / 4 consecutive superblocks of each); they are read as U 16-byte units per
// superblock (the last running into the next superblock, ignored), lane l taking units l,
// l + 64, ..., into the wave's LDS transpose buffer (superblock j at j * SBP), from which each
// lane reads its unit's fields (the direct loads put 16 superblocks' small fields in every
// load instruction). Measured on MI355X: 5120 x 17408 at one row 25.2 -> 21.3 us, but at two
// and three rows +11 % and +32 % (the buffers cost resident workgroups), 5120 x 6144 (G = 16)
// +8 % and IQ3_S +25 %.
template <int TYPE, int M, int G> constexpr bool gemv_streamed() { return TYPE == Q6_K && M == 1 && G >= 32; }
template <int TYPE> struct GemvStream {
    // superblock pitch: whole units, plus one when U is even (16 superblocks on 16 different
    // 4-bank groups of the LDS, as in MmqsStream)
    static constexpr int SB = block_bytes(TYPE), U = (SB + 15) / 16, SBP = 16 * (U + (U % 2 == 0 ? 1 : 0));
    static constexpr int UPL = (16 * U + WAVE - 1) / WAVE;  // units per lane
    static constexpr int BUF = 16 * SBP + 16;               // and a spare unit
};

// Threads per workgroup, measured on MI355X: 512 on one row set when the activation
// staging is shared by more rows without leaving too few workgroups (short rows, G <= 16:
// qkv / o_proj -2..-7 %; or three and four rows: 5120 x 17408 down -13..-16 %); 256
// otherwise (two row sets: gate/up -8 % against 512; long rows at one or two activation
// rows: down +10..17 % at 512); 128 from five rows on.
template <int M, int RS, int G, int KS = 1> constexpr int mmvq_threads() {
    return M > 4 ? (KS > 1 ? 512 : 128) : ((KS > 1 && M >= 3) || (RS == 1 && (G <= 16 || M >= 3))) ? 512 : 256;
}

// KS > 1 (one row set per wave): the waves of a workgroup form groups of KS that share WAVE / G
// rows, wave kp of a group taking the kp-th of KS equal parts of each row's units; the group's
// totals are added in LDS in part order. It multiplies the resident waves of a matrix with few
// rows without staging the activation more often.
template <int TYPE, int M, bool TWO_PASS, int DEPTH, int G, int RS, int KS = 1>
__global__ __launch_bounds__((mmvq_threads<M, RS, G, KS>()))
void mmvq_kernel(const uint8_t *__restrict__ weight, int64_t row_bytes, int nrows, int units_per_row,
                 const block_q8_1 *__restrict__ y1, const block_q8_1 *__restrict__ y2, int y_row_blocks,
                 const float *__restrict__ inverse, void *__restrict__ dst, int64_t stride_dst, int dst_bf16) {
    static_assert(KS == 1 || RS == 1, "a K split takes one row set per wave");
    using U = Unit<TYPE>;
    constexpr int THREADS = mmvq_threads<M, RS, G, KS>();
    constexpr int BYTES = block_bytes(TYPE);
    constexpr int PASSES = TWO_PASS ? 2 : 1;
    constexpr int ROWS = M * PASSES;  // activation rows staged
    extern __shared__ __align__(16) uint8_t kai_mmvq_lds[];
    __shared__ uint32_t grid_lds[TYPE == IQ3_S ? 512 : 1];
    __shared__ float inv_lds[M];
    __shared__ float part_lds[KS > 1 ? (THREADS / WAVE / KS) * (KS - 1) * (WAVE / G) * M : 1];

    const int lane = threadIdx.x % WAVE;
    const int gpos = lane % G;
    // A wave owns RS row sets of WAVE / G consecutive rows, one group of G lanes per row,
    // streamed one after the other with the load ring running across their boundaries.
    const int wv = threadIdx.x / WAVE, kp = wv % KS, rg = wv / KS;  // K part and row group of the wave
    const int wave_row0 = (blockIdx.x * (THREADS / WAVE / KS) + rg) * (WAVE / G) * RS;
    auto row_of = [&](int rs) { return wave_row0 + rs * (WAVE / G) + lane / G; };
    const int nb = y_row_blocks;
    const U unit = make_unit<TYPE>(gpos % U::PER_BLOCK, grid_lds);
    const int T = (units_per_row + G - 1) / G;
    // the wave's steps of each row: [T0, T1) (all of them without a K split)
    const int T0 = KS > 1 ? kp * T / KS : 0, T1 = KS > 1 ? (kp + 1) * T / KS : T;

    // Prime the ring first so the staging below overlaps the HBM latency. Every load is
    // unconditional (unit indices are clamped to the row, rows to the matrix, steps past
    // the last row set to its last unit; clamped units contribute zero), so the compiler's
    // vmcnt waits are exact and DEPTH units per lane stay in flight. Step t of a lane is
    // unit gpos + G (t % T) of row set t / T, tracked by counters.
    const int last = units_per_row - 1;
    // Step positions (row set, step within the set) advance by one per unit, uniformly.
    auto advance = [&](int &rs, int &tu) {
        if (++tu == T1) {
            tu = T0;
            ++rs;
        }
    };
    // Streamed formats: the lane's units of a step (superblock j = u / U of the step, unit u % U)
    // as 32-bit byte offsets from the step's first superblock of the set's first row (the
    // launcher checks the matrix and 64 more rows stay below 4 GiB). Every unit start is clamped
    // to the matrix's last 16 bytes and its LDS position moved back by as many bytes (0 for a
    // unit wholly past the end), so no load leaves the matrix; such units (rows past nrows,
    // superblocks past a row's end) belong to lanes whose products are not live.
    constexpr bool STREAM = gemv_streamed<TYPE, M, G>();
    using S = GemvStream<TYPE>;
    static_assert(!STREAM || U::PER_BLOCK == 4, "a streamed step holds 16 superblocks of four units");
    uint32_t ug[S::UPL];
    int uoff[S::UPL];
#pragma unroll
    for (int i = 0; i < S::UPL; ++i) {
        const int u = lane + WAVE * i, j = u / S::U, c = u % S::U;
        const bool real = u < 16 * S::U;
        ug[i] = real ? static_cast<uint32_t>(j / (G / 4)) * static_cast<uint32_t>(row_bytes) +
                           static_cast<uint32_t>((j % (G / 4)) * S::SB + 16 * c)
                     : 0u;
        uoff[i] = real ? j * S::SBP + 16 * c : 16 * S::SBP;
    }
    const uint32_t tail = static_cast<uint32_t>(int64_t(nrows) * row_bytes - 16);
    struct Streamed {
        uint4 v[S::UPL];
        uint32_t back;  // 4 bits per unit: the bytes its load start was moved back
    };
    using Slot = typename std::conditional<STREAM, Streamed, typename U::W>::type;
    auto load_unit = [&](Slot &w, int rs, int tu) {
        if constexpr (STREAM) {
            // past the wave's last set: re-read the last set's last step (still cached)
            const int rsc = min(rs, RS - 1), tuc = rs >= RS ? T - 1 : tu;
            const uint32_t base = static_cast<uint32_t>(wave_row0 + rsc * (WAVE / G)) * static_cast<uint32_t>(row_bytes) +
                                  static_cast<uint32_t>(tuc * (G / 4) * S::SB);
            w.back = 0;
#pragma unroll
            for (int i = 0; i < S::UPL; ++i) {
                const uint32_t g = base + ug[i], a = min(g, tail), back = g - a;
                w.v[i] = load_unaligned<uint4>(weight + a);
                w.back |= (back < 16u ? back : 0u) << (4 * i);
            }
        } else {
            // Past the wave's last set: re-read the last unit of the last row (still cached).
            const int u = rs >= RS ? last : gpos + G * tu;
            const uint8_t *wrow = weight + static_cast<int64_t>(min(row_of(min(rs, RS - 1)), nrows - 1)) * row_bytes;
            unit.load_w(w, wrow + static_cast<int64_t>(min(u, last) / U::PER_BLOCK) * BYTES);
        }
    };
    Slot ring[DEPTH];
    int lrs = 0, ltu = T0;  // position of the next load
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
        load_unit(ring[d], lrs, ltu);
        advance(lrs, ltu);
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    }

    // Stage the IQ3_S grid, inverse[] and the activation: ROWS * nb blocks copied with
    // 16-byte vectors, then the exact code sums of each block's two 16-value halves.
    if constexpr (TYPE == IQ3_S) {
        for (int i = threadIdx.x; i < 512; i += THREADS) grid_lds[i] = iq3s_grid_global[i];
    }
    if (threadIdx.x < M) inv_lds[threadIdx.x] = inverse[threadIdx.x];
    uint8_t *act = kai_mmvq_lds;
    uint32_t *sums = reinterpret_cast<uint32_t *>(kai_mmvq_lds + size_t(ROWS) * nb * 36);
    {
        // 16-byte vectors by direct global-to-LDS copies where both ends are 16-byte aligned
        // (a wave's 64 lanes fill 1 KiB in lane order), all in flight at once: copied through
        // registers, each round of vectors waited for the previous one (and for the ring's
        // loads, issued before them)
        const int pass_bytes = M * nb * 36;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const uint8_t *src = reinterpret_cast<const uint8_t *>(p ? y2 : y1);
            uint8_t *dstl = act + p * pass_bytes;
            const int vec = pass_bytes / 16;
            if ((reinterpret_cast<uintptr_t>(src) & 15) == 0 && (p * pass_bytes) % 16 == 0) {  // uniform
                for (int i0 = (threadIdx.x / WAVE) * WAVE; i0 < vec; i0 += THREADS) {
                    if (i0 + lane < vec)
                        __builtin_amdgcn_global_load_lds(static_cast<const void *>(src + 16 * (i0 + lane)),
                                                         (__attribute__((address_space(3))) uint8_t *)dstl + 16 * i0,
                                                         16, 0, 0);
                }
            } else {
                for (int i = threadIdx.x; i < vec; i += THREADS) {
                    const uint4 v = load_unaligned<uint4>(src + 16 * i);  // 4-byte aligned runs
                    __builtin_memcpy(dstl + 16 * i, &v, 16);
                }
            }
            for (int i = 4 * vec + threadIdx.x; i < pass_bytes / 4; i += THREADS)
                reinterpret_cast<uint32_t *>(dstl)[i] = reinterpret_cast<const uint32_t *>(src)[i];
        }
        __syncthreads();
        const uint4 ones = make_uint4(0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u);
        for (int b = threadIdx.x; b < ROWS * nb; b += THREADS) {
            const int slo = dot16(ones, load_unaligned<uint4>(act + 36 * b + 4));
            const int shi = dot16(ones, load_unaligned<uint4>(act + 36 * b + 20));
            sums[b] = (static_cast<uint32_t>(slo) & 0xffffu) | (static_cast<uint32_t>(shi) << 16);
        }
        __syncthreads();
    }
    if (KS == 1 && wave_row0 >= nrows) return;  // whole wave past the last row (a K split meets a barrier below)
    // the wave's transpose buffer and the lane's superblock slot in it
    lds_u8 *tb = (lds_u8 *)kai_mmvq_lds + (size_t(ROWS) * nb * 40 + 15) / 16 * 16 + (threadIdx.x / WAVE) * S::BUF;
    const int jl = (lane / G) * (G / 4) + gpos / 4;

    float acc[M];
#pragma unroll
    for (int j = 0; j < M; ++j) acc[j] = 0.0f;

    // T >= 1; a do-while keeps the prologue loads from being sunk behind a zero-trip check.
    // The memory clobbers keep each unit's loads where they are issued and the scheduling
    // barriers keep the next unit's arithmetic (and its load waits) out of this one.
    const int TT = (RS * (T1 - T0) + DEPTH - 1) / DEPTH * DEPTH;
    int t0 = 0, rs = 0, tu = T0;  // position of the unit being multiplied
    do {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            const int u = gpos + G * tu;
            const bool live = u < units_per_row && rs < RS;  // false past the row end and the last set
            typename U::P w;
            if constexpr (STREAM) {
#pragma unroll
                for (int i = 0; i < S::UPL; ++i)
                    store_unaligned(tb + uoff[i] - int((ring[d].back >> (4 * i)) & 15u), ring[d].v[i]);
                typename U::W f;
                unit.load_w(f, tb + jl * S::SBP);
                w = unit.prep(f);
            } else {
                w = unit.prep(ring[d]);
            }
            load_unit(ring[d], lrs, ltu);
            advance(lrs, ltu);
            const int blk = min(u, last) / U::PER_BLOCK;
#pragma unroll
            for (int j = 0; j < M; ++j) {
#pragma unroll
                for (int p = 0; p < PASSES; ++p) {
                    const int r = p * M + j;
                    typename U::A a;
                    unit.load_a(a, ActLds{act + size_t(r) * nb * 36, sums + size_t(r) * nb}, blk);
                    const float v = unit.dot(w, a);
                    acc[j] += live ? v : 0.0f;
                }
            }
            if (RS > 1 && tu == T - 1 && rs < RS - 1) {  // row set rs complete (uniform); the last below
#pragma unroll
                for (int j = 0; j < M; ++j) {
                    const float total = group_sum<G>(acc[j]);
                    if (gpos == j % G && row_of(rs) < nrows)
                        store_out(dst, dst_bf16 != 0, static_cast<int64_t>(j) * stride_dst + row_of(rs), total * inv_lds[j]);
                    acc[j] = 0.0f;
                }
            }
            advance(rs, tu);
            __asm__ volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
        }
        t0 += DEPTH;
    } while (t0 < TT);

    // Group totals of the last row set; lane gpos of a group stores activation rows
    // j = gpos, gpos + G, ... (with a K split: part 0 after adding the other parts in order)
    const int row = row_of(RS - 1);
    float total[M];
#pragma unroll
    for (int j = 0; j < M; ++j) total[j] = group_sum<G>(acc[j]);
    if constexpr (KS > 1) {
        float *part = part_lds + (rg * (KS - 1) * (WAVE / G) + lane / G) * M;  // [group][part - 1][row][j]
        if (kp > 0 && gpos == 0) {
#pragma unroll
            for (int j = 0; j < M; ++j) part[(kp - 1) * (WAVE / G) * M + j] = total[j];
        }
        __syncthreads();
        if (kp > 0) return;
#pragma unroll
        for (int p = 1; p < KS; ++p)
#pragma unroll
            for (int j = 0; j < M; ++j) total[j] += part[(p - 1) * (WAVE / G) * M + j];
    }
#pragma unroll
    for (int j = 0; j < M; ++j) {
        if (gpos == j % G && row < nrows)
            store_out(dst, dst_bf16 != 0, static_cast<int64_t>(j) * stride_dst + row, total[j] * inv_lds[j]);
    }
}

// Row sets per wave: two when the matrix still gives at least four waves per SIMD of the
// device (4096 on a 256-CU MI355X) after pairing its row sets, for Q4_K at one to four activation rows
// and for the other formats at three or four; the second set's loads then overlap the
// first set's reduction and the activation is staged once per twice the weight bytes.
// Measured on MI355X, 34816 x 5120: Q4_K -11 %, -9 %, -14 %, -18 % at one to four rows;
// Q2_K and IQ3_S -10 % to -22 % at three and four rows but +5 % at one; smaller matrices
// lose parallelism and stay at one set.
template <int TYPE, int M>
inline int gemv_row_sets(int64_t n, int g, int cus) {
    const int64_t sets = (n + (WAVE / g) - 1) / (WAVE / g);
    const bool rows_ok = TYPE == Q4_K ? M <= 4 : (M >= 3 && M <= 4);
    return rows_ok && sets >= 2 * 16 * int64_t(cus) ? 2 : 1;
}

// K split (one row set per wave): waves sharing each row, so that a matrix of few rows still
// puts 4 waves on every SIMD of the device: 2 below 16 waves per CU (4096 on a 256-CU
// MI355X), 4 below 8 per CU, each part
// keeping at least two steps of its rows; 512-thread workgroups at three and four activation
// rows, 256 at one and two. Measured on MI355X: at three / four rows Q6_K 5120x6144 14.4 / 16.2
// -> 13.4 / 14.6 us, IQ3_S 5120x17408 27.8 / 38.0 -> 24.7 / 35.8, Q4_0 2048x8192 at four rows
// 9.8 -> 9.0, but Q2_K 5120x17408 at three rows 26.0 -> 28.8; at one / two rows (whole calls
// with the preparation) Q2_K 5120x17408 14.7 / 20.3 -> 13.0 / 19.0, Q4_K 7168x5120 9.88 / 10.58
// -> 9.49 / 10.80, Q4_0 3072x2048 7.89 / 8.01 -> 7.00 / 7.20, Q4_0 2048x8192 8.58 / 9.43 -> 8.34 /
// 9.86, but Q6_K 5120x17408 22.97 / 27.98 -> 24.43 / 31.26 and 5120x6144 14.18 / 14.65 -> 14.86 /
// 16.10. So Q2_K splits at one and two rows; Q4_K, Q4_0 and Q8_0 at one row, and Q4_0 and Q8_0
// at two rows on rows of at most 2048 values; every other format at three and four; and Q4_0 at
// five to eight rows, which the GEMV takes only on matrices of few rows
// (gemv_rows_before_persistent), with 512-thread workgroups.
template <int TYPE, int M>
constexpr bool gemv_k_split_rows(int64_t k) {
    if (M > 4) return M <= 8 && TYPE == Q4_0;
    if (M >= 3) return TYPE != Q2_K;
    if (TYPE == Q2_K) return M <= 2;
    if (M == 1) return TYPE == Q4_K || TYPE == Q4_0 || TYPE == Q8_0;
    return M == 2 && (TYPE == Q4_0 || TYPE == Q8_0) && k <= 2048;
}
template <int TYPE, int M>
inline int gemv_k_split(int64_t n, int64_t k, int g, int cus) {
    if (!gemv_k_split_rows<TYPE, M>(k)) return 1;
    const int64_t k_units = (k / block_elems(TYPE)) * Unit<TYPE>::PER_BLOCK;
    const int64_t waves = (n + (WAVE / g) - 1) / (WAVE / g), steps = (k_units + g - 1) / g;
    const int ks = waves < 8 * int64_t(cus) ? 4 : waves < 16 * int64_t(cus) ? 2 : 1;
    return steps >= 2 * ks ? ks : steps >= 4 ? 2 : 1;
}

template <int TYPE, int M, bool TWO_PASS, int G, int RS, int KS = 1>
static void launch_sets(const uint8_t *w, int64_t n, int64_t k, const block_q8_1 *y1, const block_q8_1 *y2,
                        const float *inverse, void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream) {
    constexpr int THREADS = mmvq_threads<M, RS, G, KS>();
    // ring depth: one unit per lane in flight for the 256-value superblock formats with one
    // row set per wave; two with two row sets (whose next set's loads overlap the previous
    // set's reduction) and for the 32-value formats (one small block per unit). A deeper
    // ring costs more waves than it hides; measured on MI355X, one against two units: Q6_K
    // down and o_proj -8..-11 %, Q4_K qkv -5..-10 %, Q2_K gate/up -24 %, IQ3_S down
    // -6..-11 %, but Q4_K gate/up (two row sets) +3 % and Q4_0 down +15 %; two against
    // three: gate/up b2 -14 %, qkv and o_proj -3..-8 %.
    constexpr int DEPTH = RS == 1 && block_elems(TYPE) == 256 ? 1 : 2;
    constexpr int QK = block_elems(TYPE);
    const int64_t blocks_per_row = k / QK;
    const int64_t row_bytes = blocks_per_row * block_bytes(TYPE);
    const int units = static_cast<int>(blocks_per_row * Unit<TYPE>::PER_BLOCK);
    const int64_t rows_per_block = (THREADS / WAVE / KS) * (WAVE / G) * RS;
    constexpr bool STREAM = gemv_streamed<TYPE, M, G>();
    const size_t lds = (mmvq_act_lds_bytes(M, k, TWO_PASS) + 15) / 16 * 16 +
                       (STREAM ? size_t(THREADS / WAVE) * GemvStream<TYPE>::BUF : 0);
    if (lds + (TYPE == IQ3_S ? 2048 : 0) + 64 > size_t(MMVQ_LDS_BUDGET))
        throw Error("GEMV activation does not fit in LDS (m * k too large)");
    if (STREAM && (n + 64) * row_bytes >= (int64_t(1) << 32)) throw Error("The GEMV takes matrices below 4 GiB");
    auto kernel = mmvq_kernel<TYPE, M, TWO_PASS, DEPTH, G, RS, KS>;
    static DeviceFlags lds_raised;  // per instantiation and device
    raise_dynamic_lds(reinterpret_cast<const void *>(kernel), MMVQ_LDS_BUDGET - 4096, lds_raised,
                      "Cannot raise the GEMV dynamic LDS limit");
    kernel<<<dim3(static_cast<unsigned>((n + rows_per_block - 1) / rows_per_block)), dim3(THREADS), lds, stream>>>(
        w, row_bytes, static_cast<int>(n), units, y1, y2, static_cast<int>(k / QK8_1), inverse, dst, stride_dst,
        dst_bf16 ? 1 : 0);
}

template <int TYPE, int M, bool TWO_PASS, int G>
static void launch_variant(const uint8_t *w, int64_t n, int64_t k, const block_q8_1 *y1, const block_q8_1 *y2,
                           const float *inverse, void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream) {
    if constexpr (M <= 4 || (M <= 8 && TYPE == Q4_0)) {
        if constexpr (M <= 4) {
            if (gemv_row_sets<TYPE, M>(n, G, device_cu_count()) == 2) {
                launch_sets<TYPE, M, TWO_PASS, G, 2>(w, n, k, y1, y2, inverse, dst, dst_bf16, stride_dst, stream);
                return;
            }
        }
        switch (gemv_k_split<TYPE, M>(n, k, G, device_cu_count())) {
            case 4: launch_sets<TYPE, M, TWO_PASS, G, 1, 4>(w, n, k, y1, y2, inverse, dst, dst_bf16, stride_dst, stream); return;
            case 2: launch_sets<TYPE, M, TWO_PASS, G, 1, 2>(w, n, k, y1, y2, inverse, dst, dst_bf16, stride_dst, stream); return;
            default: break;
        }
    }
    launch_sets<TYPE, M, TWO_PASS, G, 1>(w, n, k, y1, y2, inverse, dst, dst_bf16, stride_dst, stream);
}

// Lanes per row: 16, doubled while a row would leave more than 8 units per lane. A
// group's loads then span 16-32 consecutive units (0.5-1 KiB) of its row, the shape
// that streams best on MI355X (measured across G = 8..64 for every format and matrix
// shape here); the grid size is secondary.
template <int TYPE, int M>
static int pick_group(int64_t n, int64_t k) {
    (void)n;
    const int64_t units = (k / block_elems(TYPE)) * Unit<TYPE>::PER_BLOCK;
    int g = 16;
    while (g < 64 && units / g > 8) g *= 2;
    return g;
}

template <int TYPE, int M, bool TWO_PASS>
static void launch_group(const uint8_t *w, int64_t n, int64_t k, const block_q8_1 *y1, const block_q8_1 *y2,
                         const float *inverse, void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream) {
    switch (pick_group<TYPE, M>(n, k)) {
        case 16: launch_variant<TYPE, M, TWO_PASS, 16>(w, n, k, y1, y2, inverse, dst, dst_bf16, stride_dst, stream); break;
        case 32: launch_variant<TYPE, M, TWO_PASS, 32>(w, n, k, y1, y2, inverse, dst, dst_bf16, stride_dst, stream); break;
        default: launch_variant<TYPE, M, TWO_PASS, 64>(w, n, k, y1, y2, inverse, dst, dst_bf16, stride_dst, stream); break;
    }
}

template <int TYPE, int M>
static void launch_m(const void *weight, int64_t n, int64_t k, const block_q8_1 *y1, const block_q8_1 *y2,
                     const float *inverse, void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream) {
    const auto *w = static_cast<const uint8_t *>(weight);
    if (y2) {
        if constexpr (M <= 8) launch_group<TYPE, M, true>(w, n, k, y1, y2, inverse, dst, dst_bf16, stride_dst, stream);
        else throw Error("Two-pass activations are supported for up to 8 rows");
    } else {
        launch_group<TYPE, M, false>(w, n, k, y1, y2, inverse, dst, dst_bf16, stride_dst, stream);
    }
}

template <int TYPE>
static void launch_rows(const void *weight, int64_t n, int64_t k, int64_t m, const block_q8_1 *y1,
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

// Per-type entry used by launch_mmvq; one translation unit per type keeps builds parallel.
// Activation rows are split into launches whose staged activation fits in LDS (each
// launch streams the weights once).
template <int TYPE>
void launch_mmvq_type(const void *weight, int64_t n, int64_t k, int64_t m, const block_q8_1 *y1,
                      const block_q8_1 *y2, const float *inverse, void *dst, bool dst_bf16, int64_t stride_dst,
                      hipStream_t stream) {
    const int64_t per_row = int64_t(mmvq_act_lds_bytes(1, k, y2 != nullptr));
    const int64_t fit = (MMVQ_LDS_BUDGET - 4096) / per_row;  // one streamed row's buffers fit beside any k
    if (fit < 1) throw Error("GEMV activation row does not fit in LDS");
    const int64_t nb = k / QK8_1;
    const size_t elem = dst_bf16 ? 2 : 4;
    for (int64_t j0 = 0; j0 < m; j0 += fit) {
        const int64_t mm = std::min(fit, m - j0);
        launch_rows<TYPE>(weight, n, k, mm, y1 + j0 * nb, y2 ? y2 + j0 * nb : nullptr, inverse + j0,
                          static_cast<char *>(dst) + size_t(j0) * size_t(stride_dst) * elem, dst_bf16, stride_dst,
                          stream);
    }
}

}  // namespace kai
