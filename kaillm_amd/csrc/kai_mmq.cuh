// Batched GEMM for more than 8 activation rows (kernels 2 and 3): multi-sequence
// decode, spec-verify (m = 16..80) and prefill (m = 512..2048), on int8 MFMA.
//
// Y[m, n] = inverse[m] * sum_b dot(W[n, b], q8[m, b]) with exact per-block integer dots
// and fp32 scalings. Two activations: the decode path's Q8_1 blocks (up to 8 rows, paired
// tile, reached from kai_fused_mmvq) and the batched path's planes of GGML MMQ
// quantisation (kai_fused_mmq_run, current_ggml_direct.cu:1025-1092,1196-1265), whose
// layout per format fixes the activation scale (fp32 per 32 values for D4, fp16 per 32
// for DS4, fp16 per 64 for D2S6) and the min-term sums (stored fp16 sums for DS4, per-16
// sums of D2S6 for the first 96 values of each 128, code sums times d elsewhere).
//
// Design for gfx950 (wave64, v_mfma_i32_16x16x32_i8):
//   * each wave owns 16*TN weight rows and streams their wire bytes from HBM straight
//     into registers (one K step in flight); a lane holds, for its row (lane % 16) and
//     octet (lane / 16), the 8 codes of every 32-value block that the MFMA B operand
//     needs, so weights never pass through LDS and the wave needs no barrier for them;
//   * the activation rows of the tile (MT = 16*TM) are staged once per K step into LDS
//     by the whole workgroup (double-buffered, one barrier per step) in an MFMA layout:
//     codes [block][row][32], scales d8 [block][row], and the activation factors of the
//     min terms [term][row], so the A operand is one ds_read_b64 and the four row
//     scales of a lane one ds_read_b128;
//   * per 32-value block: one int8 MFMA gives the exact block dot of 16 rows x 16 weight
//     rows, the fp32 epilogue multiplies by d8 * weight scale (three VALU operations
//     per element, the bound of this kernel: the scales on both operands change every
//     32 values, so the integer accumulation cannot run across blocks);
//   * min/offset terms (Q4_0 8*s8, Q4_K dmin*m*sum, Q2_K per-16 mins) are small rank-8/16
//     products per K step: they run on v_mfma_f32_16x16x4_f32 into the same
//     accumulators instead of the VALU;
//   * several waves of a workgroup may split K (KS) when there are too few weight rows
//     to fill the chip; their partial sums are added in LDS in a fixed order;
//   * up to 8 activation rows (PAIR): two 32-value blocks share one
//     v_mfma_i32_16x16x64_i8. The B operand is the lane's codes of blocks 2c and 2c+1,
//     the A operand holds block 2c's activation codes in rows 0-7 and block 2c+1's in
//     rows 8-15, each zero against the other block's codes, so D rows 0-7 are the dots
//     of block 2c and rows 8-15 those of block 2c+1 for the same 8 activation rows.
//     Every element of the fp32 epilogue is then a real one (a 16-row tile would pad 8
//     rows), which halves the epilogue's VALU work; the two halves are added once at
//     the end.
// Operand layouts (checked on gfx950): 16x16x32_i8: lane l holds A row l%16 and B
// column l%16 for k = 8*(l/16) .. +8; 16x16x4_f32: A row l%16, B column l%16, k = l/16;
// both: D column l%16, rows 4*(l/16) + i.
#pragma once

#include <atomic>
#include <type_traits>

#include "kai_mmq_formats.h"

namespace kai {

// Activation factors of the min terms for block kb of one row, from its Q8_1 block.
template <int TYPE>
__device__ __forceinline__ void act_terms(const uint4 q0, const uint4 q1, uint32_t ds, float d8, float *t) {
    if constexpr (TYPE == Q4_0) {
        t[0] = half_bits_to_float(ds >> 16);  // stored s8
    } else if constexpr (TYPE == Q4_K || TYPE == Q2_K) {
        const uint4 ones = make_uint4(0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u);
        const int lo = dot16(ones, q0), hi = dot16(ones, q1);
        if constexpr (TYPE == Q4_K) {
            t[0] = d8 * static_cast<float>(lo + hi);
        } else {
            t[0] = d8 * static_cast<float>(lo);
            t[1] = d8 * static_cast<float>(hi);
        }
    }
}

// Scale d8 and min-term activation factors of 32-value block b (0..7 of the K step) of one
// row, from the batched path's plane: h0 is the header word of the block (D4: fp32 d;
// DS4: half2 (d, sum); D2S6: half2 of the two per-64 scales), h1 the D2S6 word of stored
// per-16 sums of the block (absent for the last 32 values of a 128-value block).
template <int TYPE>
__device__ __forceinline__ float plane_terms(const uint4 q0, const uint4 q1, uint32_t h0, uint32_t h1, int b,
                                             float *t) {
    constexpr int L = mmq_layout(TYPE);
    float d8;
    if constexpr (L == MMQ_D4) d8 = __builtin_bit_cast(float, h0);
    else if constexpr (L == MMQ_DS4) d8 = half_bits_to_float(h0 & 0xffffu);
    else d8 = half_bits_to_float((h0 >> (16 * ((b & 3) >> 1))) & 0xffffu);
    const uint4 ones = make_uint4(0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u);
    if constexpr (TYPE == Q4_0) {
        t[0] = d8 * static_cast<float>(dot16(ones, q0) + dot16(ones, q1));
    } else if constexpr (TYPE == Q4_K) {
        t[0] = half_bits_to_float(h0 >> 16);
    } else if constexpr (TYPE == Q2_K) {
        if ((b & 3) < 3) {
            t[0] = half_bits_to_float(h1 & 0xffffu);
            t[1] = half_bits_to_float(h1 >> 16);
        } else {
            t[0] = d8 * static_cast<float>(dot16(ones, q0));
            t[1] = d8 * static_cast<float>(dot16(ones, q1));
        }
    }
    return d8;
}

template <int TYPE, int TM, bool PAIR = false>
constexpr int mmq_buf_bytes() {  // one K step of MT activation rows in LDS (PAIR: 8 rows)
    return (PAIR ? 8 : 16 * TM) * (8 * 32 + 8 * 4 + MmqW<TYPE>::NTERM * 4);
}

// LDS of a workgroup: the double-buffered activation steps of its k-groups (reused for the
// K-split sums after the loop), then each wave's weight transpose buffers (TN row tiles of 16
// rows, MmqsStream).
template <int TYPE, int TM, int TN, int KS, bool PAIR = false>
constexpr size_t mmq_act_lds_bytes() {
    const size_t act = size_t(2) * KS * mmq_buf_bytes<TYPE, TM, PAIR>();
    const size_t red = KS > 1 ? size_t(KS - 1) * (4 / KS) * WAVE * TM * TN * 4 * sizeof(float) : 0;
    return ((act > red ? act : red) + 15) / 16 * 16;
}
template <int TYPE> constexpr int mmq_tile_tbuf() { return 16 * MmqsStream<TYPE>::SBP + 16; }
// Formats whose weights go through the coalesced stream: superblocks that are not whole
// 16-byte units, whose fields are many small pieces (Q6_K 210 bytes, IQ3_S 110). Measured
// on MI355X against the direct field loads: Q6_K 5120 x 17408 at 8 / 32 / 80 rows -12 / -25
// / -23 %, 5120 x 6144 at 8 rows -17 %, IQ3_S 5120 x 17408 at 8 rows -42 %; Q4_K
// 34816 x 5120 +11 % (8 rows) to +22 % (80) and Q2_K +11 % at 512 rows, whose direct loads
// are whole 16-byte pieces already.
template <int TYPE> constexpr bool mmq_streamed() { return TYPE == Q6_K || TYPE == IQ3_S; }
template <int TYPE, int TM, int TN, int KS, bool PAIR = false>
constexpr size_t mmq_lds_bytes() {
    return mmq_act_lds_bytes<TYPE, TM, TN, KS, PAIR>() +
           (mmq_streamed<TYPE>() ? size_t(MMQ_THREADS / WAVE) * TN * mmq_tile_tbuf<TYPE>() : 0);
}

// Row r, block b (0..7) of one staged K step of MT activation rows: the codes at
// (b*MT + r)*32 with the four 8-byte octets placed at position oct ^ ((r >> 2) & 3), so that
// the A-operand reads of a wave (16 rows x 4 octets) hit distinct banks; d8 at [b][r]; the
// min-term factors at [term][r] (one per block, or two for per-16 terms).
template <int TYPE, int MT>
__device__ __forceinline__ void stage_block(uint8_t *base, int r, int b, uint4 q0, uint4 q1, float d8,
                                            const float (&t)[2]) {
    constexpr int NT = MmqW<TYPE>::NTERM, D8_OFF = MT * 8 * 32, TA_OFF = D8_OFF + MT * 8 * 4;
    const int sw = (r >> 2) & 3;
    uint4 *q = reinterpret_cast<uint4 *>(base + (b * MT + r) * 32);
    const uint4 h0 = sw & 1 ? make_uint4(q0.z, q0.w, q0.x, q0.y) : q0;
    const uint4 h1 = sw & 1 ? make_uint4(q1.z, q1.w, q1.x, q1.y) : q1;
    q[sw >> 1] = h0;
    q[(sw >> 1) ^ 1] = h1;
    reinterpret_cast<float *>(base + D8_OFF)[b * MT + r] = d8;
    if constexpr (NT > 0) {
        float *ta = reinterpret_cast<float *>(base + TA_OFF);
        if constexpr (NT == 8) {
            ta[b * MT + r] = t[0];
        } else {
            ta[(2 * b) * MT + r] = t[0];
            ta[(2 * b + 1) * MT + r] = t[1];
        }
    }
}

// One K step of the paired tile (up to 8 activation rows; decode arithmetic) for TN tiles of
// 16 weight rows: w holds each tile's fields of the step (after fix), base the step's
// activation in LDS in the paired layout (MT = 8: codes [block][row][32] with the octet
// swizzle, d8 [block][row], min-term factors [term][row]).
// PHASED: each pair of blocks in its own scheduling section, so that one pair's operands and
// MFMA results are live at a time (without it the persistent kernel's Q6_K loop spills).
template <int TYPE, int TN, bool PHASED = false>
__device__ __forceinline__ void paired_step(const typename MmqLoad<TYPE>::Raw (&w)[TN], const uint8_t *base,
                                            v4f_t (&acc)[TN], int col, int oct, int aoct, const uint32_t *grid) {
    using W = MmqLoad<TYPE>;
    constexpr int MODE = W::template mode<false>();
    constexpr int MT = 8, NT = W::NTERM, D8_OFF = MT * 8 * 32, TA_OFF = D8_OFF + MT * 8 * 4;
    const float *d8s = reinterpret_cast<const float *>(base + D8_OFF);
    const v4i_t zero = {0, 0, 0, 0};
    // lane's A row: activation row col % 8 of block 2c + col / 8; its D rows
    // 4*oct .. +4: activation rows 4*(oct % 2) .. +4 of block 2c + oct / 2
    const int mr = col & 7, hi = col >> 3, ob = oct >> 1;
    // split scales: the superblock scale (the same for every block of the step) multiplies the
    // step's sums once, at the end
    v4f_t part[TN];
    if constexpr (MODE == MMQ_ISPLIT) {
#pragma unroll
        for (int t = 0; t < TN; ++t) part[t] = v4f_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint64_t aq =
            *reinterpret_cast<const uint64_t *>(base + ((2 * c + hi) * MT + mr) * 32 + 8 * (aoct ^ ((mr >> 2) & 3)));
        const int a0 = static_cast<int>(aq), a1 = static_cast<int>(aq >> 32);
        const v4i_t av = hi ? v4i_t{0, 0, a0, a1} : v4i_t{a0, a1, 0, 0};
        const float4 dv = *reinterpret_cast<const float4 *>(d8s + (2 * c + ob) * MT + 4 * (oct & 1));
        const float d8[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
        for (int t = 0; t < TN; ++t) {
            const uint64_t c0 = W::template codes<false>(w[t], 2 * c, oct, grid),
                           c1 = W::template codes<false>(w[t], 2 * c + 1, oct, grid);
            const v4i_t bv = {static_cast<int>(c0), static_cast<int>(c0 >> 32), static_cast<int>(c1),
                              static_cast<int>(c1 >> 32)};
            if constexpr (MODE == MMQ_ISPLIT) {
                // all 32 values, and the second 16 alone: sl * (all - second) + sh * second
                const bool first = W::first_half(oct);
                const v4i_t ra = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, zero, 0, 0, 0);
                const v4i_t r2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, first ? zero : bv, zero, 0, 0, 0);
                const int sl = ob ? W::iscale(w[t], 4 * c + 2) : W::iscale(w[t], 4 * c);
                const int sh = ob ? W::iscale(w[t], 4 * c + 3) : W::iscale(w[t], 4 * c + 1);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int x = __mul24(sl, ra[i]) + __mul24(sh - sl, r2[i]);
                    part[t][i] = fmaf(d8[i], static_cast<float>(x), part[t][i]);
                }
            } else {
                const float sa = ob ? W::template scale<false>(w[t], 2 * c + 1) : W::template scale<false>(w[t], 2 * c);
                const v4i_t r = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, zero, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(d8[i] * sa, static_cast<float>(r[i]), acc[t][i]);
            }
        }
        if constexpr (PHASED) __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (MODE == MMQ_ISPLIT) {
#pragma unroll
        for (int t = 0; t < TN; ++t) {
            const float sa = W::template scale<false>(w[t], 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(sa, part[t][i], acc[t][i]);
        }
    }
    if constexpr (NT > 0) {  // the terms go to D rows 0-7 (activation rows 0-7), A rows 8-15 zero
        const float *ta = reinterpret_cast<const float *>(base + TA_OFF);
#pragma unroll
        for (int j = 0; j < NT / 4; ++j) {
            const float at = col < 8 ? ta[(4 * j + oct) * MT + col] : 0.0f;
#pragma unroll
            for (int t = 0; t < TN; ++t)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(at, W::template term<false>(w[t], j, oct), acc[t], 0, 0, 0);
        }
    }
}

// K pieces across the workgroups of one launch (the paired tile on long rows of matrices
// with too few row sets to fill the chip): each launch takes a slot of partial sums and an
// arrival count per group of workgroups that share output elements. The host rotates the slot per launch, so launches in flight at once on other
// streams take other slots; more than KAI_ZSLOTS such launches overlapping on one device race.
// Every launch leaves its counts at zero. The sums are written through to memory and read
// past the caches (system-scope stores and loads), so a count needs only the writer's own
// wait for its stores before it, not an agent-scope release (whose L2 write-back per
// workgroup costs more than the split gains).
constexpr int KAI_ZSLOTS = 4, KAI_ZCAP = 1 << 19, KAI_ZSETS = 8192;
static __device__ float kai_zpart[KAI_ZSLOTS][KAI_ZCAP];
static __device__ unsigned kai_zcount[KAI_ZSLOTS][KAI_ZSETS];
inline unsigned kai_next_zslot() {
    static std::atomic<unsigned> next{0};
    return next.fetch_add(1, std::memory_order_relaxed) % KAI_ZSLOTS;
}
__device__ __forceinline__ void zpart_store(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ float zpart_load(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
// The wave's stores are acknowledged (vmcnt counts stores on this architecture).
__device__ __forceinline__ void zpart_stores_done() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    __asm__ volatile("" ::: "memory");
}
// Arrival at a count: true for the last of `pieces` arrivals (which clears the count). Called
// by one lane after zpart_stores_done; the caller orders its later loads of the sums after it.
__device__ __forceinline__ bool zpart_arrive_last(unsigned *count, int pieces) {
    const unsigned arrived = __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = arrived == static_cast<unsigned>(pieces - 1);
    if (last) __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return last;
}

// PAIR: up to 8 rows of decode Q8_1 blocks (act: block_q8_1 [m][k/32], k % 256 == 0);
// otherwise the batched path's plane of the type's layout (act: uint8 plane), any k that is
// a whole number of blocks (a short last step reads zero activations).
// EXACT (planes only): the decode path's exact weight products in place of GGML MMQ's
// fp16-rounded ones; the legacy MMQ keeps d * sc and dmin * m in fp32 (vecdotq.cuh:353-377).
template <int TYPE, int TM, int TN, int KS, int DEPTH, bool PAIR, bool EXACT = false>
__global__ __launch_bounds__(MMQ_THREADS) void mmq_kernel(
    const uint8_t *__restrict__ weight, int64_t row_bytes, int n, int k, const void *__restrict__ act,
    int m, const float *__restrict__ inverse, void *__restrict__ dst, int64_t stride_dst, int dst_bf16,
    int zsteps, int zslot) {
    using W = MmqLoad<TYPE>;
    static_assert(!PAIR || TM == 1, "paired blocks use one tile of 8 activation rows");
    static_assert(!(PAIR && EXACT), "the paired tile's arithmetic is exact already");
    constexpr bool BATCHED = !PAIR && !EXACT;  // GGML MMQ's weight arithmetic
    constexpr int MODE = W::template mode<BATCHED>();  // decode (paired) or batched arithmetic
    constexpr int MT = PAIR ? 8 : 16 * TM, RG = 4 / KS, NT = W::NTERM;
    constexpr int BUF = mmq_buf_bytes<TYPE, TM, PAIR>();
    constexpr int D8_OFF = MT * 8 * 32, TA_OFF = D8_OFF + MT * 8 * 4;
    constexpr int PAIRS = KS * MT * 8;  // (k-group, row, block) activation blocks per iteration
    constexpr int PP = (PAIRS + MMQ_THREADS - 1) / MMQ_THREADS;
    extern __shared__ __align__(16) uint8_t kai_mmq_lds[];
    __shared__ uint32_t grid_lds[TYPE == IQ3_S ? 512 : 1];

    const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
    const int rg = wave % RG, kg = wave / RG;
    const int col = lane % 16, oct = lane / 16;
    // PAIR with zsteps > 0: this workgroup's K piece, steps [z * zsteps, (z + 1) * zsteps)
    const int nb = k / QK8_1, all_steps = (k + MMQ_STEP - 1) / MMQ_STEP;
    const int sbase = PAIR && zsteps > 0 ? static_cast<int>(blockIdx.z) * zsteps : 0;
    const int steps = PAIR && zsteps > 0 ? min(all_steps - sbase, zsteps) : all_steps;
    const int iters = (steps + KS - 1) / KS;
    const int m0 = blockIdx.y * MT;
    const int nrow0 = blockIdx.x * (16 * TN * RG) + rg * 16 * TN;
    if constexpr (TYPE == IQ3_S) {
        for (int i = tid; i < 512; i += MMQ_THREADS) grid_lds[i] = mmq_iq3s_grid[i];
    }

    // ---- activation staging: global Q8_1 blocks -> registers -> LDS (MFMA layout)
    uint4 aq0[PP], aq1[PP];
    uint32_t ads[PP], ads2[PP];
    auto aload = [&](int it) {
#pragma unroll
        for (int p = 0; p < PP; ++p) {
            const int idx = tid + p * MMQ_THREADS;
            const int r = idx % MT, b = (idx / MT) % 8, g = idx / (MT * 8);
            const int s = it * KS + g, row = m0 + r;
            aq0[p] = aq1[p] = make_uint4(0, 0, 0, 0);
            ads[p] = ads2[p] = 0;
            if (idx < PAIRS && s < steps && row < m) {
                if constexpr (PAIR) {
                    const uint8_t *src = reinterpret_cast<const uint8_t *>(
                        static_cast<const block_q8_1 *>(act) + int64_t(row) * nb + 8 * (sbase + s) + b);
                    ads[p] = load_unaligned<uint32_t>(src);
                    aq0[p] = load_unaligned<uint4>(src + 4);
                    aq1[p] = load_unaligned<uint4>(src + 20);
                } else {
                    // 128-value block 2s + b/4 of the row; 32-value block b % 4 inside it
                    const int sub = b & 3;
                    const uint8_t *blk = static_cast<const uint8_t *>(act) +
                                         (int64_t(2 * s + (b >> 2)) * m + row) * MMQ_BLOCK_BYTES;
                    const uint32_t *hdr = reinterpret_cast<const uint32_t *>(blk);
                    if constexpr (mmq_layout(TYPE) == MMQ_D2S6) {
                        ads[p] = hdr[0];
                        ads2[p] = sub < 3 ? hdr[1 + sub] : 0u;
                    } else {
                        ads[p] = hdr[sub];
                    }
                    aq0[p] = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * sub);
                    aq1[p] = *reinterpret_cast<const uint4 *>(blk + 32 + 32 * sub);
                }
            }
        }
    };
    // the staged step in the MFMA layout (stage_block)
    auto astore = [&](int buf) {
#pragma unroll
        for (int p = 0; p < PP; ++p) {
            const int idx = tid + p * MMQ_THREADS;
            if (idx < PAIRS) {
                const int r = idx % MT, b = (idx / MT) % 8, g = idx / (MT * 8);
                float d8, t[2];
                if constexpr (PAIR) {
                    d8 = half_bits_to_float(ads[p] & 0xffffu);
                    act_terms<TYPE>(aq0[p], aq1[p], ads[p], d8, t);
                } else {
                    d8 = plane_terms<TYPE>(aq0[p], aq1[p], ads[p], ads2[p], b, t);
                }
                stage_block<TYPE, MT>(kai_mmq_lds + (buf * KS + g) * BUF, r, b, aq0[p], aq1[p], d8, t);
            }
        }
    };

    // ---- weights: DEPTH K steps in flight per wave. Direct: each lane loads its fields of
    // its row (rows past n re-read row n - 1). Streamed (mmq_streamed): the coalesced unit
    // stream of each row tile (MmqsStream): the lane's units (row u / U, unit u % U) as 32-bit
    // byte offsets (the launcher checks the matrix is below 4 GiB). Every unit start is clamped
    // to the matrix's last 16 bytes and its LDS position moved back by as many bytes (0 for a
    // unit wholly past the end, whose rows are never stored), so no load leaves the matrix:
    // rows past n, the last unit of a superblock that is not whole units, a short last step.
    constexpr bool STREAM = mmq_streamed<TYPE>();
    const uint8_t *wrow[TN];
#pragma unroll
    for (int t = 0; t < TN; ++t) wrow[t] = weight + int64_t(min(nrow0 + 16 * t + col, n - 1)) * row_bytes;
    using S = MmqsStream<TYPE>;
    uint32_t ug[S::UPL];
    int uoff[S::UPL];
#pragma unroll
    for (int i = 0; i < S::UPL; ++i) {
        const int u = lane + WAVE * i, r = u / S::U, c = u % S::U;
        const bool real = u < 16 * S::U;
        ug[i] = real ? static_cast<uint32_t>(r) * static_cast<uint32_t>(row_bytes) + 16 * c : 0u;
        uoff[i] = real ? r * S::SBP + 16 * c : 16 * S::SBP;  // a spare unit past the 16 rows
    }
    const uint32_t tail = static_cast<uint32_t>(int64_t(n) * row_bytes - 16);
    lds_u8 *tbuf = (lds_u8 *)kai_mmq_lds + mmq_act_lds_bytes<TYPE, TM, TN, KS, PAIR>() + wave * TN * mmq_tile_tbuf<TYPE>();
    struct Streamed {
        uint4 v[TN][S::UPL];
        uint32_t back[TN];  // 4 bits per unit: the bytes its load start was moved back
    };
    struct Direct {
        typename W::Raw raw[TN];
    };
    using Slot = typename std::conditional<STREAM, Streamed, Direct>::type;
    Slot wr[DEPTH];
    auto wload = [&](Slot &sl, int it) {
        if constexpr (STREAM) {
            const uint32_t step = static_cast<uint32_t>(sbase + min(it * KS + kg, steps - 1)) * S::SB;
#pragma unroll
            for (int t = 0; t < TN; ++t) {
                const uint32_t base = static_cast<uint32_t>(nrow0 + 16 * t) * static_cast<uint32_t>(row_bytes) + step;
                sl.back[t] = 0;
#pragma unroll
                for (int i = 0; i < S::UPL; ++i) {
                    const uint32_t g = base + ug[i], a = min(g, tail), back = g - a;
                    sl.v[t][i] = load_unaligned<uint4>(weight + a);
                    sl.back[t] |= (back < 16u ? back : 0u) << (4 * i);
                }
            }
        } else if constexpr (PAIR) {
            const int s = sbase + min(it * KS + kg, steps - 1);  // past the end: the last step again
#pragma unroll
            for (int t = 0; t < TN; ++t) W::load(sl.raw[t], wrow[t] + int64_t(s) * W::SB, oct, 8);
        } else {
            const int s = it * KS + kg;
            if (s < steps) {
                const int nvalid = min(8, nb - 8 * s);  // 32-value blocks of this step inside the row
#pragma unroll
                for (int t = 0; t < TN; ++t) W::load(sl.raw[t], wrow[t] + int64_t(s) * W::SB, oct, nvalid);
            }
        }
    };
    // The step's fields of each row tile: streamed, from the wave's transpose buffer (each wave
    // writes and reads its own buffer, in order, so no barrier is needed).
    auto wfields = [&](const Slot &sl, typename W::Raw (&w)[TN], int it) {
        if constexpr (STREAM) {
            const int nvalid = PAIR ? 8 : min(8, nb - 8 * (it * KS + kg));  // blocks of the step inside the row
#pragma unroll
            for (int t = 0; t < TN; ++t) {
                lds_u8 *tt = tbuf + t * mmq_tile_tbuf<TYPE>();
#pragma unroll
                for (int i = 0; i < S::UPL; ++i)
                    store_unaligned(tt + uoff[i] - int((sl.back[t] >> (4 * i)) & 15u), sl.v[t][i]);
                W::load(w[t], tt + col * S::SBP, oct, nvalid);
            }
        } else {
#pragma unroll
            for (int t = 0; t < TN; ++t) w[t] = sl.raw[t];
        }
    };

    v4f_t acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int t = 0; t < TN; ++t) acc[a][t] = v4f_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int aoct = W::act_pos(oct) / 8;  // octet of the activation block this lane multiplies
    // PAIR: steps past the end (a k-group's last iteration, the ring's padding) multiply the
    // last step's weights by a zero activation and add nothing.
    auto compute = [&](const Slot &sl, int buf, int it) {
        if (!PAIR && it * KS + kg >= steps) return;  // wave-uniform
        typename W::Raw w[TN];
        wfields(sl, w, it);
#pragma unroll
        for (int t = 0; t < TN; ++t) W::fix(w[t]);
        const uint8_t *base = kai_mmq_lds + (buf * KS + kg) * BUF;
        const float *d8s = reinterpret_cast<const float *>(base + D8_OFF);
        const v4i_t zero = {0, 0, 0, 0};
        if constexpr (PAIR) {
            paired_step<TYPE, TN>(w, base, acc[0], col, oct, aoct, grid_lds);
            return;
        }
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            uint64_t bq[TN], bq2[TN];
            float sa[TN], fl[TN], fh[TN];
            int sl[TN], sh[TN];
#pragma unroll
            for (int t = 0; t < TN; ++t) {
                const uint64_t c = W::template codes<BATCHED>(w[t], b, oct, grid_lds);
                if constexpr (MODE != MMQ_BLOCK) {
                    const bool first = W::first_half(oct);
                    bq[t] = first ? c : 0ull;
                    bq2[t] = first ? 0ull : c;
                } else {
                    bq[t] = c;
                }
                if constexpr (MODE == MMQ_ISPLIT) {
                    sl[t] = W::iscale(w[t], 2 * b);
                    sh[t] = W::iscale(w[t], 2 * b + 1);
                }
                if constexpr (MODE == MMQ_FSPLIT) {
                    fl[t] = W::fscale(w[t], 2 * b);
                    fh[t] = W::fscale(w[t], 2 * b + 1);
                } else {
                    sa[t] = W::template scale<BATCHED>(w[t], b);
                }
            }
#pragma unroll
            for (int a = 0; a < TM; ++a) {
                const long aq = *reinterpret_cast<const long *>(base + (b * MT + 16 * a + col) * 32 + 8 * (aoct ^ ((col >> 2) & 3)));
                const float4 dv = *reinterpret_cast<const float4 *>(d8s + b * MT + 16 * a + 4 * oct);
                const float d8[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
                for (int t = 0; t < TN; ++t) {
                    const v4i_t c = __builtin_amdgcn_mfma_i32_16x16x32_i8(aq, static_cast<long>(bq[t]), zero, 0, 0, 0);
                    if constexpr (MODE == MMQ_ISPLIT) {
                        const v4i_t c2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(aq, static_cast<long>(bq2[t]), zero, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int x = __mul24(sl[t], c[i]) + __mul24(sh[t], c2[i]);
                            acc[a][t][i] = fmaf(d8[i] * sa[t], static_cast<float>(x), acc[a][t][i]);
                        }
                    } else if constexpr (MODE == MMQ_FSPLIT) {
                        const v4i_t c2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(aq, static_cast<long>(bq2[t]), zero, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float x = fmaf(fh[t], static_cast<float>(c2[i]), fl[t] * static_cast<float>(c[i]));
                            acc[a][t][i] = fmaf(d8[i], x, acc[a][t][i]);
                        }
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[a][t][i] = fmaf(d8[i] * sa[t], static_cast<float>(c[i]), acc[a][t][i]);
                    }
                }
            }
        }
        if constexpr (NT > 0) {
            const float *ta = reinterpret_cast<const float *>(base + TA_OFF);
#pragma unroll
            for (int j = 0; j < NT / 4; ++j) {
                float bt[TN];
#pragma unroll
                for (int t = 0; t < TN; ++t) bt[t] = W::template term<BATCHED>(w[t], j, oct);
#pragma unroll
                for (int a = 0; a < TM; ++a) {
                    const float at = ta[(4 * j + oct) * MT + 16 * a + col];
#pragma unroll
                    for (int t = 0; t < TN; ++t) acc[a][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(at, bt[t], acc[a][t], 0, 0, 0);
                }
            }
        }
    };

    // ---- pipeline. Per iteration: compute step it from LDS buffer it & 1, stage the
    // activation of step it+1 (loaded one iteration earlier) into the other buffer, load
    // the activation of step it+2, then the weights of step it+DEPTH. Vector loads retire
    // in order, so the wait for the activation of it+1 only covers weights that were
    // already due; the far-ahead weight loads stay in flight across the barrier. PAIR: the
    // loop runs whole turns of the ring (zero-activation steps pad the last) with no branch
    // in its body, so the compiler's waits count the ring exactly.
    aload(0);
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) wload(wr[d], d);
    astore(0);
    aload(1);
    __syncthreads();
    const int end = PAIR ? (iters + DEPTH - 1) / DEPTH * DEPTH : iters;
    for (int it0 = 0; it0 < end; it0 += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            const int it = it0 + d;
            if constexpr (!PAIR) {
                if (it >= iters) break;
            }
            compute(wr[d], it & 1, it);
            astore((it + 1) & 1);
            aload(it + 2);
            wload(wr[d], it + DEPTH);
            __syncthreads();
        }
    }

    // ---- K-split partial sums: k-groups 1.. write, k-group 0 adds in order
    if constexpr (KS > 1) {
        float *red = reinterpret_cast<float *>(kai_mmq_lds);
        constexpr int PER = TM * TN * 4;
        if (kg > 0) {
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int t = 0; t < TN; ++t)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        red[(((kg - 1) * RG + rg) * PER + (a * TN + t) * 4 + i) * WAVE + lane] = acc[a][t][i];
        }
        __syncthreads();
        if (kg == 0) {
#pragma unroll
            for (int g = 1; g < KS; ++g)
#pragma unroll
                for (int a = 0; a < TM; ++a)
#pragma unroll
                    for (int t = 0; t < TN; ++t)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            acc[a][t][i] += red[(((g - 1) * RG + rg) * PER + (a * TN + t) * 4 + i) * WAVE + lane];
        }
    }
    if (kg != 0) return;
    if constexpr (PAIR) {  // D rows 8-15 (lanes 32-63) hold the odd blocks' sums of rows 0-7
#pragma unroll
        for (int t = 0; t < TN; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[0][t][i] += __shfl_xor(acc[0][t][i], 32);
        if (oct >= 2) return;
        if (zsteps > 0 && gridDim.z > 1) {
            // K pieces: each wave writes its piece's sums to the launch's slot; the wave whose
            // arrival is the last for its 16*TN weight rows adds the pieces in K order (the
            // same sums whatever the arrival order) and stores them.
            const int Z = static_cast<int>(gridDim.z), z = static_cast<int>(blockIdx.z);
            float *part = kai_zpart[zslot];
#pragma unroll
            for (int t = 0; t < TN; ++t) {
                const int c = nrow0 + 16 * t + col;
                if (c < n)
#pragma unroll
                    for (int i = 0; i < 4; ++i) zpart_store(&part[(size_t(z) * n + c) * 8 + 4 * oct + i], acc[0][t][i]);
            }
            zpart_stores_done();
            int last = 0;
            if (lane == 0) last = zpart_arrive_last(&kai_zcount[zslot][blockIdx.x * RG + rg], Z) ? 1 : 0;
            if (!__shfl(last, 0)) return;
            __asm__ volatile("" ::: "memory");  // no load of the sums above the count
#pragma unroll
            for (int t = 0; t < TN; ++t) {
                const int c = min(nrow0 + 16 * t + col, n - 1);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float v = 0.0f;
                    for (int zz = 0; zz < Z; ++zz)
                        v += zz == z ? acc[0][t][i] : zpart_load(&part[(size_t(zz) * n + c) * 8 + 4 * oct + i]);
                    acc[0][t][i] = v;
                }
            }
        }
    }

    // ---- epilogue: x inverse[m], F32 or BF16, strided store
#pragma unroll
    for (int a = 0; a < TM; ++a) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = m0 + 16 * a + 4 * oct + i;
            if (row >= m) continue;
            const float inv = inverse[row];
#pragma unroll
            for (int t = 0; t < TN; ++t) {
                const int c = nrow0 + 16 * t + col;
                if (c < n) {
                    const int64_t idx = int64_t(row) * stride_dst + c;
                    if (dst_bf16) static_cast<uint16_t *>(dst)[idx] = float_to_bf16_bits(acc[a][t][i] * inv);
                    else static_cast<float *>(dst)[idx] = acc[a][t][i] * inv;
                }
            }
        }
    }
}

template <int TYPE, int TM, int TN, int KS, bool PAIR = false, bool EXACT = false>
static void launch_mmq_tile(const void *weight, int64_t n, int64_t k, const void *act, int64_t m,
                            const float *inverse, void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream,
                            int pieces = 1) {
    constexpr int MT = PAIR ? 8 : 16 * TM, ROWS = 16 * TN * (4 / KS);
    const int64_t row_bytes = (k / block_elems(TYPE)) * block_bytes(TYPE);
    if (n * row_bytes >= (int64_t(1) << 32)) throw Error("MMQ takes matrices below 4 GiB");
    const size_t lds = mmq_lds_bytes<TYPE, TM, TN, KS, PAIR>();
    // weight steps in flight: one. Measured on MI355X with one / two / three steps: the
    // paired tile (whose loop has no branch, so its waits count the ring exactly) on Q6_K
    // 5120x17408 at 8 rows 37.5 / 41.1 / 43.6 us, Q4_K 7168x5120 12.0 / 14.1 / 14.8 us; the
    // tiled kernel at 32-80 rows one against two steps, Q4_0 -5..-13 %, Q6_K and Q2_K
    // unchanged. Again with K pieces, one against two steps at 8 rows (whole calls): Q6_K
    // 5120x17408 30.1 / 40.8 us, 5120x6144 17.6 / 19.2 us, Q4_K 7168x5120 13.7 / 15.7 us.
    constexpr int DEPTH = 1;
    auto kernel = mmq_kernel<TYPE, TM, TN, KS, DEPTH, PAIR, EXACT>;
    static DeviceFlags lds_raised;
    raise_dynamic_lds(reinterpret_cast<const void *>(kernel), lds, lds_raised, "Cannot raise the MMQ dynamic LDS limit");
    // K pieces (paired tile only): as many as keep the whole grid resident at once (a second
    // round of workgroups would double the time), at most `pieces`; whole turns of the KS
    // k-groups per piece, no empty piece.
    const int steps = static_cast<int>((k + MMQ_STEP - 1) / MMQ_STEP);
    int zsteps = 0, z = 1, slot = 0;
    if (PAIR && pieces > 1 && steps > 1) {
        static const int per_cu = [&] {
            int blocks = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, reinterpret_cast<const void *>(kernel),
                                                             MMQ_THREADS, lds) != hipSuccess)
                throw Error("Cannot query the MMQ occupancy");
            return blocks;
        }();
        const int64_t wgs = (n + ROWS - 1) / ROWS;
        pieces = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(pieces, int64_t(per_cu) * device_cu_count() / wgs)));
        const int turns = (steps + KS - 1) / KS;  // a piece is whole turns of the KS k-groups
        zsteps = (turns + pieces - 1) / pieces * KS;
        z = (steps + zsteps - 1) / zsteps;
        if (z < 2) zsteps = 0, z = 1;
        const int64_t sets = (n + ROWS - 1) / ROWS * (4 / KS);
        if (z * n * 8 > KAI_ZCAP || sets > KAI_ZSETS) zsteps = 0, z = 1;
        else if (z > 1) slot = static_cast<int>(kai_next_zslot());
    }
    const dim3 grid(static_cast<unsigned>((n + ROWS - 1) / ROWS), static_cast<unsigned>((m + MT - 1) / MT),
                    static_cast<unsigned>(z));
    kernel<<<grid, MMQ_THREADS, lds, stream>>>(static_cast<const uint8_t *>(weight), row_bytes, static_cast<int>(n),
                                               static_cast<int>(k), act, static_cast<int>(m), inverse, dst, stride_dst,
                                               dst_bf16 ? 1 : 0, zsteps, slot);
}

// Tile choice. Activation tile MT = 16*TM rows: all rows up to 64 (weights streamed
// once), 32-row tiles from 65 to 80 rows and 64-row tiles beyond (weights re-read per tile,
// from the last-level cache when the tiles of one weight range run together). Weight rows
// per workgroup: 16*TN per wave, with KS waves splitting K. The first choice that fills the
// chip wins, trying the largest activation tile first: 1.5 workgroups per CU up to 80 rows,
// 2 beyond; LDS per workgroup stays within 80 KiB so that two fit on a CU. Measured on
// MI355X against one 80-row tile and 2 workgroups per CU: at 80 rows Q4_K 5120x17408 -17 %,
// Q6_K -11 %, IQ3_S -26 %, Q2_K 34816x5120 -11 %, Q4_K 34816x5120 -3.5 % (IQ3_S +5 %); at
// 48 rows Q4_K 5120x17408 -11 %, Q6_K 5120x6144 -7 %; at 24 rows 7168x5120 -9 %; at 64
// rows 7168x5120 +10 %.
constexpr bool mmq_allowed(int tm, int ks) { return ks == 1 || (ks == 2 && tm <= 3) || (ks == 4 && tm == 1); }

// PLANES: act is the batched path's plane of the type's layout (kai_fused_mmq_run, any m,
// k a whole number of blocks); otherwise decode Q8_1 blocks, up to 8 rows on the paired
// tile (kai_fused_mmvq), k % 256 == 0. EXACT: planes with mmq_kernel's exact weight products.
template <int TYPE, bool PLANES, bool EXACT = false>
void launch_mmq_type(const void *weight, int64_t n, int64_t k, int64_t m, const void *act, const float *inverse,
                     void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream) {
    if (!PLANES && k % MMQ_STEP) throw Error("MMQ on decode activations needs k to be a multiple of 256");
    if (!PLANES && m > 8) throw Error("MMQ on decode activations takes at most 8 rows");
    if (k % block_elems(TYPE)) throw Error("MMQ needs k to be a whole number of weight blocks");
    static constexpr int CFG[5][2] = {{2, 1}, {1, 1}, {2, 2}, {1, 2}, {1, 4}};
    // Q4_0 keeps 24 registers of wire bytes per row tile and K step: one tile per wave
    constexpr bool wide = TYPE != Q4_0;
    const int64_t want = PLANES && m <= 80 ? 3 * int64_t(device_cu_count()) / 2 : 2 * int64_t(device_cu_count());
    int tm = 1, tn = 1, ks = 4;
    bool found = false;
    for (int t = m > 80 ? 4 : m > 64 ? 2 : static_cast<int>((m + 15) / 16); t >= 1 && !found; --t) {
        for (const auto &c : CFG) {
            if (!mmq_allowed(t, c[1]) || (c[0] == 2 && !wide)) continue;
            const int64_t rows = 16 * c[0] * (4 / c[1]);
            if ((n + rows - 1) / rows * ((m + 16 * t - 1) / (16 * t)) >= want) {
                tm = t, tn = c[0], ks = c[1], found = true;
                break;
            }
        }
    }
    const int key = tm * 100 + tn * 10 + ks;
    if constexpr (!PLANES) {  // one tile of 8 activation rows, two blocks per MFMA
        // Too few row sets to fill the chip, and long rows: K pieces across workgroups, at
        // most 8 (each piece's sums cost a round trip to memory and back, which K of fewer
        // than 32 steps does not repay). Measured on MI355X at 8 rows: Q6_K 5120 x 17408
        // (68 steps) 36.2 -> 30.2 us whole calls, 5120 x 6144 (24 steps) 17.7 -> 17.3 us,
        // Q4_K 7168 x 5120 (20 steps) 13.8 -> 16.1 us.
        const int pieces = found || k < 32 * MMQ_STEP ? 1 : 8;
        switch (key) {
#define KAI_P(TN, KS) \
    case 100 + TN * 10 + KS: \
        if constexpr (TN == 1 || wide) \
            launch_mmq_tile<TYPE, 1, TN, KS, true>(weight, n, k, act, m, inverse, dst, dst_bf16, stride_dst, stream, \
                                                   pieces); \
        return;
            KAI_P(2, 1) KAI_P(1, 1) KAI_P(2, 2) KAI_P(1, 2) KAI_P(1, 4)
#undef KAI_P
            default: throw Error("MMQ tile selection failed");
        }
    } else {
        switch (key) {
#define KAI_C(TM, TN, KS) \
    case TM * 100 + TN * 10 + KS: \
        if constexpr (TN == 1 || wide) \
            launch_mmq_tile<TYPE, TM, TN, KS, false, EXACT>(weight, n, k, act, m, inverse, dst, dst_bf16, stride_dst, \
                                                           stream); \
        break;
            KAI_C(1, 2, 1) KAI_C(1, 1, 1) KAI_C(1, 2, 2) KAI_C(1, 1, 2) KAI_C(1, 1, 4)
            KAI_C(2, 2, 1) KAI_C(2, 1, 1) KAI_C(2, 2, 2) KAI_C(2, 1, 2)
            KAI_C(3, 2, 1) KAI_C(3, 1, 1) KAI_C(3, 2, 2) KAI_C(3, 1, 2)
            KAI_C(4, 2, 1) KAI_C(4, 1, 1) KAI_C(5, 2, 1) KAI_C(5, 1, 1)
#undef KAI_C
            default: throw Error("MMQ tile selection failed");
        }
    }
}

}  // namespace kai
