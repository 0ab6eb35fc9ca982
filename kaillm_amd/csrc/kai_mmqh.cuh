// Batched GEMM for more than 16 activation rows (spec-verify m = 17..80, prefill m = 512..2048)
// on fp16 MFMA with the block scales folded into the operands: kai_fused_mmq_run's product for
// Q4_K, Q4_0, Q8_0, IQ3_S and Q2_K.
//
// Arithmetic. GGML MMQ (the reference's batched path, current_ggml_direct.cu:1196-1265) sums,
// per 32-value block (16 for Q2_K), the integer dot of the activation codes q with the weight
// codes c times the activation scale dx and the weight scale dw, minus the min terms. Here both
// scales are folded into fp16 operands, x' = half(dx q) (written by the preparation) and
// w' = half(dw (c - c0)) with the codes centred by c0 (Q4_K 8, Q2_K 2; Q4_0 carries its own
// -8, Q8_0 and IQ3_S are signed), and the MFMA accumulates sum_k w'_k x'_k across all blocks
// in fp32 with no per-block step. Per superblock one more MFMA pass adds the centring back,
// c0 dw X with X = dx sum q the block's exact activation sum (high and low fp16 parts), and the
// min terms -half(dmin m) S against the stored fp16 sums S, as the reference forms them. The
// departure from the reference's arithmetic is the two fp16 roundings of w' and x' (2^-11
// relative each; centring keeps the offset c0 dw from amplifying the activation rounding):
// about 4e-4 of a row's largest output, against the 1e-3 the tests allow.
//
// Layout: D[j][i] with A = weights (32 weight rows j) and B = activations (32 activation rows
// i). v_mfma_f32_32x32x16_f16 operands: lane l holds row / column l % 32, k = 8 * (l / 32)
// .. +8; result: column l % 32, rows 8 * (r / 4) + 4 * (l / 32) + r % 4 for r = 0..15.
//
// Workgroup: 2 * GN * GM waves. The first GN * GM compute: each owns WN x WM tiles of 32 x 32,
// BN = 32 WN GN weight rows by BM = 32 WM GM activation rows; they read their operands from LDS
// and run MFMAs, and, after issuing a stage's MFMAs, convert every other stage's weights from
// raw LDS (no global memory and no MFMA result is touched, so the MFMA stream does not stall,
// and the conversion fills time the wave would spend at the barrier). The other GN * GM
// produce: they copy the activation image into LDS, load the weights' wire bytes and convert
// the other stages' weights and each superblock's min-pass factors. Waves w and w + GN GM share a SIMD
// (waves are dealt to the 4 SIMDs in turn), so each SIMD runs one of each.
//
// K runs in stages of 64 values (4 groups of 16), 4 stages a step (256 values, one superblock).
// LDS, static arrays:
//   * 2 activation stages, the codes [group 4][BM rows][32 B];
//   * 2 weight stages, the folded codes [4][BN][32 B];
//   * 2 raw weight steps (one array), each row's wire bytes of one step [BN][RS] (copied 16
//     bytes a lane, consecutive lanes along a row, so that a wave's loads touch few cache lines);
//   * the current superblock's min-pass operands, WMIN [BN][64 B] and AMIN [BM][AB].
// In the code blocks the two 16-byte halves of row r are exchanged when bit 2 of r differs from
// bit 3 (mmqh_swz): 8 or 16 lanes reading consecutive rows then hit distinct banks.
//
// Stage s, between two s_barriers:
//   producers: copy stage s + 1's activation chunks from global memory straight into LDS
//     (global_load_lds_dwordx4, no registers) and wait for them at the stage's end; at a step's
//     first stage, write step i + 1's wire bytes (loaded a step earlier) to raw LDS and load
//     step i + 2's (Q4_K, whose step is nine whole 16-byte copies: copy step i + 1's wire bytes
//     straight into raw LDS instead); convert stage s + 1's weights from raw LDS when s + 1 is
//     even; at a step's third stage, the next superblock's min-pass factors (WMIN);
//   compute: stage s's MFMAs from LDS stage s % 2, at a step's first stage also the min pass;
//     then convert stage s + 1's weights when s + 1 is odd.
// The barrier is a bare s_barrier after lgkmcnt(0) (a memory fence would wait for every load in
// flight). Every global load is issued unconditionally, clamped to the split's last stage at its
// end. Loads complete in issue order for the wait counter: the wire bytes and min-pass operands
// are loaded after the stage's copies, so the wait for the copies leaves them in flight. The
// register ring this replaced (activation loaded three stages ahead into registers, then
// written to LDS) was 5-11 % slower at 512-2048 rows: the producers' LDS writes and their waits
// were part of every stage.
// Rows past the activation image and past the matrix are clamped; their outputs are never
// stored. Split-K (grid.y > 1): each split writes its fp32 sums to scratch and
// mmqh_reduce_kernel adds them in split order; the same for the K pieces of a tail's tiles
// (MmqhTail), over the tail's rectangle of the output.
#pragma once

#include <algorithm>
#include <type_traits>

#include "kai_mmq_formats.h"

namespace kai {

typedef _Float16 v8h_t __attribute__((ext_vector_type(8)));
typedef float v16f_t __attribute__((ext_vector_type(16)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

// The activation image of one layout (layout and sizes in kai_launch.h).
struct MmqhArgs {
    const uint8_t *codes, *mins;
    int mpad;
};
// A launch whose last round of workgroups would be a small fraction of the CUs: the tiles of a
// rectangle at the output's end (activation rows [r0, r0 + rows) = [r0, m), weight rows
// [c0, c0 + cols) = [c0, n), r0 and c0 on tile bounds) run in `splits` K pieces of `stages`
// stages whose fp32 sums go to scratch [piece][rows][cols] for mmqh_reduce_kernel; the other
// `main` tiles run whole (K unsplit). No tail: main is every tile and rows is 0.
struct MmqhTail {
    int main, splits, stages, r0, rows, c0, cols;
};

__device__ __forceinline__ uint32_t h2_bits(h2_t v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h2_t bits_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }
__device__ __forceinline__ h2_t h2_splat(uint32_t half_bits) { return bits_h2((half_bits & 0xffffu) * 0x10001u); }

// Four bytes b (each 0..255) -> two words of fp16 (b - bias) * scale: fp16 1024 + b is exact,
// and so is the subtraction; the product rounds once (v_pk_mul_f16).
__device__ __forceinline__ uint2 bytes_to_h4(uint32_t w, float bias, h2_t scale) {
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u);
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u);
    const h2_t b = {static_cast<_Float16>(1024.0f + bias), static_cast<_Float16>(1024.0f + bias)};
    return make_uint2(h2_bits((bits_h2(lo) - b) * scale), h2_bits((bits_h2(hi) - b) * scale));
}
// 16 bytes -> 16 folded fp16 values (two uint4)
__device__ __forceinline__ void bytes16_to_h(uint4 w, float bias, h2_t scale, uint4 &o0, uint4 &o1) {
    const uint2 a = bytes_to_h4(w.x, bias, scale), b = bytes_to_h4(w.y, bias, scale),
                c = bytes_to_h4(w.z, bias, scale), d = bytes_to_h4(w.w, bias, scale);
    o0 = make_uint4(a.x, a.y, b.x, b.y);
    o1 = make_uint4(c.x, c.y, d.x, d.y);
}
// fp16 bits of half(a * n) for fp16 a and a small integer n (exact in fp32, one rounding)
__device__ __forceinline__ uint32_t half_times(float a, uint32_t n) { return float_to_half_bits(a * static_cast<float>(n)); }
__device__ __forceinline__ uint32_t pack2(uint32_t lo, uint32_t hi) { return (lo & 0xffffu) | (hi << 16); }

// Weight side per format. SEG: wire bytes of a row per step (256 values); RS: the raw LDS row
// stride (SEG rounded up to 16, chosen so that 16 lanes reading consecutive rows at one offset
// hit distinct banks); convert: the 32 folded values of unit (stage j4 of the step, half h) of a
// row from its raw bytes (blocks from `valid` on, past the row's end, take the scale 0); C0 and
// mins: the min-pass weight factors of a row, the 32 bytes at 32 h of its WMIN row (C0 = 0: no
// min pass).
template <int TYPE> struct MmqhW;

// Q4_0 (vecdotq.cuh:46-66; GGML MMQ's tile takes the codes minus 8): block b = 2 j4 + h of
// the step, 18 bytes: fp16 d, 16 bytes of nibbles (values 0-15 low, 16-31 high).
template <> struct MmqhW<Q4_0> {
    static constexpr int SEG = 144, RS = 144, C0 = 0;
    static __device__ void convert(const lds_u8 *seg, int j4, int h, int valid, const uint32_t *, uint4 (&o)[4]) {
        const int b = 2 * j4 + h;
        const lds_u8 *p = seg + 18 * b;
        const h2_t d = h2_splat(b < valid ? load_unaligned<uint16_t>(p) : 0u);
        const uint4 q = load_unaligned<uint4>(p + 2);
        const uint4 lo = make_uint4(q.x & 0x0f0f0f0fu, q.y & 0x0f0f0f0fu, q.z & 0x0f0f0f0fu, q.w & 0x0f0f0f0fu);
        const uint4 hi = make_uint4((q.x >> 4) & 0x0f0f0f0fu, (q.y >> 4) & 0x0f0f0f0fu, (q.z >> 4) & 0x0f0f0f0fu,
                                    (q.w >> 4) & 0x0f0f0f0fu);
        bytes16_to_h(lo, 8.0f, d, o[0], o[1]);
        bytes16_to_h(hi, 8.0f, d, o[2], o[3]);
    }
};

// Q8_0 (vecdotq.cuh:165-177): block b = 2 j4 + h, 34 bytes: fp16 d, 32 int8 codes.
template <> struct MmqhW<Q8_0> {
    static constexpr int SEG = 272, RS = 272, C0 = 0;
    static __device__ void convert(const lds_u8 *seg, int j4, int h, int valid, const uint32_t *, uint4 (&o)[4]) {
        const int b = 2 * j4 + h;
        const lds_u8 *p = seg + 34 * b;
        const h2_t d = h2_splat(b < valid ? load_unaligned<uint16_t>(p) : 0u);
        const uint4 q0 = load_unaligned<uint4>(p + 2), q1 = load_unaligned<uint4>(p + 18);
        const uint32_t f = 0x80808080u;  // int8 -> x + 128
        bytes16_to_h(make_uint4(q0.x ^ f, q0.y ^ f, q0.z ^ f, q0.w ^ f), 128.0f, d, o[0], o[1]);
        bytes16_to_h(make_uint4(q1.x ^ f, q1.y ^ f, q1.z ^ f, q1.w ^ f), 128.0f, d, o[2], o[3]);
    }
};

// IQ3_S (vecdotq.cuh:1649-1672; quants.py:1097-1125): block b = 2 j4 + h; eight grid entries
// qs[8b + i] | (qh[b] bit i) << 8 of four levels, sign bits from signs[4b..]; the code times
// the block scale (1 + 2 sc) is exact in fp16 (|code| <= 465), then times the superblock's d
// (the one rounding).
template <> struct MmqhW<IQ3_S> {
    static constexpr int SEG = 110, RS = 112, C0 = 0;
    static __device__ void convert(const lds_u8 *seg, int j4, int h, int, const uint32_t *grid, uint4 (&o)[4]) {
        const int b = 2 * j4 + h;
        const h2_t d = h2_splat(load_unaligned<uint16_t>(seg));
        const uint2 qs = load_unaligned<uint2>(seg + 2 + 8 * b);
        const uint32_t qh = seg[66 + b], signs = load_unaligned<uint32_t>(seg + 74 + 4 * b);
        const uint32_t sc = (seg[106 + b / 2] >> (4 * (b & 1))) & 15u;
        const _Float16 f = static_cast<_Float16>(static_cast<float>(1 + 2 * static_cast<int>(sc)));
        const h2_t scode = {f, f}, one = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
        uint32_t words[16];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t byte = ((i < 4 ? qs.x : qs.y) >> (8 * (i % 4))) & 0xffu;
            const uint32_t idx = byte | (((qh >> i) & 1u) << 8);
            // signed levels as int8 bytes -> + 128 -> fp16 levels (exact) -> * (1 + 2 sc) -> * d
            const uint32_t v = Unit<IQ3_S>::signed_levels(grid[idx], (signs >> (4 * i)) & 0x0fu) ^ 0x80808080u;
            const uint2 hv = bytes_to_h4(v, 128.0f, scode);
            words[2 * i] = h2_bits(bits_h2(hv.x) * d * one);
            words[2 * i + 1] = h2_bits(bits_h2(hv.y) * d * one);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) o[c] = make_uint4(words[4 * c], words[4 * c + 1], words[4 * c + 2], words[4 * c + 3]);
    }
};

// Q4_K (load_tiles_q4_K of GGML MMQ; quants.py:480-502 for the scale packing): block
// b = 2 j4 + h of the superblock, codes nibble h of qs[32 j4 ..]; dw = half(d sc_b),
// mw = half(dmin m_b). WMIN row: [-mw_0..7 | 8 dw_0..7 | 8 dw_0..7 | 0 x 8] against the
// activation's [S_0..7 | Xhi_0..7 | Xlo_0..7 | 0 x 8].
template <> struct MmqhW<Q4_K> {
    static constexpr int SEG = 144, RS = 144, C0 = 8;
    static __device__ uint32_t sc6(uint4 hdr, int b) {
        return b < 4 ? bits(hdr.y, 8 * b, 6) : bits(hdr.w, 8 * (b - 4), 4) | (bits(hdr.y, 8 * (b - 4) + 6, 2) << 4);
    }
    static __device__ uint32_t m6(uint4 hdr, int b) {
        return b < 4 ? bits(hdr.z, 8 * b, 6) : bits(hdr.w, 8 * (b - 4) + 4, 4) | (bits(hdr.z, 8 * (b - 4) + 6, 2) << 4);
    }
    static __device__ void convert(const lds_u8 *seg, int j4, int h, int, const uint32_t *, uint4 (&o)[4]) {
        const uint4 hdr = load_unaligned<uint4>(seg);
        const uint4 q0 = load_unaligned<uint4>(seg + 16 + 32 * j4), q1 = load_unaligned<uint4>(seg + 32 + 32 * j4);
        const int b = 2 * j4 + h, sh = 4 * h;
        const h2_t dw = h2_splat(half_times(half_bits_to_float(hdr.x & 0xffffu), sc6(hdr, b)));
        const uint4 n0 = make_uint4((q0.x >> sh) & 0x0f0f0f0fu, (q0.y >> sh) & 0x0f0f0f0fu,
                                    (q0.z >> sh) & 0x0f0f0f0fu, (q0.w >> sh) & 0x0f0f0f0fu);
        const uint4 n1 = make_uint4((q1.x >> sh) & 0x0f0f0f0fu, (q1.y >> sh) & 0x0f0f0f0fu,
                                    (q1.z >> sh) & 0x0f0f0f0fu, (q1.w >> sh) & 0x0f0f0f0fu);
        bytes16_to_h(n0, 8.0f, dw, o[0], o[1]);
        bytes16_to_h(n1, 8.0f, dw, o[2], o[3]);
    }
    // h = 0: [-mw_0..7 | 8 dw_0..7]; h = 1: [8 dw_0..7 | 0]
    static __device__ void mins(const lds_u8 *seg, int h, uint4 &o0, uint4 &o1) {
        const uint4 hdr = load_unaligned<uint4>(seg);
        const float d = half_bits_to_float(hdr.x & 0xffffu), dmin = half_bits_to_float(hdr.x >> 16);
        uint32_t f[8], g[8];
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            g[b] = float_to_half_bits(8.0f * half_bits_to_float(half_times(d, sc6(hdr, b))));  // exact: a power of 2
            f[b] = half_times(dmin, m6(hdr, b)) ^ 0x8000u;  // -half(dmin m): the sign bit
        }
        const uint4 fg = make_uint4(pack2(f[0], f[1]), pack2(f[2], f[3]), pack2(f[4], f[5]), pack2(f[6], f[7]));
        const uint4 gg = make_uint4(pack2(g[0], g[1]), pack2(g[2], g[3]), pack2(g[4], g[5]), pack2(g[6], g[7]));
        o0 = h ? gg : fg;
        o1 = h ? make_uint4(0, 0, 0, 0) : gg;
    }
};

// Q2_K (load_tiles_q2_K of GGML MMQ; quants.py:407-429): 32-value block kb = 2 j4 + h, codes
// (qs[32 (kb / 4) + v] >> 2 (kb % 4)) & 3; two 16-value groups g = 2 kb, 2 kb + 1 with
// dw = half(d sc_g), mw = half(dmin m_g) (scales[g]: low nibble sc, high nibble m). Centred
// codes c - 2 are -2..1, so the folded values are exact. WMIN row: [-mw_0..15 | 2 dw_0..15]
// against the activation's [Shi | Slo] and [Xhi | Xlo].
template <> struct MmqhW<Q2_K> {
    static constexpr int SEG = 84, RS = 112, C0 = 2;
    static __device__ void convert(const lds_u8 *seg, int j4, int h, int, const uint32_t *, uint4 (&o)[4]) {
        const int kb = 2 * j4 + h, sh = 2 * (kb % 4);
        const uint4 q0 = load_unaligned<uint4>(seg + 16 + 32 * (kb / 4)),
                    q1 = load_unaligned<uint4>(seg + 32 + 32 * (kb / 4));
        const uint32_t pair = load_unaligned<uint16_t>(seg + 2 * kb);  // scale bytes 2 kb, 2 kb + 1
        const float d = half_bits_to_float(load_unaligned<uint16_t>(seg + 80));
        const h2_t dw0 = h2_splat(half_times(d, pair & 15u)), dw1 = h2_splat(half_times(d, (pair >> 8) & 15u));
        const uint32_t m3 = 0x03030303u;
        bytes16_to_h(make_uint4((q0.x >> sh) & m3, (q0.y >> sh) & m3, (q0.z >> sh) & m3, (q0.w >> sh) & m3), 2.0f,
                     dw0, o[0], o[1]);
        bytes16_to_h(make_uint4((q1.x >> sh) & m3, (q1.y >> sh) & m3, (q1.z >> sh) & m3, (q1.w >> sh) & m3), 2.0f,
                     dw1, o[2], o[3]);
    }
    // h = 0: -mw of groups 0..15; h = 1: 2 dw of groups 0..15
    static __device__ void mins(const lds_u8 *seg, int h, uint4 &o0, uint4 &o1) {
        const uint4 sc = load_unaligned<uint4>(seg);
        const uint32_t dm = load_unaligned<uint32_t>(seg + 80);
        const float d = half_bits_to_float(dm & 0xffffu), dmin = half_bits_to_float(dm >> 16);
        const uint32_t w[4] = {sc.x, sc.y, sc.z, sc.w};
        uint32_t f[16];
#pragma unroll
        for (int g = 0; g < 16; ++g) {
            const uint32_t byte = (w[g / 4] >> (8 * (g % 4))) & 0xffu;
            f[g] = h ? float_to_half_bits(2.0f * half_bits_to_float(half_times(d, byte & 15u)))
                     : half_times(dmin, byte >> 4) ^ 0x8000u;
        }
        o0 = make_uint4(pack2(f[0], f[1]), pack2(f[2], f[3]), pack2(f[4], f[5]), pack2(f[6], f[7]));
        o1 = make_uint4(pack2(f[8], f[9]), pack2(f[10], f[11]), pack2(f[12], f[13]), pack2(f[14], f[15]));
    }
};

template <int TYPE> constexpr bool mmqh_type() {
    return TYPE == Q4_K || TYPE == Q4_0 || TYPE == Q8_0 || TYPE == IQ3_S || TYPE == Q2_K;
}
// Min-pass operand bytes per activation row and superblock (0: none).
template <int TYPE> constexpr int mmqh_amin_bytes() { return TYPE == Q4_K ? 64 : TYPE == Q2_K ? 128 : 0; }

// Raw LDS row stride of a tile: the format's, but 96 bytes for Q2_K's 256-row tile, whose LDS
// then fits in 160 KiB (the 112-byte rows spread a quarter-wave's 16-byte reads over every bank:
// Q2_K 34816 x 5120 at 40-120 rows 2-4 % faster than with 96)
template <int TYPE, int BM>
constexpr int mmqh_rs() {
    return TYPE == Q2_K && BM == 256 ? 96 : MmqhW<TYPE>::RS;
}
template <int TYPE, int BN, int BM>
struct MmqhLds {
    static constexpr int ASTAGE = 128 * BM, WSTAGE = 128 * BN, RAW = BN * mmqh_rs<TYPE, BM>();
    static constexpr int WMIN = MmqhW<TYPE>::C0 ? 64 * BN : 16;
    static constexpr int AMIN = mmqh_amin_bytes<TYPE>() ? mmqh_amin_bytes<TYPE>() * BM : 16;
    static constexpr int TOTAL = 2 * ASTAGE + 2 * WSTAGE + 2 * RAW + WMIN + AMIN + (TYPE == IQ3_S ? 2048 : 0);
};

// byte of 16-byte half h of row r within a group's [rows][32 B] block
__host__ __device__ constexpr int mmqh_swz(int r, int h) { return 32 * r + 16 * (h ^ (((r >> 2) ^ (r >> 3)) & 1)); }

// all but this wave's last N vector-memory loads are done (the global-to-LDS copies before them
// have written the LDS)
template <int N>
__device__ __forceinline__ void mmqh_wait_loads() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15) | ((N >> 4) << 14));
}
// this wave's LDS writes are done, then every wave of the workgroup meets (no fence)
__device__ __forceinline__ void mmqh_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

template <int TYPE, int WN, int WM, int GN, int GM>
__global__ __launch_bounds__(128 * GN * GM) __attribute__((amdgpu_waves_per_eu(2, 2))) void mmqh_kernel(
    const uint8_t *__restrict__ weight, int64_t row_bytes, int n, int k, MmqhArgs img, int m,
    const float *__restrict__ inverse, void *__restrict__ dst, int64_t stride_dst, int dst_bf16,
    float *__restrict__ partial, int tiles_n, int tiles_m, int split_stages, MmqhTail tail) {
    using W = MmqhW<TYPE>;
    constexpr int CW = GN * GM, THREADS = 64 * CW, BN = 32 * WN * GN, BM = 32 * WM * GM;
    constexpr int AB = mmqh_amin_bytes<TYPE>();
    constexpr bool SHORT = block_elems(TYPE) == 32;  // K may end inside a step
    constexpr int RS = mmqh_rs<TYPE, BM>();           // raw LDS row stride
    using L = MmqhLds<TYPE, BN, BM>;
    constexpr int UNITS = 2 * BN, UPT = UNITS / THREADS;  // weight units per producer thread and stage
    static_assert(UNITS % THREADS == 0 && (8 * BM) % THREADS == 0, "whole units and copies per producer thread");
    __shared__ __align__(16) uint8_t act_lds0[L::ASTAGE];
    __shared__ __align__(16) uint8_t act_lds1[L::ASTAGE];
    __shared__ __align__(16) uint8_t wt_lds0[L::WSTAGE];
    __shared__ __align__(16) uint8_t wt_lds1[L::WSTAGE];
    __shared__ __align__(16) uint8_t raw_lds[2 * L::RAW];  // one array: its two halves by offset
    __shared__ __align__(16) uint8_t wmin_lds[L::WMIN];
    __shared__ __align__(16) uint8_t amin_lds[L::AMIN];
    __shared__ uint32_t grid_lds[TYPE == IQ3_S ? 512 : 1];
    lds_u8 *const A0 = (lds_u8 *)act_lds0, *const A1 = (lds_u8 *)act_lds1;
    lds_u8 *const W0 = (lds_u8 *)wt_lds0, *const W1 = (lds_u8 *)wt_lds1;
    // the raw step of step i (the compiler then sees every access's array, and so that the
    // activation's global-to-LDS copies cannot touch the other buffers)
    auto raw_of = [&](int i) __attribute__((always_inline)) { return (lds_u8 *)raw_lds + (i & 1) * L::RAW; };
    lds_u8 *const wmin = (lds_u8 *)wmin_lds, *const amin = (lds_u8 *)amin_lds;

    const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
    // tile of this workgroup: each XCD (workgroups dealt round-robin over 8) gets a contiguous
    // range of the whole tiles, weight tiles fastest, so the workgroups running together on an
    // XCD share an activation tile in its L2. The whole tiles are those of the activation tiles
    // above the tail's rectangle, then those left of it; a tail workgroup takes one K piece of
    // a tile of the rectangle.
    int t = blockIdx.x, piece = blockIdx.y, piece_stages = split_stages, tile_m, tile_n;
    const bool tail_piece = t >= tail.main;  // uniform
    const int tr0 = tail.r0 / BM, tc0 = tail.c0 / BN;
    if (tail_piece) {
        const int q = t - tail.main, tt = q / tail.splits, width = tiles_n - tc0;
        tile_m = tr0 + tt / width;
        tile_n = tc0 + tt % width;
        piece = q % tail.splits;
        piece_stages = tail.stages;
    } else {
        if (tail.main % 8 == 0) t = (t % 8) * (tail.main / 8) + t / 8;
        if (tail.rows > 0 && t >= tr0 * tiles_n) {  // beside the rectangle: tc0 > 0
            const int u = t - tr0 * tiles_n;
            tile_m = tr0 + u / tc0;
            tile_n = u % tc0;
        } else {
            tile_m = t / tiles_n;
            tile_n = t % tiles_n;
        }
    }
    const int n0 = tile_n * BN, m0 = tile_m * BM;
    // K runs to the image's padding, whole steps of 256 values; the pieces are multiples of 4
    // stages, so every piece is whole steps and s % 4 is the stage's place in its step
    const int stages = (k + 255) / 256 * 4;
    const int s0 = piece * piece_stages, s1 = min(stages, s0 + piece_stages), last = s1 - 1;
    if constexpr (TYPE == IQ3_S) {
        for (int i = tid; i < 512; i += 2 * THREADS) grid_lds[i] = mmq_iq3s_grid[i];
    }
    using J0 = std::integral_constant<int, 0>;
    using J1 = std::integral_constant<int, 1>;
    using J2 = std::integral_constant<int, 2>;
    using J3 = std::integral_constant<int, 3>;

    // Weight conversion of stage s into wb from raw LDS, by either role: thread ctid of the
    // producers or of the compute waves converts the same units. The producers convert the
    // stages that start a superblock's halves (even stages, with the superblock's min-pass
    // factors at its first), the compute waves the odd stages in the time they would otherwise
    // spend at the barrier (their MFMAs are still in the pipe; the conversion reads only LDS).
    const int ctid = wave >= CW ? tid - THREADS : tid;
    // weights: unit u = h * BN + j (32 values of row j: half h of a stage)
    // first: s is a superblock's first stage (its min-pass factors go to WMIN)
    auto wstore = [&](int s, lds_u8 *wb, auto first) __attribute__((always_inline)) {
        const lds_u8 *rb = raw_of(s >> 2);
        const int valid = SHORT ? k / QK8_1 - 8 * (s >> 2) : 8;  // blocks of the step in the row
#pragma unroll
        for (int p = 0; p < UPT; ++p) {
            const int u = ctid + p * THREADS, j = u % BN, h = u / BN;
            uint4 c[4];
            W::convert(rb + j * RS, s & 3, h, valid, grid_lds, c);
            store16(wb + (2 * h) * BN * 32 + mmqh_swz(j, 0), c[0]);
            store16(wb + (2 * h) * BN * 32 + mmqh_swz(j, 1), c[1]);
            store16(wb + (2 * h + 1) * BN * 32 + mmqh_swz(j, 0), c[2]);
            store16(wb + (2 * h + 1) * BN * 32 + mmqh_swz(j, 1), c[3]);
            if constexpr (W::C0 != 0) {
                if constexpr (decltype(first)::value) {
                    uint4 o0, o1;
                    W::mins(rb + j * RS, h, o0, o1);
                    store16(wmin + j * 64 + 32 * h, o0);
                    store16(wmin + j * 64 + 32 * h + 16, o1);
                }
            }
        }
    };
    // the min-pass factors of stage s's superblock (s its first stage) into WMIN
    auto wmins = [&](int s) __attribute__((always_inline)) {
        if constexpr (W::C0 != 0) {
            const lds_u8 *rb = raw_of(s >> 2);
#pragma unroll
            for (int p = 0; p < UPT; ++p) {
                const int u = ctid + p * THREADS, j = u % BN, h = u / BN;
                uint4 o0, o1;
                W::mins(rb + j * RS, h, o0, o1);
                store16(wmin + j * 64 + 32 * h, o0);
                store16(wmin + j * 64 + 32 * h + 16, o1);
            }
        }
    };
    if (wave >= CW) {
        // ================= producer waves
        const int ptid = tid - THREADS;
        // wire bytes: copy c of a step is row c / CPR, 16 bytes at 16 (c % CPR) of the row's step
        // (the last copy ends at the step's last byte, overlapping the one before when the step
        // is not a multiple of 16 bytes, so that no copy reads past the row's step)
        constexpr int CPR = (W::SEG + 15) / 16, RAWC = BN * CPR, RPT = (RAWC + THREADS - 1) / THREADS;
        const uint8_t *raw_row[RPT];
        int raw_at[RPT], raw_piece[RPT];
#pragma unroll
        for (int p = 0; p < RPT; ++p) {
            const int c = min(ptid + p * THREADS, RAWC - 1), r = c / CPR;
            raw_row[p] = weight + int64_t(min(n0 + r, n - 1)) * row_bytes;
            raw_at[p] = r * RS;
            raw_piece[p] = 16 * (c % CPR);
        }
        const int nblocks = k / QK8_1;
        uint4 rawv[RPT];
        int raw_off[RPT];
        auto rload = [&](int step) __attribute__((always_inline)) {
            // bytes of the row in this step (short formats: the last step may hold fewer blocks)
            const int have = SHORT ? min(W::SEG, static_cast<int>(row_bytes - int64_t(step) * W::SEG)) : W::SEG;
#pragma unroll
            for (int p = 0; p < RPT; ++p) {
                raw_off[p] = min(raw_piece[p], have - 16);
                rawv[p] = load_unaligned<uint4>(raw_row[p] + int64_t(step) * W::SEG + raw_off[p]);
            }
        };
        auto rstore = [&](lds_u8 *rb) __attribute__((always_inline)) {
#pragma unroll
            for (int p = 0; p < RPT; ++p)
                if (RAWC % THREADS == 0 || ptid + p * THREADS < RAWC) store_unaligned(rb + raw_at[p] + raw_off[p], rawv[p]);
        };
        // RAW_DMA (whole 256-value steps whose wire bytes are a whole number of 16-byte copies:
        // Q4_K): copy c of a step lands at 16 c of the raw step, so a wave's copies fill 1 KiB in
        // lane order and go straight from global memory to LDS, as the activation does (below).
        // The last copy index may end inside the waves; RAWC is a whole number of waves, so a wave
        // issues all of a copy index or none of it.
        constexpr bool RAW_DMA = !SHORT && W::SEG == RS && W::SEG % 16 == 0;
        static_assert(!RAW_DMA || RAWC % WAVE == 0, "whole waves of wire-byte copies");
        const int pwave = __builtin_amdgcn_readfirstlane(ptid / WAVE);
        const bool raw_all = RAWC % THREADS == 0 || (RPT - 1) * THREADS + WAVE * pwave < RAWC;  // uniform
        auto rdma = [&](int step, lds_u8 *rb) __attribute__((always_inline)) {
#pragma unroll
            for (int p = 0; p < RPT; ++p) {
                if (p < RPT - 1 || raw_all) {
                    const uint32_t la = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(rb + 16 * (p * THREADS + WAVE * pwave)));
                    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
                                 :: "s"(la), "v"(raw_row[p] + int64_t(step) * W::SEG + raw_piece[p]) : "memory", "m0");
                }
            }
        };
        // all but the wire-byte copies just issued are done (their count is the wave's)
        auto wait_but_raw = [&]() __attribute__((always_inline)) {
            if (raw_all) mmqh_wait_loads<RPT>();
            else mmqh_wait_loads<RPT - 1>();
        };
        // activation: per stage, the image's 16-byte chunks (4 groups x BM rows x 32 bytes; chunk
        // w of a group holds row w / 2, half (w % 2) swizzled), copied to LDS a stage ahead; per
        // superblock its min-pass operands (BM x AB bytes). Rows past the image read its last row.
        const int rows_here = min(BM, img.mpad - m0);
        constexpr int MIN_CH = AB * BM / 16;
        constexpr int CODE_PW = 8 * BM / THREADS, MIN_PW = (MIN_CH + THREADS - 1) / THREADS;
        int code_src[CODE_PW], min_src[MIN_PW > 0 ? MIN_PW : 1];
#pragma unroll
        for (int p = 0; p < CODE_PW; ++p) {
            const int c = ptid + p * THREADS, g = c / (2 * BM), w = c % (2 * BM), r = w >> 1;
            const int hsrc = (w & 1) ^ (((r >> 2) ^ (r >> 3)) & 1);
            code_src[p] = g * img.mpad * 32 + 32 * min(r, rows_here - 1) + 16 * hsrc;
        }
#pragma unroll
        for (int p = 0; p < MIN_PW; ++p) min_src[p] = 16 * min(ptid + p * THREADS, rows_here * AB / 16 - 1);
        // stage s's chunks straight into LDS (global_load_lds_dwordx4: a wave's 64 lanes fill
        // 1 KiB in lane order at the wave-uniform LDS address in M0; no registers, no LDS
        // write). Written as an asm statement: the compiler would otherwise make every later
        // LDS read of this wave that it cannot tell apart from the copy wait for it. Nothing
        // else in the kernel uses M0. The compiler does not count these loads, so its own waits
        // for the loads issued before them wait longer, never shorter; the stage's waits for
        // the copies are explicit (mmqh_wait_loads).
        auto adma = [&](int s, lds_u8 *ab) __attribute__((always_inline)) {
            const uint8_t *cb = img.codes + (int64_t(4 * s) * img.mpad + m0) * 32;
#pragma unroll
            for (int p = 0; p < CODE_PW; ++p) {
                const uint32_t la = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(ab + 16 * (p * THREADS + WAVE * pwave)));
                asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
                             :: "s"(la), "v"(cb + code_src[p]) : "memory", "m0");
            }
        };
        uint4 mv[MIN_PW > 0 ? MIN_PW : 1];
        auto mload = [&](int s) __attribute__((always_inline)) {  // s: a superblock's first stage
            const uint8_t *mb = img.mins + (int64_t(s / 4) * img.mpad + m0) * AB;
#pragma unroll
            for (int p = 0; p < MIN_PW; ++p) mv[p] = *reinterpret_cast<const uint4 *>(mb + min_src[p]);
        };
        auto mstore = [&]() __attribute__((always_inline)) {
#pragma unroll
            for (int p = 0; p < MIN_PW; ++p)
                if (MIN_CH % THREADS == 0 || ptid + p * THREADS < MIN_CH) store16(amin + 16 * (ptid + p * THREADS), mv[p]);
        };
        // stage J of a step i (s = 4 i + J): copy stage s + 1's activation into LDS first; the
        // min-pass operands of a superblock are loaded two stages before its first stage (J = 1)
        // and written a stage before it (J = 3); at J = 0 the wire bytes of step i + 1 (loaded
        // at step i - 1) go to raw LDS and those of step i + 2 are loaded (RAW_DMA: step i + 1's
        // are copied into its raw buffer, whose last reader, the conversion of step i - 1's last
        // stage, ran two stages before; their first reader, the min-pass factors at J = 2, comes
        // after J = 1's wait). Loads complete in issue order for the wait counter, so the wait
        // for the stage's copies before the barrier leaves the loads issued after them in flight.
        auto pstep = [&](int s, auto jtag, lds_u8 *anext, lds_u8 *wnext) __attribute__((always_inline)) {
            constexpr int J = decltype(jtag)::value;
            const int sw = min(s + 1, last), step = s >> 2;
            // the register stores first: their waits then cover only the copies of earlier stages
            if constexpr (!RAW_DMA && J == 0) rstore(raw_of(step + 1));
            if constexpr (MIN_PW > 0 && J == 3) mstore();
            __builtin_amdgcn_sched_barrier(0);
            adma(sw, anext);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (!RAW_DMA && J == 0) rload(min(step + 2, last >> 2));
            if constexpr (RAW_DMA && J == 0) rdma(min(step + 1, last >> 2), raw_of(step + 1));
            if constexpr (MIN_PW > 0 && J == 1) mload(min(s + 3, last) / 4 * 4);
            // the next superblock's min-pass factors a stage before its first conversion (the
            // compute waves read WMIN at each superblock's first stage only)
            if constexpr (J == 2) wmins(min(s + 2, last) / 4 * 4);
            if constexpr (J == 1 || J == 3) wstore(sw, wnext, std::false_type{});
            (void)wnext;
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (J == 0 && RAW_DMA) wait_but_raw();
            else mmqh_wait_loads<(J == 0 ? RPT : 0) + (J == 1 ? MIN_PW : 0)>();
            mmqh_barrier();
        };
        if constexpr (TYPE == IQ3_S) mmqh_barrier();  // the grid, before the first conversion
        if (s0 < s1) {
            if constexpr (RAW_DMA) {
                rdma(s0 >> 2, raw_of(s0 >> 2));
                if constexpr (MIN_PW > 0) mload(s0);
                adma(s0, A0);
                if constexpr (MIN_PW > 0) mstore();
                __builtin_amdgcn_sched_barrier(0);
                mmqh_wait_loads<0>();
            } else {
                rload(s0 >> 2);
                rstore(raw_of(s0 >> 2));
                if constexpr (MIN_PW > 0) mload(s0);
                adma(s0, A0);
                __builtin_amdgcn_sched_barrier(0);
                rload(min((s0 >> 2) + 1, last >> 2));
                if constexpr (MIN_PW > 0) mstore();
                __builtin_amdgcn_sched_barrier(0);
                mmqh_wait_loads<RPT>();
            }
            mmqh_barrier();  // the wire bytes of the first step, its activation and min operands
            wstore(s0, W0, std::true_type{});
            mmqh_barrier();
            for (int s = s0; s < s1; s += 4) {
                pstep(s, J0{}, A1, W1);
                pstep(s + 1, J1{}, A0, W0);
                pstep(s + 2, J2{}, A1, W1);
                pstep(s + 3, J3{}, A0, W0);
            }
        }
        return;
    }

    // ================= compute waves
    const int wn = wave % GN, wm = wave / GN;
    const int col = lane & 31, kh = lane >> 5;
    v16f_t acc[WN][WM];
#pragma unroll
    for (int a = 0; a < WN; ++a)
#pragma unroll
        for (int b = 0; b < WM; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;

    // Lane (col, kh) reads operand row col of each tile, k half kh. The stage's operands are read
    // up front, group by group, so that the first group's products start while the rest arrive;
    // within a group the tiles' MFMAs are independent.
    const int wrow0 = wn * 32 * WN, arow0 = wm * 32 * WM;
    const int a_off = mmqh_swz(wrow0 + col, kh), b_off = mmqh_swz(arow0 + col, kh);
    auto compute = [&](const lds_u8 *ab, const lds_u8 *wb, auto first, int sconv, lds_u8 *wconv)
                       __attribute__((always_inline)) {
        v8h_t a[4][WN], b[4][WM];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
#pragma unroll
            for (int tn = 0; tn < WN; ++tn) a[g][tn] = load_unaligned<v8h_t>(wb + g * BN * 32 + 32 * 32 * tn + a_off);
#pragma unroll
            for (int tm = 0; tm < WM; ++tm) b[g][tm] = load_unaligned<v8h_t>(ab + g * BM * 32 + 32 * 32 * tm + b_off);
        }
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int tn = 0; tn < WN; ++tn)
#pragma unroll
                for (int tm = 0; tm < WM; ++tm)
                    acc[tn][tm] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[g][tn], b[g][tm], acc[tn][tm], 0, 0, 0);
        if constexpr (W::C0 != 0) {
          if constexpr (decltype(first)::value) {
            // the superblock's min pass: 64 bytes of weight factors against AB bytes of activation
            // sums per row, 32 bytes per MFMA (lane kh takes the 16 at 16 kh). Q4_K:
            // (-mw | 8 dw) x (S | Xhi), (8 dw | 0) x (Xlo | 0); Q2_K: -mw x Shi, -mw x Slo,
            // 2 dw x Xhi, 2 dw x Xlo
            constexpr int PASSES = AB / 32;
            v8h_t am[2][WN], bm[PASSES][WM];
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
                for (int tn = 0; tn < WN; ++tn)
                    am[q][tn] = load_unaligned<v8h_t>(wmin + (wrow0 + 32 * tn + col) * 64 + 32 * q + 16 * kh);
#pragma unroll
            for (int q = 0; q < PASSES; ++q)
#pragma unroll
                for (int tm = 0; tm < WM; ++tm)
                    bm[q][tm] = load_unaligned<v8h_t>(amin + (arow0 + 32 * tm + col) * AB + 32 * q + 16 * kh);
#pragma unroll
            for (int q = 0; q < PASSES; ++q)
#pragma unroll
                for (int tn = 0; tn < WN; ++tn)
#pragma unroll
                    for (int tm = 0; tm < WM; ++tm)
                        acc[tn][tm] = __builtin_amdgcn_mfma_f32_32x32x16_f16(am[PASSES == 2 ? q : q / 2][tn],
                                                                             bm[q][tm], acc[tn][tm], 0, 0, 0);
          }
        }
        if (wconv) wstore(sconv, wconv, std::false_type{});
        mmqh_barrier();
    };
    if constexpr (TYPE == IQ3_S) mmqh_barrier();
    if (s0 < s1) {
        mmqh_barrier();  // the producers' wire bytes of the first step
        mmqh_barrier();  // and its first stage
        for (int s = s0; s < s1; s += 4) {
            compute(A0, W0, std::true_type{}, min(s + 1, last), W1);
            compute(A1, W1, std::false_type{}, 0, nullptr);
            compute(A0, W0, std::false_type{}, min(s + 3, last), W1);
            compute(A1, W1, std::false_type{}, 0, nullptr);
        }
    }

    // ---- epilogue: lane (col, kh) holds activation row i = col of each activation tile and
    // weight rows 8 q + 4 kh + (0..3) of each weight tile; one branch per kind of output
    // A lane's four consecutive weight rows of one activation row go out as one 16-byte (f32) or
    // 8-byte (bf16) store where the row is aligned for it: a quarter of the store requests of
    // element stores (Q4_K 34816 x 5120 at 2048 rows 1235 -> 1063 us, 5120 x 17408 818 -> 655 us).
    auto store_all = [&](auto kind_tag) __attribute__((always_inline)) {
        constexpr int KIND = decltype(kind_tag)::value;  // 0 partial sums, 1 f32, 2 bf16
        // partial sums: [split][m][n], or a tail piece's [piece][tail rows][tail cols]
        const int64_t pstride = tail_piece ? tail.cols : n;
        float *const pbase = tail_piece ? partial + (int64_t(piece) * tail.rows - tail.r0) * pstride - tail.c0
                                        : partial + int64_t(piece) * m * n;
        const bool vec = KIND == 0 ? pstride % 4 == 0
                                   : stride_dst % 4 == 0 && (reinterpret_cast<uintptr_t>(dst) & (KIND == 1 ? 15 : 7)) == 0;
#pragma unroll
        for (int tm = 0; tm < WM; ++tm) {
            const int i = m0 + arow0 + 32 * tm + col;
            if (i >= m) continue;
            const float inv = KIND == 0 ? 1.0f : inverse[i];
            float *rowf = KIND == 0 ? pbase + int64_t(i) * pstride
                                    : static_cast<float *>(dst) + int64_t(i) * stride_dst;
            uint16_t *rowh = static_cast<uint16_t *>(dst) + int64_t(i) * stride_dst;
#pragma unroll
            for (int tn = 0; tn < WN; ++tn) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int j0 = n0 + wrow0 + 32 * tn + 8 * q + 4 * kh;
                    if (vec && j0 + 3 < n) {
                        const float v0 = acc[tn][tm][4 * q] * inv, v1 = acc[tn][tm][4 * q + 1] * inv,
                                    v2 = acc[tn][tm][4 * q + 2] * inv, v3 = acc[tn][tm][4 * q + 3] * inv;
                        if constexpr (KIND == 2)
                            *reinterpret_cast<uint2 *>(rowh + j0) =
                                make_uint2(float_to_bf16_bits(v0) | (uint32_t(float_to_bf16_bits(v1)) << 16),
                                           float_to_bf16_bits(v2) | (uint32_t(float_to_bf16_bits(v3)) << 16));
                        else
                            *reinterpret_cast<float4 *>(rowf + j0) = make_float4(v0, v1, v2, v3);
                        continue;
                    }
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if (j0 + e < n) {
                            const float v = acc[tn][tm][4 * q + e] * inv;
                            if constexpr (KIND == 2) rowh[j0 + e] = float_to_bf16_bits(v);
                            else rowf[j0 + e] = v;
                        }
                    }
                }
            }
        }
    };
    if (tail_piece || gridDim.y > 1) store_all(std::integral_constant<int, 0>{});
    else if (dst_bf16) store_all(std::integral_constant<int, 2>{});
    else store_all(std::integral_constant<int, 1>{});
}

// Split-K sums: out[i][j] = inverse[i] * sum over splits in order.
__global__ __launch_bounds__(256) void mmqh_reduce_kernel(const float *__restrict__ partial, int splits, int m, int n,
                                                          const float *__restrict__ inverse, void *__restrict__ dst,
                                                          int64_t stride_dst, int dst_bf16);

// Tile configurations: (WN, WM, GN, GM).
struct MmqhConfig {
    int wn, wm, gn, gm;
    int bn() const { return 32 * wn * gn; }
    int bm() const { return 32 * wm * gm; }
};

// Launch plan of an m-row product. It depends only on the type and shape (sized for the 256
// CUs of an MI355X), so the scratch query and the launch agree on any device.
struct MmqhPlan {
    MmqhConfig cfg;
    int tiles_n = 0, tiles_m = 0, splits = 1, split_stages = 0;
    MmqhTail tail = {};
    bool has_tail() const { return tail.main < tiles_n * tiles_m; }
};
// Scratch a tail's K pieces may use: written once and read once, 32 MiB cost ~13 us at HBM
// rate, against the tens of microseconds of a last round cut to an eighth or a half.
constexpr size_t MMQH_TAIL_BYTES = size_t(32) << 20;
constexpr int MMQH_CUS = 256;
template <int TYPE, int WN, int WM, int GN, int GM>
constexpr bool mmqh_fits() {
    return MmqhLds<TYPE, 32 * WN * GN, 32 * WM * GM>::TOTAL <= 160 * 1024;
}
// One workgroup per CU: its 8 waves fill the 4 SIMDs two each (amdgpu_waves_per_eu(2, 2)).
template <int TYPE, int WN, int WM, int GN, int GM>
constexpr int mmqh_per_cu() {
    static_assert(GN * GM == 4, "one compute and one producer wave per SIMD");
    static_assert(MmqhLds<TYPE, 32 * WN * GN, 32 * WM * GM>::TOTAL <= 160 * 1024, "LDS");
    return 1;
}
// Each configuration's time for the product, in units of one CU's time for one 32 x 32 tile of
// the whole K: rounds of resident workgroups times the workgroup's tiles per split, plus the
// split-K sums (written and read once); the fastest wins.
template <int TYPE, int WN, int WM, int GN, int GM>
inline void mmqh_consider(MmqhPlan &best, double &best_t, int64_t n, int64_t k, int64_t m) {
    constexpr int BN = 32 * WN * GN, BM = 32 * WM * GM, PER = mmqh_per_cu<TYPE, WN, WM, GN, GM>();
    const int stages = static_cast<int>((k + 255) / 256 * 4), quantum = 4;  // whole steps
    const int64_t tn = (n + BN - 1) / BN, tm = (m + BM - 1) / BM, slots = int64_t(MMQH_CUS) * PER;
    const double tile_time = double(WN * GN * WM * GM) * PER;  // per workgroup, at PER per CU
    for (int want = 1; want <= 8; ++want) {
        const int chunk = ((stages + want - 1) / want + quantum - 1) / quantum * quantum;
        const int splits = (stages + chunk - 1) / chunk;
        if (splits != want || (splits > 1 && chunk < 16)) continue;
        const int64_t wgs = tn * tm * splits, rounds = (wgs + slots - 1) / slots;
        // the sums: 8 bytes per output and split at ~5 TB/s, against ~4 TOPS per CU for a tile
        const double reduce = splits > 1 ? double(splits) * double(m) * double(n) / (320.0 * double(k)) : 0.0;
        const double t = double(rounds) * tile_time / splits + reduce;
        if (t < best_t) {
            best_t = t;
            best.cfg = {WN, WM, GN, GM};
            best.tiles_n = static_cast<int>(tn);
            best.tiles_m = static_cast<int>(tm);
            best.splits = splits;
            best.split_stages = chunk;
        }
    }
}
// A plan with more tiles than CUs whose last round of workgroups would hold at most half the
// CUs' worth of tiles: the last tiles (inside the last activation tile) run in K pieces, as
// many as fill that round's CUs, at most 8 and at most MMQH_TAIL_BYTES of sums, the others
// whole. Taken where the cost model of mmqh_consider puts it ahead of the chosen plan (an
// unsplit one's last round, or a K split's extra rounds). Measured on MI355X, Q4_K
// 34816 x 5120: at 512 rows (544 tiles of 256 x 128, a third round of 32, now 7 pieces)
// 303 -> 251 us; at 2048 rows (a ninth round of 128, now 2 pieces) 922 -> 915 us (a half-empty
// round already runs faster per tile); IQ3_S at 2048 rows 1048 -> 1018 us; in place of a
// three-way K split (272 tiles: 256 whole, 16 in 7 pieces) at 17 / 80 / 97 / 256 rows
// 95 / 103 / 112 / 185 -> 81 / 80 / 92 / 144 us; Q4_K 5120 x 17408 at 2048 rows, in place of a
// four-way K split (320 tiles: 256 whole, the last 32 weight tiles of the last 2 activation
// tiles in 4 pieces) 551 -> 498 us.
inline void mmqh_tail(MmqhPlan &p, double best_t, int64_t n, int64_t k, int64_t m) {
    const int tiles = p.tiles_n * p.tiles_m, slots = MMQH_CUS;
    p.tail = {tiles, 1, 0, 0, 0, 0, 0};
    const int rem = tiles % slots, full = tiles - rem;
    if (full == 0 || rem == 0 || 2 * rem > slots) return;
    // the rectangle: the fewest activation tiles whose last `width` weight tiles make `rem`
    int height = 1;
    while (height <= p.tiles_m && (rem % height || rem / height > p.tiles_n)) ++height;
    if (height > p.tiles_m) return;
    const int64_t r0 = int64_t(p.tiles_m - height) * p.cfg.bm(), c0 = int64_t(p.tiles_n - rem / height) * p.cfg.bn();
    const int64_t rows = m - r0, cols = n - c0;
    const int stages = static_cast<int>((k + 255) / 256 * 4);
    int64_t pieces = std::min<int64_t>({slots / rem, 8, stages / 4,
                                        static_cast<int64_t>(MMQH_TAIL_BYTES / size_t(rows * cols * 4))});
    if (pieces < 2) return;
    const int chunk = static_cast<int>(((stages + pieces - 1) / pieces + 3) / 4 * 4);
    pieces = (stages + chunk - 1) / chunk;
    if (pieces < 2) return;
    // mmqh_consider's units: whole rounds of whole tiles, the pieces' round, their sums
    const double tile_time = double(p.cfg.wn * p.cfg.gn * p.cfg.wm * p.cfg.gm);
    const double t = double(full / slots) * tile_time + tile_time * chunk / stages +
                     double(pieces) * double(rows) * double(cols) / (320.0 * double(k));
    if (t >= best_t) return;
    p.splits = 1;
    p.split_stages = stages;
    p.tail = {full, static_cast<int>(pieces), chunk, static_cast<int>(r0), static_cast<int>(rows), static_cast<int>(c0),
              static_cast<int>(cols)};
}
template <int TYPE>
inline MmqhPlan mmqh_plan(int64_t n, int64_t k, int64_t m) {
    MmqhPlan best;
    double t = 1e300;
    if (m <= 96) {
        mmqh_consider<TYPE, 1, 3, 4, 1>(best, t, n, k, m);
    } else {
        // 256-row tiles from 129 rows: one partly filled 256-row tile takes less time than two
        // 128-row tiles (MI355X, 160 / 240 rows: Q4_K 34816 x 5120 158 / 161 -> 140 / 143 us,
        // IQ3_S 223 -> 166 us, Q4_K 5120 x 17408 94 / 104 -> 84 / 97 us)
        if constexpr (mmqh_fits<TYPE, 2, 4, 2, 2>()) {
            if (m > 128) mmqh_consider<TYPE, 2, 4, 2, 2>(best, t, n, k, m);
            else mmqh_consider<TYPE, 2, 2, 2, 2>(best, t, n, k, m);
        } else {
            mmqh_consider<TYPE, 2, 2, 2, 2>(best, t, n, k, m);
        }
    }
    mmqh_tail(best, t, n, k, m);
    return best;
}
inline size_t mmqh_partial_bytes(const MmqhPlan &p, int64_t m, int64_t n) {
    if (p.splits > 1) return size_t(p.splits) * size_t(m) * size_t(n) * sizeof(float);
    if (p.has_tail()) return size_t(p.tail.splits) * size_t(p.tail.rows) * size_t(p.tail.cols) * sizeof(float);
    return 0;
}

template <int TYPE, int WN, int WM, int GN, int GM>
void launch_mmqh_cfg(const void *weight, int64_t n, int64_t k, int64_t m, const MmqhArgs &img, const float *inverse,
                     float *partial, const MmqhPlan &p, void *dst, bool dst_bf16, int64_t stride_dst,
                     hipStream_t stream) {
    constexpr int BN = 32 * WN * GN, BM = 32 * WM * GM;
    static_assert(MmqhLds<TYPE, BN, BM>::TOTAL <= 160 * 1024, "mmqh LDS");  // static arrays
    const int64_t row_bytes = (k / block_elems(TYPE)) * block_bytes(TYPE);
    const int tiles = p.tiles_n * p.tiles_m;
    const int wgs = p.has_tail() ? p.tail.main + (tiles - p.tail.main) * p.tail.splits : tiles;
    const dim3 grid(static_cast<unsigned>(wgs), static_cast<unsigned>(p.splits));
    mmqh_kernel<TYPE, WN, WM, GN, GM><<<grid, 128 * GN * GM, 0, stream>>>(
        static_cast<const uint8_t *>(weight), row_bytes, static_cast<int>(n), static_cast<int>(k), img,
        static_cast<int>(m), inverse, dst, stride_dst, dst_bf16 ? 1 : 0, partial, p.tiles_n, p.tiles_m,
        p.split_stages, p.tail);
    if (p.splits > 1) {
        mmqh_reduce_kernel<<<static_cast<unsigned>((m * n + 1023) / 1024), 256, 0, stream>>>(
            partial, p.splits, static_cast<int>(m), static_cast<int>(n), inverse, dst, stride_dst, dst_bf16 ? 1 : 0);
    } else if (p.has_tail()) {  // the tail tiles' rectangle of the output
        const MmqhTail &t = p.tail;
        const int64_t at = int64_t(t.r0) * stride_dst + t.c0;
        void *tail_dst = dst_bf16 ? static_cast<void *>(static_cast<uint16_t *>(dst) + at)
                                  : static_cast<void *>(static_cast<float *>(dst) + at);
        mmqh_reduce_kernel<<<static_cast<unsigned>((int64_t(t.rows) * t.cols + 1023) / 1024), 256, 0, stream>>>(
            partial, t.splits, t.rows, t.cols, inverse + t.r0, tail_dst, stride_dst, dst_bf16 ? 1 : 0);
    }
}

template <int TYPE>
void launch_mmqh(const void *weight, int64_t n, int64_t k, int64_t m, const MmqhArgs &img, const float *inverse,
                 float *partial, size_t partial_bytes, void *dst, bool dst_bf16, int64_t stride_dst,
                 hipStream_t stream) {
    static_assert(mmqh_type<TYPE>(), "fp16 GEMM format");
    const MmqhPlan p = mmqh_plan<TYPE>(n, k, m);
    if (mmqh_partial_bytes(p, m, n) > partial_bytes || ((p.splits > 1 || p.has_tail()) && !partial))
        throw Error("Scratch too small for the fp16 GEMM's split-K sums");
    if (n * ((k / block_elems(TYPE)) * block_bytes(TYPE)) >= (int64_t(1) << 40)) throw Error("Matrix too large");
    // the short formats' wire-byte copies are 16 bytes, within the row's last step: one block at least
    if (k % block_elems(TYPE) || (k / block_elems(TYPE)) * block_bytes(TYPE) < 16) throw Error("Invalid fp16 GEMM shape");
    const MmqhConfig &c = p.cfg;
#define KAI_H(WN, WM, GN, GM) \
    if (c.wn == WN && c.wm == WM && c.gn == GN && c.gm == GM) \
        return launch_mmqh_cfg<TYPE, WN, WM, GN, GM>(weight, n, k, m, img, inverse, partial, p, dst, dst_bf16, \
                                                     stride_dst, stream);
    KAI_H(2, 2, 2, 2) KAI_H(1, 3, 4, 1)
    if constexpr (mmqh_fits<TYPE, 2, 4, 2, 2>()) {
        KAI_H(2, 4, 2, 2)
    }
#undef KAI_H
    throw Error("fp16 GEMM configuration");
}

}  // namespace kai
