// Per-format "units" for the v_dot4 GEMV: the slice of one wire block that one
// lane decodes in one step, the matching Q8_1 activation blocks, and the scaled
// integer dot product of the two.
//
// A unit is about 32 bytes of codes (plus the block header it needs), so that
// scale unpacking and the fp32 epilogue are amortised over 32-128 values, and it
// always covers whole Q8_1 activation blocks. Units per block divide 8, so with
// lane groups of 8 per row a lane's position inside a block is fixed for the whole
// kernel and every index below is loop-invariant.
//
// Three steps per unit: load_w (wire bytes -> registers), prep (decode codes and
// scales once per weight unit, branch-free), dot (per activation row: exact int8
// dot products with v_dot4_i32_i8, then fp32 scaling). Arithmetic per format
// follows the reference's block dot products vec_dot_*_q8_1 (in-tree text
// vllm_gguf_plugin/csrc/gguf/vecdotq.cuh, cited per format); only the order of
// the fp32 scale multiplications differs. Activation sums over 16-value halves
// (exact integers) come precomputed with the activation view.
#pragma once

#include "kai_device.h"

namespace kai {

// One activation row in LDS: the Q8_1 blocks byte for byte (36 bytes each, 4-byte
// aligned) and, per block, the exact sums of its codes over values 0..15 and 16..31
// packed as two int16.
struct ActLds {
    const uint8_t *row;
    const uint32_t *sums;
    __device__ uint4 q16(int b, int first) const { return load_unaligned<uint4>(row + 36 * b + 4 + first); }
    __device__ uint32_t ds(int b) const { return *reinterpret_cast<const uint32_t *>(row + 36 * b); }
    __device__ float d(int b) const { return half_bits_to_float(ds(b) & 0xffffu); }
    __device__ int sum_lo(int b) const { return static_cast<int16_t>(sums[b] & 0xffffu); }
    __device__ int sum_hi(int b) const { return static_cast<int16_t>(sums[b] >> 16); }
    __device__ int sum(int b) const { return sum_lo(b) + sum_hi(b); }
};

__device__ __forceinline__ int dot16(const uint4 w, const uint4 u, int c = 0) {
    return dot4(w.w, u.w, dot4(w.z, u.z, dot4(w.y, u.y, dot4(w.x, u.x, c))));
}
__device__ __forceinline__ uint4 and4(uint4 v, uint32_t m) { return make_uint4(v.x & m, v.y & m, v.z & m, v.w & m); }
__device__ __forceinline__ uint4 shr4(uint4 v, int s) { return make_uint4(v.x >> s, v.y >> s, v.z >> s, v.w >> s); }
__device__ __forceinline__ float i2f(int v) { return static_cast<float>(v); }

// A full Q8_1 block of codes (32 values) as two 16-value halves.
struct Q32 {
    uint4 lo, hi;
};
template <class Y>
__device__ __forceinline__ Q32 act32(const Y &y, int b) { return {y.q16(b, 0), y.q16(b, 16)}; }

template <int TYPE> struct Unit;

// Q8_0: 1 unit per 34-byte block. Result d_w * d8 * sum(q_w q8). vecdotq.cuh:165-177,852-867.
template <> struct Unit<Q8_0> {
    static constexpr int PER_BLOCK = 1;
    struct W { uint4 q0, q1; uint32_t d; };
    struct P { uint4 q0, q1; float d; };
    struct A { Q32 u; float d8; };
    __device__ explicit Unit(int) {}
    __device__ void load_w(W &w, const uint8_t *blk) const {
        w.d = load_unaligned<uint16_t>(blk);
        w.q0 = load_unaligned<uint4>(blk + 2);
        w.q1 = load_unaligned<uint4>(blk + 18);
    }
    __device__ P prep(const W &w) const { return {w.q0, w.q1, half_bits_to_float(w.d)}; }
    template <class Y> __device__ void load_a(A &a, const Y &y, int blk) const {
        a.u = act32(y, blk);
        a.d8 = y.d(blk);
    }
    __device__ float dot(const P &p, const A &a) const {
        return p.d * a.d8 * i2f(dot16(p.q1, a.u.hi, dot16(p.q0, a.u.lo)));
    }
};

// Q4_0: 1 unit per 18-byte block; value j < 16 = low nibble of qs[j], j >= 16 high.
// Result d * (d8 * sum(nibble * q8) - 8 * s8) with s8 the stored fp16 d8*sum(q8).
// vecdotq.cuh:46-66,493-509.
template <> struct Unit<Q4_0> {
    static constexpr int PER_BLOCK = 1;
    struct W { uint4 q; uint32_t d; };
    struct P { uint4 lo, hi; float d; };
    struct A { Q32 u; float d8, s8x8; };
    __device__ explicit Unit(int) {}
    __device__ void load_w(W &w, const uint8_t *blk) const {
        w.d = load_unaligned<uint16_t>(blk);
        w.q = load_unaligned<uint4>(blk + 2);
    }
    __device__ P prep(const W &w) const {
        return {and4(w.q, 0x0f0f0f0fu), and4(shr4(w.q, 4), 0x0f0f0f0fu), half_bits_to_float(w.d)};
    }
    template <class Y> __device__ void load_a(A &a, const Y &y, int blk) const {
        a.u = act32(y, blk);
        const uint32_t ds = y.ds(blk);
        a.d8 = half_bits_to_float(ds & 0xffffu);
        a.s8x8 = 8.0f * half_bits_to_float(ds >> 16);
    }
    __device__ float dot(const P &p, const A &a) const {
        return p.d * fmaf(a.d8, i2f(dot16(p.hi, a.u.hi, dot16(p.lo, a.u.lo))), -a.s8x8);
    }
};

// Q4_K: 4 units per 144-byte superblock. Unit j holds qs[32j, 32j+32): low nibbles are
// sub-block 2j, high nibbles sub-block 2j+1 (32 values each). The 6-bit scales/mins
// (12 bytes) are unpacked in registers per gguf-py quants.py:480-502.
// Result sum_i d8_i (d sc_i dot_i - dmin m_i sum(q8_i)). vecdotq.cuh:328-351,1159-1202.
template <> struct Unit<Q4_K> {
    static constexpr int PER_BLOCK = 4;
    struct W { uint4 q0, q1, hdr; };
    struct P { uint4 l0, l1, h0, h1; float dlo, dhi, mlo, mhi; };  // d*sc and dmin*m per sub-block
    struct A { Q32 lo, hi; float d8lo, d8hi, slo, shi; };
    int j;
    __device__ explicit Unit(int sub) : j(sub) {}
    __device__ void load_w(W &w, const uint8_t *blk) const {
        w.hdr = load_unaligned<uint4>(blk);
        w.q0 = load_unaligned<uint4>(blk + 16 + 32 * j);
        w.q1 = load_unaligned<uint4>(blk + 32 + 32 * j);
    }
    __device__ P prep(const W &w) const {
        const float d = half_bits_to_float(w.hdr.x & 0xffffu);
        const float dmin = half_bits_to_float(w.hdr.x >> 16);
        const int sh = 16 * (j & 1);
        const uint32_t s03 = (w.hdr.y >> sh) & 0xffffu, s47 = (w.hdr.z >> sh) & 0xffffu,
                       s8b = (w.hdr.w >> sh) & 0xffffu;
        // sub-blocks 0..3: 6 low bits of bytes 0..3 (scale) and 4..7 (min);
        // sub-blocks 4..7: low/high nibble of bytes 8..11 plus the top 2 bits of 0..7.
        const uint32_t sc = j < 2 ? (s03 & 0x3f3fu) : ((s8b & 0x0f0fu) | ((s03 & 0xc0c0u) >> 2));
        const uint32_t mn = j < 2 ? (s47 & 0x3f3fu) : (((s8b >> 4) & 0x0f0fu) | ((s47 & 0xc0c0u) >> 2));
        P p;
        p.l0 = and4(w.q0, 0x0f0f0f0fu);
        p.l1 = and4(w.q1, 0x0f0f0f0fu);
        p.h0 = and4(shr4(w.q0, 4), 0x0f0f0f0fu);
        p.h1 = and4(shr4(w.q1, 4), 0x0f0f0f0fu);
        p.dlo = d * i2f(static_cast<int>(sc & 0xffu));
        p.dhi = d * i2f(static_cast<int>(sc >> 8));
        p.mlo = dmin * i2f(static_cast<int>(mn & 0xffu));
        p.mhi = dmin * i2f(static_cast<int>(mn >> 8));
        return p;
    }
    template <class Y> __device__ void load_a(A &a, const Y &y, int blk) const {
        const int b = 8 * blk + 2 * j;
        a.lo = act32(y, b);
        a.hi = act32(y, b + 1);
        a.d8lo = y.d(b);
        a.d8hi = y.d(b + 1);
        a.slo = i2f(y.sum(b));
        a.shi = i2f(y.sum(b + 1));
    }
    __device__ float dot(const P &p, const A &a) const {
        const int ilo = dot16(p.l1, a.lo.hi, dot16(p.l0, a.lo.lo));
        const int ihi = dot16(p.h1, a.hi.hi, dot16(p.h0, a.hi.lo));
        const float tlo = fmaf(p.dlo, i2f(ilo), -p.mlo * a.slo);
        const float thi = fmaf(p.dhi, i2f(ihi), -p.mhi * a.shi);
        return fmaf(a.d8lo, tlo, a.d8hi * thi);
    }
};

// Q6_K: 4 units per 210-byte superblock. Value e = 128h + 32s + l takes its low
// 4 bits from ql[64h + 32(s%2) + l] (nibble s/2) and its high 2 bits from
// qh[32h + l] (bits 2s), minus 32; scale scales[e/16] (gguf-py quants.py:553-573).
// Unit c = 2h + p reads ql[32c, 32c+32) and qh[32h, 32h+32): low nibbles are group
// s = p, high nibbles group s = p + 2, each a full Q8_1 block.
// Result d * sum_g d8 sc_g dot(q - 32, q8) over 16-value groups. vecdotq.cuh:447-465,1417-1441.
template <> struct Unit<Q6_K> {
    static constexpr int PER_BLOCK = 4;
    struct W { uint4 l0, l1, h0, h1; uint2 sc; uint32_t d; };
    struct P { uint4 a0, a1, b0, b1; float da0, da1, db0, db1; };  // codes 0..63, d*sc per 16-group
    struct A { Q32 ua, ub; float d8a, d8b; int sa0, sa1, sb0, sb1; };
    int c, h, p;
    __device__ explicit Unit(int sub) : c(sub), h(sub / 2), p(sub % 2) {}
    template <typename P>  // global memory or the GEMV's LDS transpose buffer
    __device__ void load_w(W &w, P blk) const {
        w.l0 = load_unaligned<uint4>(blk + 32 * c);
        w.l1 = load_unaligned<uint4>(blk + 32 * c + 16);
        w.h0 = load_unaligned<uint4>(blk + 128 + 32 * h);
        w.h1 = load_unaligned<uint4>(blk + 144 + 32 * h);
        // scales[8h + 2p .. 8h + 2p + 6): groups (s = p: +0, +1) and (s = p + 2: +4, +5)
        w.sc = load_unaligned<uint2>(blk + 192 + 8 * h + 2 * p);
        w.d = load_unaligned<uint16_t>(blk + 208);
    }
    __device__ static uint32_t code(uint32_t ql, uint32_t qh, int nib, int sh) {
        return ((ql >> (4 * nib)) & 0x0f0f0f0fu) | (((qh >> sh) & 0x03030303u) << 4);
    }
    __device__ P prep(const W &w) const {
        const int sha = 2 * p, shb = 2 * p + 4;
        P r;
        r.a0 = make_uint4(code(w.l0.x, w.h0.x, 0, sha), code(w.l0.y, w.h0.y, 0, sha),
                          code(w.l0.z, w.h0.z, 0, sha), code(w.l0.w, w.h0.w, 0, sha));
        r.a1 = make_uint4(code(w.l1.x, w.h1.x, 0, sha), code(w.l1.y, w.h1.y, 0, sha),
                          code(w.l1.z, w.h1.z, 0, sha), code(w.l1.w, w.h1.w, 0, sha));
        r.b0 = make_uint4(code(w.l0.x, w.h0.x, 1, shb), code(w.l0.y, w.h0.y, 1, shb),
                          code(w.l0.z, w.h0.z, 1, shb), code(w.l0.w, w.h0.w, 1, shb));
        r.b1 = make_uint4(code(w.l1.x, w.h1.x, 1, shb), code(w.l1.y, w.h1.y, 1, shb),
                          code(w.l1.z, w.h1.z, 1, shb), code(w.l1.w, w.h1.w, 1, shb));
        const float d = half_bits_to_float(w.d);
        r.da0 = d * i2f(static_cast<int8_t>(w.sc.x & 0xffu));
        r.da1 = d * i2f(static_cast<int8_t>((w.sc.x >> 8) & 0xffu));
        r.db0 = d * i2f(static_cast<int8_t>(w.sc.y & 0xffu));
        r.db1 = d * i2f(static_cast<int8_t>((w.sc.y >> 8) & 0xffu));
        return r;
    }
    template <class Y> __device__ void load_a(A &a, const Y &y, int blk) const {
        const int b = 8 * blk + 4 * h + p;
        a.ua = act32(y, b);
        a.ub = act32(y, b + 2);
        a.d8a = y.d(b);
        a.d8b = y.d(b + 2);
        a.sa0 = 32 * y.sum_lo(b);
        a.sa1 = 32 * y.sum_hi(b);
        a.sb0 = 32 * y.sum_lo(b + 2);
        a.sb1 = 32 * y.sum_hi(b + 2);
    }
    __device__ float dot(const P &r, const A &a) const {
        // exact dots of (code - 32) and q8 per 16-value group
        const float ta = fmaf(r.da0, i2f(dot16(r.a0, a.ua.lo) - a.sa0), r.da1 * i2f(dot16(r.a1, a.ua.hi) - a.sa1));
        const float tb = fmaf(r.db0, i2f(dot16(r.b0, a.ub.lo) - a.sb0), r.db1 * i2f(dot16(r.b1, a.ub.hi) - a.sb1));
        return fmaf(a.d8a, ta, a.d8b * tb);
    }
};

// Q2_K: 2 units per 84-byte superblock. Value e = 128h + 32s + l is
// (qs[32h + l] >> 2s) & 3 with scale byte scales[e/16] (low nibble sc, high m)
// (gguf-py quants.py:407-429). Unit h reads qs[32h, 32h+32) and covers Q8_1 blocks
// 4h + s, s = 0..3 (8 groups of 16 values).
// Result sum_g d8 (d sc_g dot_g - dmin m_g sum(q8_g)). vecdotq.cuh:204-230,923-944.
template <> struct Unit<Q2_K> {
    static constexpr int PER_BLOCK = 2;
    struct W { uint4 q0, q1; uint2 sc; uint32_t dm; };
    struct P { uint4 q0, q1; float dsc[8], mmn[8]; };
    struct A { Q32 u[4]; float d8[4]; float s[8]; };
    int h;
    __device__ explicit Unit(int sub) : h(sub) {}
    __device__ void load_w(W &w, const uint8_t *blk) const {
        w.q0 = load_unaligned<uint4>(blk + 16 + 32 * h);
        w.q1 = load_unaligned<uint4>(blk + 32 + 32 * h);
        w.sc = load_unaligned<uint2>(blk + 8 * h);
        w.dm = load_unaligned<uint32_t>(blk + 80);
    }
    __device__ P prep(const W &w) const {
        const float d = half_bits_to_float(w.dm & 0xffffu);
        const float dmin = half_bits_to_float(w.dm >> 16);
        P p;
        p.q0 = w.q0;
        p.q1 = w.q1;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint32_t byte = ((g < 4 ? w.sc.x : w.sc.y) >> (8 * (g % 4))) & 0xffu;
            p.dsc[g] = d * i2f(static_cast<int>(byte & 0x0fu));
            p.mmn[g] = dmin * i2f(static_cast<int>(byte >> 4));
        }
        return p;
    }
    template <class Y> __device__ void load_a(A &a, const Y &y, int blk) const {
        const int b = 8 * blk + 4 * h;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            a.u[s] = act32(y, b + s);
            a.d8[s] = y.d(b + s);
            a.s[2 * s] = i2f(y.sum_lo(b + s));
            a.s[2 * s + 1] = i2f(y.sum_hi(b + s));
        }
    }
    __device__ float dot(const P &p, const A &a) const {
        float acc = 0.0f;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int ilo = dot16(and4(shr4(p.q0, 2 * s), 0x03030303u), a.u[s].lo);
            const int ihi = dot16(and4(shr4(p.q1, 2 * s), 0x03030303u), a.u[s].hi);
            const float t = fmaf(p.dsc[2 * s], i2f(ilo), fmaf(p.dsc[2 * s + 1], i2f(ihi),
                                 -(p.mmn[2 * s] * a.s[2 * s] + p.mmn[2 * s + 1] * a.s[2 * s + 1])));
            acc = fmaf(a.d8[s], t, acc);
        }
        return acc;
    }
};

// IQ3_S: 4 units per 110-byte superblock, unit q covering groups 2q and 2q+1 (32 values
// each). Value t = 4i + j of group g is level j of grid entry qs[8g+i] | (bit i of qh[g]) << 8,
// negated when bit t of signs[4g..4g+4) is set; group scale d*(1 + 2*nibble g of
// scales) (gguf-py quants.py:1097-1125). The 512-entry grid lives in LDS.
// Result sum_g d d8_g (1 + 2 sc_g) dot(level * sign, q8_g). vecdotq.cuh:1649-1672.
template <> struct Unit<IQ3_S> {
    static constexpr int PER_BLOCK = 4;
    struct W { uint4 qs; uint2 signs; uint32_t qh, sc, d; };
    struct P { uint4 v[4]; float d0, d1; };  // signed levels of 64 values, d*(1+2sc) per group
    struct A { Q32 u0, u1; float d80, d81; };
    int q;
    const uint32_t *grid;  // LDS
    __device__ Unit(int sub, const uint32_t *lds_grid) : q(sub), grid(lds_grid) {}
    template <typename P>  // global memory or the GEMV's LDS transpose buffer
    __device__ void load_w(W &w, P blk) const {
        w.d = load_unaligned<uint16_t>(blk);
        w.qs = load_unaligned<uint4>(blk + 2 + 16 * q);
        w.qh = load_unaligned<uint16_t>(blk + 66 + 2 * q);
        w.signs = load_unaligned<uint2>(blk + 74 + 8 * q);
        w.sc = blk[106 + q];
    }
    __device__ static uint32_t signed_levels(uint32_t levels, uint32_t nibble) {
        // spread the 4 sign bits to the 4 bytes, then negate those bytes (levels <= 15,
        // so no byte carries into its neighbour)
        const uint32_t m = ((nibble * 0x00204081u) & 0x01010101u) * 0xffu;
        return (levels ^ m) + (m & 0x01010101u);
    }
    __device__ P prep(const W &w) const {
        const uint32_t idx8[4] = {w.qs.x, w.qs.y, w.qs.z, w.qs.w};
        const uint32_t sg[2] = {w.signs.x, w.signs.y};
        uint32_t v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {  // value slots 4i..4i+3 of the unit (group i / 8)
            const uint32_t byte = (idx8[i / 4] >> (8 * (i % 4))) & 0xffu;
            const uint32_t idx = byte | (((w.qh >> i) & 1u) << 8);
            v[i] = signed_levels(grid[idx], (sg[i / 8] >> (4 * (i % 8))) & 0x0fu);
        }
        const float d = half_bits_to_float(w.d);
        return {{make_uint4(v[0], v[1], v[2], v[3]), make_uint4(v[4], v[5], v[6], v[7]),
                 make_uint4(v[8], v[9], v[10], v[11]), make_uint4(v[12], v[13], v[14], v[15])},
                d * i2f(static_cast<int>(1 + 2 * (w.sc & 0x0fu))), d * i2f(static_cast<int>(1 + 2 * (w.sc >> 4)))};
    }
    template <class Y> __device__ void load_a(A &a, const Y &y, int blk) const {
        const int b = 8 * blk + 2 * q;
        a.u0 = act32(y, b);
        a.u1 = act32(y, b + 1);
        a.d80 = y.d(b);
        a.d81 = y.d(b + 1);
    }
    __device__ float dot(const P &p, const A &a) const {
        const int i0 = dot16(p.v[1], a.u0.hi, dot16(p.v[0], a.u0.lo));
        const int i1 = dot16(p.v[3], a.u1.hi, dot16(p.v[2], a.u1.lo));
        return fmaf(p.d0 * a.d80, i2f(i0), p.d1 * a.d81 * i2f(i1));
    }
};

}  // namespace kai
