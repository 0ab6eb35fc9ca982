// Per-format "units" for the v_dot4 GEMV: the slice of one wire block that one
// lane decodes in one step, the matching slice of the Q8_1 activation, and the
// scaled integer dot product of the two.
//
// A unit is chosen so that the lanes of a wave that walk consecutive units read
// consecutive 16-byte pieces of the weight stream (coalesced), and so that the
// number of units per block divides 64: a lane's position inside a block is then
// fixed for the whole kernel and every index below is loop-invariant.
//
// Three steps per unit: load_w (wire bytes -> registers), prep (decode codes and
// scales once per weight unit, branch-free), dot (per activation row: exact int8
// dot products with v_dot4_i32_i8, then fp32 scaling). Arithmetic per format
// follows the reference's block dot products vec_dot_*_q8_1 (in-tree text
// vllm_gguf_plugin/csrc/gguf/vecdotq.cuh, cited per format); only the order of
// the fp32 scale multiplications differs.
#pragma once

#include "kai_device.h"

namespace kai {

// 4 Q8_1 ints (16 activation values) starting at value `first` of block b.
__device__ __forceinline__ uint4 act16(const block_q8_1 *b, int first) {
    return load_unaligned<uint4>(b->qs + first);
}
__device__ __forceinline__ float act_d(const block_q8_1 *b) {
    return half_bits_to_float(load_unaligned<uint16_t>(&b->d));
}
__device__ __forceinline__ int sum16(const uint4 u) {
    return dot4(0x01010101, u.w, dot4(0x01010101, u.z, dot4(0x01010101, u.y, dot4(0x01010101, u.x, 0))));
}
__device__ __forceinline__ int dot16(const uint4 w, const uint4 u) {
    return dot4(w.w, u.w, dot4(w.z, u.z, dot4(w.y, u.y, dot4(w.x, u.x, 0))));
}
__device__ __forceinline__ uint4 and4(uint4 v, uint32_t m) { return make_uint4(v.x & m, v.y & m, v.z & m, v.w & m); }
__device__ __forceinline__ uint4 shr4(uint4 v, int s) { return make_uint4(v.x >> s, v.y >> s, v.z >> s, v.w >> s); }
__device__ __forceinline__ float i2f(int v) { return static_cast<float>(v); }

template <int TYPE> struct Unit;

// Q8_0: 2 units per 34-byte block, 16 values each. vecdotq.cuh:165-177,852-867.
template <> struct Unit<Q8_0> {
    static constexpr int PER_BLOCK = 2;
    struct W { uint4 q; uint32_t d; };
    struct P { uint4 q; float d; };
    struct A { uint4 u; float d8; };
    int half;
    __device__ explicit Unit(int sub) : half(sub) {}
    __device__ void load_w(W &w, const uint8_t *blk) const {
        w.d = load_unaligned<uint16_t>(blk);
        w.q = load_unaligned<uint4>(blk + 2 + 16 * half);
    }
    __device__ P prep(const W &w) const { return {w.q, half_bits_to_float(w.d)}; }
    __device__ void load_a(A &a, const block_q8_1 *y, int blk) const {
        a.u = act16(y + blk, 16 * half);
        a.d8 = act_d(y + blk);
    }
    __device__ float dot(const P &p, const A &a) const { return p.d * a.d8 * i2f(dot16(p.q, a.u)); }
};

// Q4_0: 1 unit per 18-byte block; value j < 16 = low nibble of qs[j], j >= 16 high.
// Result d * (d8 * sum(nibble * q8) - 8 * s8) with s8 the stored fp16 d8*sum(q8).
// vecdotq.cuh:46-66,493-509.
template <> struct Unit<Q4_0> {
    static constexpr int PER_BLOCK = 1;
    struct W { uint4 q; uint32_t d; };
    struct P { uint4 lo, hi; float d; };
    struct A { uint4 lo, hi; float d8, s8x8; };
    __device__ explicit Unit(int) {}
    __device__ void load_w(W &w, const uint8_t *blk) const {
        w.d = load_unaligned<uint16_t>(blk);
        w.q = load_unaligned<uint4>(blk + 2);
    }
    __device__ P prep(const W &w) const {
        return {and4(w.q, 0x0f0f0f0fu), and4(shr4(w.q, 4), 0x0f0f0f0fu), half_bits_to_float(w.d)};
    }
    __device__ void load_a(A &a, const block_q8_1 *y, int blk) const {
        a.lo = act16(y + blk, 0);
        a.hi = act16(y + blk, 16);
        const uint32_t ds = load_unaligned<uint32_t>(&y[blk].d);
        a.d8 = half_bits_to_float(ds & 0xffffu);
        a.s8x8 = 8.0f * half_bits_to_float(ds >> 16);
    }
    __device__ float dot(const P &p, const A &a) const {
        const int s = dot16(p.hi, a.hi) + dot16(p.lo, a.lo);
        return p.d * fmaf(a.d8, i2f(s), -a.s8x8);
    }
};

// Q4_K: 8 units per 144-byte superblock. Unit c holds qs[16c, 16c+16): its low
// nibbles are values 16(c%2).. of sub-block 2(c/2), its high nibbles the same
// values of sub-block 2(c/2)+1. Scales/mins (6-bit, 12 bytes) are unpacked in
// registers per gguf-py quants.py:480-502.
// Result sum_i d8_i (d sc_i dot_i - dmin m_i sum(q8_i)). vecdotq.cuh:328-351,1159-1202.
template <> struct Unit<Q4_K> {
    static constexpr int PER_BLOCK = 8;
    struct W { uint4 q, hdr; };
    struct P { uint4 lo, hi; float dlo, dhi, mlo, mhi; };  // d*sc and dmin*m per sub-block
    struct A { uint4 lo, hi; float d8lo, d8hi, slo, shi; };
    int c, pair, half;
    __device__ explicit Unit(int sub) : c(sub), pair(sub / 2), half(sub % 2) {}
    __device__ void load_w(W &w, const uint8_t *blk) const {
        w.hdr = load_unaligned<uint4>(blk);
        w.q = load_unaligned<uint4>(blk + 16 + 16 * c);
    }
    __device__ P prep(const W &w) const {
        const float d = half_bits_to_float(w.hdr.x & 0xffffu);
        const float dmin = half_bits_to_float(w.hdr.x >> 16);
        const int sh = 16 * (pair & 1);
        const uint32_t s03 = (w.hdr.y >> sh) & 0xffffu, s47 = (w.hdr.z >> sh) & 0xffffu,
                       s8b = (w.hdr.w >> sh) & 0xffffu;
        // sub-blocks 0..3: 6 low bits of bytes 0..3 (scale) and 4..7 (min);
        // sub-blocks 4..7: low/high nibble of bytes 8..11 plus the top 2 bits of 0..7.
        const uint32_t sc_lo4 = s03 & 0x3f3fu, mn_lo4 = s47 & 0x3f3fu;
        const uint32_t sc_hi4 = (s8b & 0x0f0fu) | ((s03 & 0xc0c0u) >> 2);
        const uint32_t mn_hi4 = ((s8b >> 4) & 0x0f0fu) | ((s47 & 0xc0c0u) >> 2);
        const uint32_t sc = pair < 2 ? sc_lo4 : sc_hi4;
        const uint32_t mn = pair < 2 ? mn_lo4 : mn_hi4;
        P p;
        p.lo = and4(w.q, 0x0f0f0f0fu);
        p.hi = and4(shr4(w.q, 4), 0x0f0f0f0fu);
        p.dlo = d * i2f(static_cast<int>(sc & 0xffu));
        p.dhi = d * i2f(static_cast<int>(sc >> 8));
        p.mlo = dmin * i2f(static_cast<int>(mn & 0xffu));
        p.mhi = dmin * i2f(static_cast<int>(mn >> 8));
        return p;
    }
    __device__ void load_a(A &a, const block_q8_1 *y, int blk) const {
        const block_q8_1 *b = y + 8 * blk + 2 * pair;
        a.lo = act16(b, 16 * half);
        a.hi = act16(b + 1, 16 * half);
        a.d8lo = act_d(b);
        a.d8hi = act_d(b + 1);
        a.slo = i2f(sum16(a.lo));
        a.shi = i2f(sum16(a.hi));
    }
    __device__ float dot(const P &p, const A &a) const {
        const float tlo = fmaf(p.dlo, i2f(dot16(p.lo, a.lo)), -p.mlo * a.slo);
        const float thi = fmaf(p.dhi, i2f(dot16(p.hi, a.hi)), -p.mhi * a.shi);
        return fmaf(a.d8lo, tlo, a.d8hi * thi);
    }
};

// Q6_K: 8 units per 210-byte superblock. Value e = 128h + 32s + l takes its low
// 4 bits from ql[64h + 32(s%2) + l] (nibble s/2) and its high 2 bits from
// qh[32h + l] (bits 2s), minus 32; scale scales[e/16] (gguf-py quants.py:553-573).
// Unit c reads ql[16c, 16c+16) (h = c/4, p = (c/2)%2, half = c%2): low nibbles are
// the 16 values of group s = p, high nibbles those of s = p + 2.
// Result d * sum_g d8 sc_g dot(q - 32, q8). vecdotq.cuh:447-465,1417-1441.
template <> struct Unit<Q6_K> {
    static constexpr int PER_BLOCK = 8;
    struct W { uint4 ql, qh; uint2 sc; uint32_t d; };
    struct P { uint4 ca, cb; float da, db; };  // codes 0..63 and d*sc per group
    struct A { uint4 ua, ub; float d8a, d8b; int sa32, sb32; };
    int c, h, p, half, sc_word, sc_shift;
    __device__ explicit Unit(int sub) : c(sub), h(sub / 4), p((sub / 2) % 2), half(sub % 2) {
        const int idx = 8 * h + 2 * p + half;  // scale of group s = p; group s = p+2 is idx + 4
        sc_word = idx / 4;
        sc_shift = 8 * (idx % 4);
    }
    __device__ void load_w(W &w, const uint8_t *blk) const {
        w.ql = load_unaligned<uint4>(blk + 16 * c);
        w.qh = load_unaligned<uint4>(blk + 128 + 32 * h + 16 * half);
        w.sc = load_unaligned<uint2>(blk + 192 + 4 * sc_word);
        w.d = load_unaligned<uint16_t>(blk + 208);
    }
    __device__ P prep(const W &w) const {
        const int sha = 2 * p, shb = 2 * p + 4;
        P r;
        r.ca = make_uint4((w.ql.x & 0x0f0f0f0fu) | (((w.qh.x >> sha) & 0x03030303u) << 4),
                          (w.ql.y & 0x0f0f0f0fu) | (((w.qh.y >> sha) & 0x03030303u) << 4),
                          (w.ql.z & 0x0f0f0f0fu) | (((w.qh.z >> sha) & 0x03030303u) << 4),
                          (w.ql.w & 0x0f0f0f0fu) | (((w.qh.w >> sha) & 0x03030303u) << 4));
        r.cb = make_uint4(((w.ql.x >> 4) & 0x0f0f0f0fu) | (((w.qh.x >> shb) & 0x03030303u) << 4),
                          ((w.ql.y >> 4) & 0x0f0f0f0fu) | (((w.qh.y >> shb) & 0x03030303u) << 4),
                          ((w.ql.z >> 4) & 0x0f0f0f0fu) | (((w.qh.z >> shb) & 0x03030303u) << 4),
                          ((w.ql.w >> 4) & 0x0f0f0f0fu) | (((w.qh.w >> shb) & 0x03030303u) << 4));
        const float d = half_bits_to_float(w.d);
        r.da = d * i2f(static_cast<int8_t>((w.sc.x >> sc_shift) & 0xffu));
        r.db = d * i2f(static_cast<int8_t>((w.sc.y >> sc_shift) & 0xffu));
        return r;
    }
    __device__ void load_a(A &a, const block_q8_1 *y, int blk) const {
        const block_q8_1 *b = y + 8 * blk + 4 * h + p;
        a.ua = act16(b, 16 * half);
        a.ub = act16(b + 2, 16 * half);
        a.d8a = act_d(b);
        a.d8b = act_d(b + 2);
        a.sa32 = 32 * sum16(a.ua);
        a.sb32 = 32 * sum16(a.ub);
    }
    __device__ float dot(const P &r, const A &a) const {
        const int ia = dot16(r.ca, a.ua) - a.sa32;  // exact dot of (code - 32) and q8
        const int ib = dot16(r.cb, a.ub) - a.sb32;
        return fmaf(r.da * a.d8a, i2f(ia), r.db * a.d8b * i2f(ib));
    }
};

// Q2_K: 4 units per 84-byte superblock. Value e = 128h + 32s + l is
// (qs[32h + l] >> 2s) & 3 with scale byte scales[e/16] (low nibble sc, high m)
// (gguf-py quants.py:407-429). Unit c reads qs[16c, 16c+16) (h = c/2, half = c%2)
// and covers 4 groups of 16 values, s = 0..3.
// Result sum_g d8 (d sc_g dot_g - dmin m_g sum(q8_g)). vecdotq.cuh:204-230,923-944.
template <> struct Unit<Q2_K> {
    static constexpr int PER_BLOCK = 4;
    struct W { uint4 q; uint2 sc; uint32_t dm; };
    struct P { uint4 q; float dsc[4], mmn[4]; };
    struct A { uint4 u[4]; float d8[4], s[4]; };
    int c, h, half;
    __device__ explicit Unit(int sub) : c(sub), h(sub / 2), half(sub % 2) {}
    __device__ void load_w(W &w, const uint8_t *blk) const {
        w.q = load_unaligned<uint4>(blk + 16 + 16 * c);
        w.sc = load_unaligned<uint2>(blk + 8 * h);
        w.dm = load_unaligned<uint32_t>(blk + 80);
    }
    __device__ P prep(const W &w) const {
        const float d = half_bits_to_float(w.dm & 0xffffu);
        const float dmin = half_bits_to_float(w.dm >> 16);
        const uint32_t s01 = w.sc.x >> (8 * half), s23 = w.sc.y >> (8 * half);
        const uint32_t scb[4] = {s01 & 0xffu, (s01 >> 16) & 0xffu, s23 & 0xffu, (s23 >> 16) & 0xffu};
        P p;
        p.q = w.q;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            p.dsc[s] = d * i2f(static_cast<int>(scb[s] & 0x0fu));
            p.mmn[s] = dmin * i2f(static_cast<int>(scb[s] >> 4));
        }
        return p;
    }
    __device__ void load_a(A &a, const block_q8_1 *y, int blk) const {
        const block_q8_1 *b = y + 8 * blk + 4 * h;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            a.u[s] = act16(b + s, 16 * half);
            a.d8[s] = act_d(b + s);
            a.s[s] = i2f(sum16(a.u[s]));
        }
    }
    __device__ float dot(const P &p, const A &a) const {
        float acc = 0.0f;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int di = dot16(and4(shr4(p.q, 2 * s), 0x03030303u), a.u[s]);
            acc = fmaf(a.d8[s], fmaf(p.dsc[s], i2f(di), -p.mmn[s] * a.s[s]), acc);
        }
        return acc;
    }
};

// IQ3_S: 8 units per 110-byte superblock, one per 32-value group g. Value
// t = 4i + j of group g is level j of grid entry qs[8g+i] | (bit i of qh[g]) << 8,
// negated when bit t of signs[4g..4g+4) is set; group scale d*(1 + 2*nibble g of
// scales) (gguf-py quants.py:1097-1125). The 512-entry grid lives in LDS.
// Result sum_g d d8_g (1 + 2 sc_g) dot(level * sign, q8_g). vecdotq.cuh:1649-1672.
template <> struct Unit<IQ3_S> {
    static constexpr int PER_BLOCK = 8;
    struct W { uint2 qs; uint32_t signs, qh, sc, d; };
    struct P { uint4 lo, hi; float dg; };  // signed levels of the 32 values, d*(1+2sc)
    struct A { uint4 lo, hi; float d8; };
    int g;
    const uint32_t *grid;  // LDS
    __device__ Unit(int sub, const uint32_t *lds_grid) : g(sub), grid(lds_grid) {}
    __device__ void load_w(W &w, const uint8_t *blk) const {
        w.d = load_unaligned<uint16_t>(blk);
        w.qs = load_unaligned<uint2>(blk + 2 + 8 * g);
        w.qh = blk[66 + g];
        w.signs = load_unaligned<uint32_t>(blk + 74 + 4 * g);
        w.sc = blk[106 + g / 2];
    }
    __device__ static uint32_t signed_levels(uint32_t levels, uint32_t nibble) {
        // spread the 4 sign bits to the 4 bytes, then negate those bytes (levels <= 15,
        // so no byte carries into its neighbour)
        const uint32_t m = ((nibble * 0x00204081u) & 0x01010101u) * 0xffu;
        return (levels ^ m) + (m & 0x01010101u);
    }
    __device__ P prep(const W &w) const {
        uint32_t v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t byte = (i < 4 ? w.qs.x >> (8 * i) : w.qs.y >> (8 * (i - 4))) & 0xffu;
            const uint32_t idx = byte | (((w.qh >> i) & 1u) << 8);
            v[i] = signed_levels(grid[idx], (w.signs >> (4 * i)) & 0x0fu);
        }
        const uint32_t sc = (w.sc >> (4 * (g % 2))) & 0x0fu;
        return {make_uint4(v[0], v[1], v[2], v[3]), make_uint4(v[4], v[5], v[6], v[7]),
                half_bits_to_float(w.d) * i2f(static_cast<int>(1 + 2 * sc))};
    }
    __device__ void load_a(A &a, const block_q8_1 *y, int blk) const {
        const block_q8_1 *b = y + 8 * blk + g;
        a.lo = act16(b, 0);
        a.hi = act16(b, 16);
        a.d8 = act_d(b);
    }
    __device__ float dot(const P &p, const A &a) const {
        return p.dg * a.d8 * i2f(dot16(p.hi, a.hi) + dot16(p.lo, a.lo));
    }
};

}  // namespace kai
