// Weight side of the int8-MFMA kernels, per GGUF format: what one lane loads for one
// 256-value K step of its weight row, the int8 codes of its octet of block kb (the MFMA
// B operand), the fp32 scale of block kb, and the weight factors of the min terms.
// Used by the batched MMQ kernel (kai_mmq.cuh). Arithmetic per format follows the
// reference's block dots
// vec_dot_*_q8_1 (in-tree text vllm_gguf_plugin/csrc/gguf/vecdotq.cuh, cited per format).
#pragma once

#include "kai_iq3s_grid.h"
#include "kai_launch.h"
#include "kai_units.h"

namespace kai {

typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef float v4f_t __attribute__((ext_vector_type(4)));

static __device__ const uint32_t mmq_iq3s_grid[512] = {KAI_IQ3S_GRID_VALUES};

constexpr int MMQ_THREADS = 256;
constexpr int MMQ_STEP = 256;  // values per K step (one superblock, or 8 blocks of 32)

__device__ __forceinline__ uint64_t u64(uint2 v) { return uint64_t(v.x) | (uint64_t(v.y) << 32); }
// v rounded to fp16 and back: the half products GGML MMQ's tile loaders form.
__device__ __forceinline__ float half_round(float v) { return half_bits_to_float(float_to_half_bits(v)); }

// Epilogue of one 32-value block: one MFMA with a block scale (BLOCK), or two MFMAs over
// its 16-value halves combined with integer scales (ISPLIT) or with fp32 scales (FSPLIT).
enum MmqMode : int { MMQ_BLOCK = 0, MMQ_ISPLIT = 1, MMQ_FSPLIT = 2 };
__device__ __forceinline__ uint32_t bits(uint32_t w, uint32_t shift, uint32_t width) {
    return (w >> shift) & ((1u << width) - 1u);
}


// Weight side of the MMQ kernel, per format: what one lane loads for one K step of its
// row (load), the int8 codes of its octet of block kb (codes), the scale of block kb
// (scale: multiplies d8 * C), and the weight factors of the min terms (term: the B
// operand of the fp32 MFMA for terms 4j .. 4j+3, the lane taking term 4j + oct).
// The template flag MMA selects the batched path's weight arithmetic (GGML MMQ's tensor-
// core tile loaders, which round d*sc and dmin*m to fp16 for Q4_K and Q2_K and scale Q2_K
// per 16 values) over the decode path's (MMVQ, exact products).
template <int TYPE> struct MmqW;

// Q8_0: 8 blocks of 34 bytes per step. y += d8 * d * C. vecdotq.cuh:165-177.
template <> struct MmqW<Q8_0> {
    static constexpr int SB = 8 * 34, NTERM = 0;
    struct Raw {
        uint2 q[8];
        uint32_t d[8];
    };
    // nvalid < 8 only on a short last K step: blocks past the row end re-read its last block
    // (their activation is zero). Blocks are independent, so a caller may load them one at a
    // time (LAZY) right before their use.
    static constexpr bool LAZY = true;
    template <typename P>
    static __device__ void load_block(Raw &r, P p, int o, int nvalid, int b) {
        const int c = nvalid == 8 ? b : min(b, nvalid - 1);
        r.d[b] = load_unaligned<uint16_t>(p + 34 * c);
        r.q[b] = load_unaligned<uint2>(p + 34 * c + 2 + 8 * o);
    }
    template <typename P>
    static __device__ void load(Raw &r, P p, int o, int nvalid) {
#pragma unroll
        for (int b = 0; b < 8; ++b) load_block(r, p, o, nvalid, b);
    }
    template <bool MMA> static constexpr int mode() { return MMQ_BLOCK; }
    template <bool MMA> static __device__ uint64_t codes(const Raw &r, int b, int, const uint32_t *) { return u64(r.q[b]); }
    template <bool MMA> static __device__ float scale(const Raw &r, int b) { return half_bits_to_float(r.d[b]); }
    template <bool MMA> static __device__ float term(const Raw &, int, int) { return 0.0f; }
};

// Q4_0: 8 blocks of 18 bytes; value v < 16 is the low nibble of qs[v], v >= 16 the high
// nibble of qs[v - 16]. y += d * (d8 * C - 8 * t): t is the stored fp16 d8*sum(q8) on the
// decode activation (vecdotq.cuh:46-66), d8 * sum(q8) on the batched one (GGML MMQ's
// tensor-core tile takes the codes minus 8).
template <> struct MmqW<Q4_0> {
    static constexpr int SB = 8 * 18, NTERM = 8;
    struct Raw {
        uint2 q[8];
        uint32_t d[8];
    };
    static constexpr bool LAZY = true;  // independent blocks, as Q8_0
    template <typename P>
    static __device__ void load_block(Raw &r, P p, int o, int nvalid, int b) {
        const int c = nvalid == 8 ? b : min(b, nvalid - 1);
        r.d[b] = load_unaligned<uint16_t>(p + 18 * c);
        r.q[b] = load_unaligned<uint2>(p + 18 * c + 2 + 8 * (o & 1));
    }
    template <typename P>
    static __device__ void load(Raw &r, P p, int o, int nvalid) {
#pragma unroll
        for (int b = 0; b < 8; ++b) load_block(r, p, o, nvalid, b);
    }
    template <bool MMA> static constexpr int mode() { return MMQ_BLOCK; }
    template <bool MMA> static __device__ uint64_t codes(const Raw &r, int b, int o, const uint32_t *) {
        return (u64(r.q[b]) >> (4 * (o >> 1))) & 0x0f0f0f0f0f0f0f0full;
    }
    template <bool MMA> static __device__ float scale(const Raw &r, int b) { return half_bits_to_float(r.d[b]); }
    template <bool MMA> static __device__ float term(const Raw &r, int j, int o) {  // block 4j + o: -8 d
        const uint32_t d = o == 0 ? r.d[4 * j] : o == 1 ? r.d[4 * j + 1] : o == 2 ? r.d[4 * j + 2] : r.d[4 * j + 3];
        return -8.0f * half_bits_to_float(d);
    }
};

// Q4_K superblock: d, dmin (fp16), 12 bytes of 6-bit scales/mins, qs[128]. Chunk c holds
// blocks 2c (low nibbles) and 2c+1 (high nibbles); octet o of both is qs[32c + 8o, +8).
// y += d8 * d * sc * C - dmin * m * t, t = d8 * sum(q8) (decode, vecdotq.cuh:328-351) or
// y += d8 * half(d * sc) * C - half(dmin * m) * s8 with the stored sum s8 (batched, GGML
// MMQ's load_tiles_q4_K and its tensor-core dot). Scale packing gguf-py quants.py:480-502.
template <> struct MmqW<Q4_K> {
    static constexpr int SB = 144, NTERM = 8;
    struct Raw {
        uint4 hdr;
        uint2 q[4];
    };
    template <typename P>  // whole superblocks: no short step
    static __device__ void load(Raw &r, P p, int o, int) {
        r.hdr = load_unaligned<uint4>(p);
#pragma unroll
        for (int c = 0; c < 4; ++c) r.q[c] = load_unaligned<uint2>(p + 16 + 32 * c + 8 * o);
    }
    template <bool MMA> static constexpr int mode() { return MMQ_BLOCK; }
    template <bool MMA> static __device__ uint64_t codes(const Raw &r, int b, int, const uint32_t *) {
        const uint64_t q = u64(r.q[b / 2]);
        return ((b & 1) ? q >> 4 : q) & 0x0f0f0f0f0f0f0f0full;
    }
    template <bool MMA> static __device__ float scale(const Raw &r, int b) {
        const float d = half_bits_to_float(r.hdr.x & 0xffffu);
        const uint32_t sc = b < 4 ? bits(r.hdr.y, 8 * b, 6)
                                  : bits(r.hdr.w, 8 * (b - 4), 4) | (bits(r.hdr.y, 8 * (b - 4) + 6, 2) << 4);
        const float v = d * static_cast<float>(sc);  // exact: 11 x 6 bits
        return MMA ? half_round(v) : v;
    }
    template <bool MMA> static __device__ float term(const Raw &r, int j, int o) {  // block 4j + o: -dmin * m
        const float dmin = half_bits_to_float(r.hdr.x >> 16);
        const uint32_t mn = j == 0 ? bits(r.hdr.z, 8 * o, 6)
                                   : bits(r.hdr.w, 8 * o + 4, 4) | (bits(r.hdr.z, 8 * o + 6, 2) << 4);
        const float v = dmin * static_cast<float>(mn);
        return -(MMA ? half_round(v) : v);
    }
};

// Q6_K superblock: ql[128], qh[64], int8 scales[16], d. Block kb = 4h + s, value v:
// ql[64h + 32(s&1) + v] nibble s>>1, qh[32h + v] bits 2s; code q - 32 with one int8
// scale per 16 values, so two MFMAs per block (the other half's codes zeroed) and the
// two scales combined in 24-bit integer arithmetic. vecdotq.cuh:447-465; layout
// gguf-py quants.py:553-573.
template <> struct MmqW<Q6_K> {
    static constexpr int SB = 210, NTERM = 0;
    struct Raw {
        uint2 ql[4];
        uint2 qh[2];
        uint4 sc;
        uint32_t d;
    };
    template <typename P>  // whole superblocks: no short step
    static __device__ void load(Raw &r, P p, int o, int) {
#pragma unroll
        for (int i = 0; i < 4; ++i) r.ql[i] = load_unaligned<uint2>(p + 64 * (i / 2) + 32 * (i % 2) + 8 * o);
#pragma unroll
        for (int h = 0; h < 2; ++h) r.qh[h] = load_unaligned<uint2>(p + 128 + 32 * h + 8 * o);
        r.sc = load_unaligned<uint4>(p + 192);
        r.d = load_unaligned<uint16_t>(p + 208);
    }
    // code - 32 = (high 2 bits - 2) * 16 + low nibble: the high bits select the int8 high
    // nibble (0xE0, 0xF0, 0x00, 0x10) from a byte table (v_perm_b32, selectors 0-3 pick the
    // second operand's bytes), the low nibble is OR-ed in.
    static __device__ uint32_t codes4(uint32_t ql, uint32_t qh, int nshift, int hshift) {
        const uint32_t hi = __builtin_amdgcn_perm(0u, 0x1000f0e0u, (qh >> hshift) & 0x03030303u);
        return ((ql >> nshift) & 0x0f0f0f0fu) | hi;
    }
    template <bool MMA> static __device__ uint64_t codes(const Raw &r, int b, int, const uint32_t *) {
        const int h = b / 4, s = b % 4;
        const uint2 ql = r.ql[2 * h + (s & 1)], qh = r.qh[h];
        return u64(make_uint2(codes4(ql.x, qh.x, 4 * (s >> 1), 2 * s), codes4(ql.y, qh.y, 4 * (s >> 1), 2 * s)));
    }
    static __device__ int iscale(const Raw &r, int g) {  // int8 scale of 16-value group g
        const uint32_t w = g < 4 ? r.sc.x : g < 8 ? r.sc.y : g < 12 ? r.sc.z : r.sc.w;
        return static_cast<int8_t>(bits(w, 8 * (g % 4), 8));
    }
    template <bool MMA> static constexpr int mode() { return MMQ_ISPLIT; }
    template <bool MMA> static __device__ float scale(const Raw &r, int) { return half_bits_to_float(r.d); }
    template <bool MMA> static __device__ float term(const Raw &, int, int) { return 0.0f; }
};

// Q2_K superblock: scales[16] (low nibble scale, high nibble min, per 16 values),
// qs[64], d, dmin. Block kb = 4h + s: code (qs[32h + v] >> 2s) & 3.
// Decode (vecdotq.cuh:204-230): the code times its 4-bit scale (<= 45, no int8 overflow)
// so one MFMA covers both 16-value groups; y += d8 * d * C' - dmin * (m_lo t_lo + m_hi t_hi),
// t = d8 * sum(q8) per 16 values.
// Batched (GGML MMQ's load_tiles_q2_K and tensor-core dot): raw codes, one MFMA per
// 16-value half with its own fp32 scale half(d * sc); y += d8 * (half(d sc_lo) C_lo +
// half(d sc_hi) C_hi) - half(dmin m_lo) S_lo - half(dmin m_hi) S_hi, S the D2S6 sums.
// Layout gguf-py quants.py:407-429.
template <> struct MmqW<Q2_K> {
    static constexpr int SB = 84, NTERM = 16;
    struct Raw {
        uint4 sc;
        uint2 q[2];
        uint32_t dm;
    };
    template <typename P>  // whole superblocks: no short step
    static __device__ void load(Raw &r, P p, int o, int) {
        r.sc = load_unaligned<uint4>(p);
#pragma unroll
        for (int h = 0; h < 2; ++h) r.q[h] = load_unaligned<uint2>(p + 16 + 32 * h + 8 * o);
        r.dm = load_unaligned<uint32_t>(p + 80);
    }
    static __device__ uint32_t word(const Raw &r, int i) { return i == 0 ? r.sc.x : i == 1 ? r.sc.y : i == 2 ? r.sc.z : r.sc.w; }
    template <bool MMA> static constexpr int mode() { return MMA ? MMQ_FSPLIT : MMQ_BLOCK; }
    template <bool MMA> static __device__ uint64_t codes(const Raw &r, int b, int o, const uint32_t *) {
        const int h = b / 4, s = b % 4;
        const uint64_t q = (u64(r.q[h]) >> (2 * s)) & 0x0303030303030303ull;
        if constexpr (MMA) return q;
        // scale byte 2b + (o >> 1) lies in word b / 2
        const uint32_t sc = bits(word(r, b / 2), 8 * (2 * (b & 1) + (o >> 1)), 4);
        return q * sc;
    }
    template <bool MMA> static __device__ float scale(const Raw &r, int) { return half_bits_to_float(r.dm & 0xffffu); }
    static __device__ float fscale(const Raw &r, int g) {  // batched: half(d * sc) of 16-value group g
        return half_round(half_bits_to_float(r.dm & 0xffffu) * static_cast<float>(bits(word(r, g / 4), 8 * (g % 4), 4)));
    }
    template <bool MMA> static __device__ float term(const Raw &r, int j, int o) {  // 16-value group 4j + o: -dmin * m
        const float v = half_bits_to_float(r.dm >> 16) * static_cast<float>(bits(word(r, j), 8 * o + 4, 4));
        return -(MMA ? half_round(v) : v);
    }
};

// IQ3_S superblock: d, qs[64] (8-bit grid index low bits), qh[8], signs[32], scales[4].
// Block kb, octet o: grid entries qs[8kb + 2o + i] | bit (2o + i) of qh[kb] << 8, signs
// byte 4kb + o. y += d8 * d * (1 + 2 sc) * C. vecdotq.cuh:1649-1672; layout gguf-py
// quants.py:1097-1125.
template <> struct MmqW<IQ3_S> {
    static constexpr int SB = 110, NTERM = 0;
    struct Raw {
        uint32_t qs[8];
        uint32_t sg[8];
        uint2 qh;
        uint32_t sc;
        uint32_t d;
    };
    template <typename P>  // whole superblocks: no short step
    static __device__ void load(Raw &r, P p, int o, int) {
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            r.qs[b] = load_unaligned<uint16_t>(p + 2 + 8 * b + 2 * o);
            r.sg[b] = p[74 + 4 * b + o];
        }
        r.qh = load_unaligned<uint2>(p + 66);
        r.sc = load_unaligned<uint32_t>(p + 106);
        r.d = load_unaligned<uint16_t>(p);
    }
    template <bool MMA> static constexpr int mode() { return MMQ_BLOCK; }
    template <bool MMA> static __device__ uint64_t codes(const Raw &r, int b, int o, const uint32_t *grid) {
        const uint32_t qh = bits(b < 4 ? r.qh.x : r.qh.y, 8 * (b % 4), 8) >> (2 * o);
        const uint32_t i0 = (r.qs[b] & 0xffu) | ((qh & 1u) << 8);
        const uint32_t i1 = (r.qs[b] >> 8) | ((qh & 2u) << 7);
        return uint64_t(Unit<IQ3_S>::signed_levels(grid[i0], r.sg[b] & 0x0fu)) |
               (uint64_t(Unit<IQ3_S>::signed_levels(grid[i1], r.sg[b] >> 4)) << 32);
    }
    template <bool MMA> static __device__ float scale(const Raw &r, int b) {
        return half_bits_to_float(r.d) * static_cast<float>(1 + 2 * static_cast<int>(bits(r.sc, 4 * b, 4)));
    }
    template <bool MMA> static __device__ float term(const Raw &, int, int) { return 0.0f; }
};


// Coalesced weight stream. One K step of a wave's 16 rows is 16 runs of SB bytes (one per
// row); each run is read as U 16-byte units (unit c = bytes [16c, 16c + 16) of the run, the
// last one running into the next run, which is ignored), lane l taking units l, l + 64, ...,
// so that a load instruction reads whole 16-byte pieces of a few contiguous runs. The units
// go into the wave's LDS transpose buffer (row r at r * SBP) from which each lane reads its
// MFMA operand fields. (Loading the fields straight from HBM puts 16 rows in every load
// instruction, and with superblocks of 210 bytes (Q6_K) that halves the achieved bandwidth.)
template <int TYPE>
struct MmqsStream {
    // row pitch: whole units, plus one when U is even, so that the 16 rows start on 16
    // different 4-bank groups of the LDS (a pitch of 4U dwords with U even puts two rows on
    // each group, and the lanes' field reads of a step conflict in pairs)
    static constexpr int SB = MmqW<TYPE>::SB, U = (SB + 15) / 16, SBP = 16 * (U + (U % 2 == 0 ? 1 : 0));
    static constexpr int UPL = (16 * U + WAVE - 1) / WAVE;  // units per lane
};

// The MMQ kernel's view of a format: MmqW plus the lane's activation octet and the
// 16-value half it holds (used by the split Q6_K MFMA), and a post-load fix-up hook.
template <typename W, typename = void>
struct LazyLoad {
    static constexpr bool value = false;
};
template <typename W>
struct LazyLoad<W, decltype(void(W::LAZY))> {
    static constexpr bool value = W::LAZY;
};

template <int TYPE>
struct MmqLoad : MmqW<TYPE> {
    static __device__ int act_pos(int g) { return 8 * g; }
    static __device__ bool first_half(int g) { return g < 2; }  // lanes holding values 0..15
    static __device__ void fix(typename MmqW<TYPE>::Raw &) {}
};

}  // namespace kai
