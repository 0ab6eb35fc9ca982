// Prefill GEMM for K-quant weights on fp16 MFMA (kernel "mmf"), m >= MMF_MIN_ROWS.
//
// Y[m, n] = inverse[m] * sum_k a[m, k] w[n, k] over the row-normalised Q8_1 activation
// a = d8 * q8 and the dequantised weight w, the product the reference's MMQ path computes
// (kai_fused_mmq_run, vllm_gguf_plugin/native/kernels/current_ggml_direct.cu:1196-1265;
// per-format block dots in vllm_gguf_plugin/csrc/gguf/vecdotq.cuh).
//
// Why fp16 and not int8 MFMA: the reference's integer block dot needs a scale pair per
// 32 values on both operands (d8 and the sub-block scale), i.e. at least a convert and two
// fp32 operations per output element and 32-value block, and gfx950 issues VALU and MFMA
// work through one port (4 fp32 FMAs per 16x16x32 MFMA already cut its rate by a third).
// Here the scales live inside the operands:
//   * weights: B = sc * q * 2^-P (Q4_K), exact in fp16, in units of the superblock's
//     u = d * 2^P (P >= 0, only above 0 when dmin / d is so large that the min operands
//     below would leave fp16's range);
//   * activations: a16 = half(d8 * q8), written by prepare_mmf_kernel; its rounding (one
//     fp16 rounding per element, relative 2^-12) is the only departure from the integer
//     path. Its mean part, which the uncentred codes would multiply, is removed exactly:
//     u8 = sum(a16 - d8 q8) per 32-value block enters with weight -8 sc 2^-P;
//   * min terms -dmin * m * (d8 sum q8), in units of u, and that correction run as one
//     more fp16 MFMA per superblock on split operands t = hi + lo, e = -dmin m / u =
//     e_hi + e_lo: lane groups k = [0,8) hi*e_hi, [8,16) lo*e_hi, [16,24) hi*e_lo,
//     [24,32) u8*f;
//   * one fp32 accumulator set: it holds the sum in units of the current superblock's u
//     and is rescaled by u_s / u_(s+1) at each superblock end (the last by u itself), four
//     VALU multiplies per 16x16 tile per 256 values.
// Measured against the CPU restatement the result stays within 4e-4 normwise (tolerance
// 1e-3).
//
// Tiling for gfx950: 256 threads, 256 weight rows x 128 activation rows per workgroup;
// each wave owns 64 weight rows and all 128 activation rows (4 x 8 MFMA 16x16x32 tiles,
// 128 accumulator VGPRs). The weight bytes go from global memory straight into the
// lane's registers and are dequantised there into MFMA operands (no LDS traffic for the
// weights: LDS bandwidth, about 110 bytes per clock per CU, is what bounds this kernel);
// the activation tile (fp16) is shared through LDS, written by global_load_lds_dwordx4,
// double-buffered in K steps of 64 values. Two workgroups per CU. LDS activation rows are
// 128 bytes (8 chunks of 16 bytes); chunk c of row r sits at c ^ swz(r) so that the MFMA
// operand reads (16 rows, one chunk each) hit distinct banks.
// Operand layout of v_mfma_f32_16x16x32_f16: lane l holds A row l%16 and B column l%16
// for k = 8*(l/16) .. +8; D column l%16, rows 4*(l/16) + i. A = weights, B = activations.
#pragma once

#include "kai_mmq_formats.h"

namespace kai {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

constexpr int MMF_THREADS = 256;
constexpr int MMF_MT = MMF_TILE_M;    // activation rows per workgroup (6 MFMA tiles)
constexpr int MMF_MTILES = MMF_MT / 16;
constexpr int MMF_NT = MMF_TILE_N;    // weight rows per workgroup, 64 per wave
constexpr int MMF_KS = 64;            // values per K step
constexpr int MMF_ROWB = 2 * MMF_KS;  // bytes per LDS activation row of one step
constexpr int MMF_STAGE = MMF_MT * MMF_ROWB;

__device__ __forceinline__ int mmf_swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

__device__ __forceinline__ uint32_t h2_bits(h2_t v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h2_t bits_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }
__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
    return uint32_t(float_to_half_bits(lo)) | (uint32_t(float_to_half_bits(hi)) << 16);
}

// Two fp16 codes from bytes (sel) of w, each 1024 + byte (fp16 bits 0x6400 | byte).
template <uint32_t SEL>
__device__ __forceinline__ h2_t magic_pair(uint32_t w) {
    return bits_h2(__builtin_amdgcn_perm(0x64646464u, w, SEL));
}
constexpr uint32_t SEL_B01 = 0x04010400u;  // bytes 0, 1 of w into the two low halves
constexpr uint32_t SEL_B23 = 0x04030402u;  // bytes 2, 3

// Weight loads are buffer loads (descriptor in SGPRs, 32-bit lane offset plus a uniform
// step offset) issued as instructions the compiler does not track, like the LDS DMAs:
// every operand of the software pipeline is in flight for two K steps and the kernel
// waits with explicit vmcnt counts (vector-memory operations complete in order). The
// loaded registers are tied to those waits, so nothing reads them earlier.
// The compiler cannot see inside these asm statements, so each carries the wait states
// the hardware requires before it: 5 after a VALU write of an SGPR it reads (the
// descriptors and offsets come from v_readfirstlane), and 1 between writing M0 and the
// LDS DMA that uses it.
// Descriptor of [p, p + bytes) from uniform values, kept in SGPRs (readfirstlane: values
// computed on the VALU would otherwise reach the asm operands in VGPRs).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t mmf_rsrc(const void *p, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    const uint64_t lo = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(a))));
    const uint64_t hi = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(a >> 32))));
    void *u = reinterpret_cast<void *>(lo | (hi << 32));
    return __builtin_amdgcn_make_buffer_rsrc(u, static_cast<short>(0), uint32_t(__builtin_amdgcn_readfirstlane(int(bytes))),
                                             0x00020000);
}
__device__ __forceinline__ u2_t mmf_load8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    u2_t v;
    __asm__ volatile("s_nop 4\n\tbuffer_load_dwordx2 %0, %1, %2, %3 offen" : "=v"(v) : "v"(voff), "s"(r), "s"(soff) : "memory");
    return v;
}
__device__ __forceinline__ u4_t mmf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    u4_t v;
    __asm__ volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(v) : "v"(voff), "s"(r), "s"(soff) : "memory");
    return v;
}
// Wait until at most N vector-memory operations of this wave are outstanding; the tied
// registers (loads issued before the N most recent operations) are valid afterwards.
template <int N>
__device__ __forceinline__ void mmf_wait() {
    __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void mmf_wait(u4_t (&q)[4]) {
    __asm__ volatile("s_waitcnt vmcnt(%4)" : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]) : "n"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void mmf_wait(u4_t (&q)[4], u4_t &h) {
    __asm__ volatile("s_waitcnt vmcnt(%5)" : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]), "+v"(h) : "n"(N) : "memory");
}
// 16 bytes per lane from base + voff to LDS at lds + 16 * lane.
__device__ __forceinline__ void mmf_dma16(const void *base, uint32_t voff, uint32_t lds) {
    __asm__ volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds)
                     : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

// Per-row constants of one superblock.
struct MmfRow {
    float unit;     // u = d * 2^P, the unit of this superblock's accumulation
    float scale2p;  // 2^-P, or 0 when the main term is dropped (d = 0 or negligible)
};

// Weight side per format.
template <int TYPE> struct MmfW;

// Q4_K (vecdotq.cuh:328-351): step c of a superblock covers blocks 2c (low nibbles of
// qs[32c, +32)) and 2c + 1 (high nibbles); lane group g takes qs[32c + 8g, +8).
template <> struct MmfW<Q4_K> {
    static constexpr int SBB = 144;  // superblock bytes
    static constexpr int TROW = 64;  // bytes per row of min-term operands (4 block pairs)
    // 6-bit scale and min of block b (0..7) from the 12 scale bytes (h.y, h.z, h.w). Both
    // layouts are computed and one is selected by bit arithmetic, so a block index that
    // differs between lanes costs no divergent branch.
    static __device__ uint32_t pick(uint32_t lo4, uint32_t hi4, int b) {
        const uint32_t m = 0u - uint32_t(b >> 2);  // all ones for blocks 4..7
        return (lo4 & ~m) | (hi4 & m);
    }
    static __device__ uint32_t sc(u4_t h, int b) {
        const uint32_t j = 8u * uint32_t(b & 3);
        return pick((h.y >> j) & 63u, ((h.w >> j) & 15u) | (((h.y >> (j + 6u)) & 3u) << 4), b);
    }
    static __device__ uint32_t mn(u4_t h, int b) {
        const uint32_t j = 8u * uint32_t(b & 3);
        return pick((h.z >> j) & 63u, ((h.w >> (j + 4u)) & 15u) | (((h.z >> (j + 6u)) & 3u) << 4), b);
    }
    // From the superblock header (d, dmin, scales): the unit u = d 2^P keeps
    // |e| = |dmin| m / |u| <= 64 * 63, with P = ceil(log2(|dmin| / (64 |d|))) when
    // positive. When that would exceed 20 (sc q 2^-P / 16 must stay a multiple of 2^-24,
    // exact in fp16), and for d = 0, the main term is dropped (it is then below 2^-21 of
    // the min term) and u = |dmin| / 64 (or 1).
    static __device__ MmfRow row(u4_t h) {  // branch-free: selects, no divergence
        const float d = half_bits_to_float(h.x & 0xffffu), dmin = half_bits_to_float(h.x >> 16);
        const float ad = fabsf(d), need = fabsf(dmin) * 0.015625f;  // smallest |u| keeping e in range
        // Smallest p with ad 2^p >= need when need > ad (1 <= p <= 20 where the main term
        // is kept), else 0: ad 2^p0 has need's binary exponent, one more doubling when its
        // mantissa is still below need's.
        int p = __builtin_amdgcn_frexp_expf(need) - __builtin_amdgcn_frexp_expf(ad);
        p += __builtin_amdgcn_ldexpf(ad, p) < need ? 1 : 0;
        p = need > ad ? p : 0;
        const bool drop = d == 0.0f || need > ad * 1048576.0f;
        MmfRow r;
        r.unit = drop ? (need > 0.0f ? need : 1.0f) : copysignf(__builtin_amdgcn_ldexpf(ad, p), d);
        r.scale2p = drop ? 0.0f : __builtin_bit_cast(float, uint32_t(127 - p) << 23);
        return r;
    }
    // Dequantisation constants of blocks b (even) and b + 1: fp16 pairs (mul, add) with
    // (1024 + q) mul + add = sc q 2^-P for the low nibble and (1024 + 16 q) mul + add the
    // same for the high one (one rounding of an exactly representable value).
    static __device__ u2_t consts(u4_t h, const MmfRow &r, int b) {
        const float s0 = float(sc(h, b)) * r.scale2p, s1 = float(sc(h, b + 1)) * r.scale2p;
        return u2_t{pack_h2(s0, -1024.0f * s0), pack_h2(s1 * 0.0625f, -64.0f * s1)};
    }
    // MFMA A operand of block 2c + b (b = 0: low nibbles, 1: high) from the lane's 8 code
    // bytes and that block's constant pair k = (mul, add).
    template <int B>
    static __device__ h8_t frag(u2_t q, uint32_t k) {
        const h2_t kk = bits_h2(k);
        const h2_t mul = h2_t{kk.x, kk.x}, add = h2_t{kk.y, kk.y};
        constexpr uint32_t MASK = B == 0 ? 0x0f0f0f0fu : 0xf0f0f0f0u;
        uint32_t v[4];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t w = (i == 0 ? q.x : q.y) & MASK;
            v[2 * i] = h2_bits(__builtin_elementwise_fma(magic_pair<SEL_B01>(w), mul, add));
            v[2 * i + 1] = h2_bits(__builtin_elementwise_fma(magic_pair<SEL_B23>(w), mul, add));
        }
        return __builtin_bit_cast(h8_t, u4_t{v[0], v[1], v[2], v[3]});
    }
    // Min-term weight operand of block pair g (blocks 2g, 2g + 1): fp16
    // [e_hi e_hi' e_hi e_hi' e_lo e_lo' f f'] with e = -dmin m / u = e_hi + e_lo and
    // f = -8 sc 2^-P; the activation operand (prepare_mmf_kernel) is
    // [t_hi t_hi' t_lo t_lo' t_hi t_hi' u8 u8'], so the MFMA's 8-value run of lane group g
    // sums e t + f u8 over the pair (t = t_hi + t_lo; the e_lo t_lo term is below 2^-22).
    static __device__ u4_t min_pair(u4_t h, const MmfRow &r, int g) {
        // -dmin / u to within 2 ulp (one reciprocal): e keeps 22 of its bits in hi + lo.
        const float ne = -half_bits_to_float(h.x >> 16) * __builtin_amdgcn_rcpf(r.unit);
        float e[2], fv[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            e[s] = ne * float(mn(h, 2 * g + s));
            fv[s] = -8.0f * float(sc(h, 2 * g + s)) * r.scale2p;
        }
        const uint32_t hb = pack_h2(e[0], e[1]);
        const uint32_t lb = pack_h2(e[0] - half_bits_to_float(hb & 0xffffu), e[1] - half_bits_to_float(hb >> 16));
        return u4_t{hb, hb, lb, pack_h2(fv[0], fv[1])};
    }
    // All four pairs of one row (64 bytes), the layout the GEMM keeps in LDS.
    static __device__ void min_row(u4_t h, const MmfRow &r, uint8_t *trow) {
#pragma unroll
        for (int g = 0; g < 4; ++g) *reinterpret_cast<u4_t *>(trow + 16 * g) = min_pair(h, r, g);
    }
};

template <int TYPE>
__global__ __launch_bounds__(MMF_THREADS, 2) void mmf_kernel(
    const uint8_t *weight, int64_t row_bytes, int n, int k, const uint16_t *a16, const uint8_t *tmin,
    const float *__restrict__ inverse, int m, void *__restrict__ dst, int64_t stride_dst, int dst_bf16,
    int tiles_m, int tiles_n) {
    using F = MmfW<TYPE>;
    constexpr int TROW = F::TROW;
    // Min-operand DMA: MT rows of TROW bytes, TROW / 16 chunks each, the same number of
    // whole instructions in every wave (surplus lanes re-fetch the final chunk into padding).
    constexpr int TCH = MMF_MT * TROW / 16, TINS = (TCH + 4 * 64 - 1) / (4 * 64), TCHP = TINS * 4 * 64;
    __shared__ __align__(16) uint8_t a16s[3][MMF_STAGE];  // activation stages of steps j, j+1, j+2
    __shared__ __align__(16) uint8_t tmins[TCHP * 16];
    __shared__ __align__(16) uint8_t wmin[MMF_NT * TROW];
    __shared__ __align__(16) u2_t wconst[2][MMF_NT][4];  // per superblock parity, row, block pair
    __shared__ __align__(16) float ratio[MMF_NT];

    // Tile: workgroups are dispatched round-robin over the 8 XCDs; give each XCD a
    // contiguous range of tiles, walked in groups of 8 activation tiles per weight tile
    // so that concurrent workgroups of one XCD share both operands in its L2.
    const int T = tiles_m * tiles_n;
    int lin = blockIdx.x;
    if ((T & 7) == 0) lin = (lin & 7) * (T >> 3) + (lin >> 3);
    constexpr int GROUP = 8;
    const int per_group = GROUP * tiles_n;
    const int first_m = (lin / per_group) * GROUP;
    const int gsize = min(tiles_m - first_m, GROUP);
    const int tm = first_m + (lin % per_group) % gsize, tn = (lin % per_group) / gsize;
    // Uniform by construction; readfirstlane keeps them (and the descriptors) in SGPRs.
    const int m0 = __builtin_amdgcn_readfirstlane(tm * MMF_MT), n0 = __builtin_amdgcn_readfirstlane(tn * MMF_NT);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, g = lane >> 4;
    const int swz_col = mmf_swz(col);
    const int nsb = k / 256, steps = k / MMF_KS;
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    // Buffer descriptors per weight tile of this wave (16 rows each) and for the
    // workgroup's rows: loads past the last weight row read zeros (the range check), so no
    // per-lane clamps; one lane offset serves all four tiles.
    auto tile_rsrc = [&](int t) {  // scalar work, rebuilt at each use rather than held
        const int r0 = n0 + 64 * wave_u + 16 * t;
        return mmf_rsrc(weight + int64_t(min(r0, n)) * row_bytes, uint32_t(max(0, min(16, n - r0))) * uint32_t(row_bytes));
    };
    const __amdgpu_buffer_rsrc_t hres =
        mmf_rsrc(weight + int64_t(n0) * row_bytes, uint32_t(min(MMF_NT, n - n0)) * uint32_t(row_bytes));

    // Weight operand role: row col of each tile, code bytes [16g, 16g + 16) of each half
    // superblock (steps 2p and 2p + 1 of its pair p).
    const uint32_t woff = uint32_t(col) * uint32_t(row_bytes) + 16u + 16u * g;
    // Row-constant role: thread tid prepares row n0 + tid (rows past n read zeros: d = 0).
    const uint32_t hoff = uint32_t(tid) * uint32_t(row_bytes);

    // Activation DMA: chunk q = (AINS wave + i) * 64 + lane of the MT * 8 per stage, LDS
    // row q / 8 at physical chunk q % 8, which holds logical chunk (q % 8) ^ swz(row).
    constexpr int AINS = MMF_STAGE / 16 / 64 / 4;  // DMA instructions per wave and stage
    static_assert(AINS * 4 * 64 * 16 == MMF_STAGE, "whole DMA instructions per stage");
    uint32_t aoff[AINS];
#pragma unroll
    for (int i = 0; i < AINS; ++i) {
        const int q = (AINS * wave + i) * 64 + lane, r = q >> 3;
        aoff[i] = uint32_t(min(m0 + r, m - 1)) * uint32_t(k) * 2u + uint32_t(((q & 7) ^ mmf_swz(r)) * 16);
    }

    auto issue_act = [&](int step, int st) {
        const uint8_t *base = reinterpret_cast<const uint8_t *>(a16) + size_t(step) * MMF_ROWB;
#pragma unroll
        for (int i = 0; i < AINS; ++i) mmf_dma16(base, aoff[i], lds_addr(&a16s[st][(AINS * wave_u + i) * 1024]));
    };
    auto issue_tmin = [&](int sb) {  // once per superblock: offsets computed here, not held
        const uint8_t *base = tmin + size_t(sb) * TROW;
#pragma unroll
        for (int i = 0; i < TINS; ++i) {
            int ln = lane;
            __asm__ volatile("" : "+v"(ln));  // keep the offset out of the loop-invariant set
            const int q = min((TINS * wave_u + i) * 64 + ln, TCH - 1);
            const int r = q / (TROW / 16), c = q % (TROW / 16);
            const uint32_t off = uint32_t(min(m0 + r, m - 1)) * uint32_t(nsb * TROW) + uint32_t(16 * c);
            mmf_dma16(base, off, lds_addr(&tmins[(TINS * wave_u + i) * 1024]));
        }
    };
    auto load_codes = [&](u4_t(&q)[4], int pair) {  // pair p of superblock s: index 2 s + p
        const uint32_t soff = uint32_t(pair >> 1) * F::SBB + 64u * uint32_t(pair & 1);
#pragma unroll
        for (int t = 0; t < 4; ++t) q[t] = mmf_load16(tile_rsrc(t), woff, soff);
    };
    auto write_consts = [&](u4_t h, const MmfRow &r, int buf) {
#pragma unroll
        for (int c = 0; c < 4; ++c) wconst[buf][tid][c] = F::consts(h, r, 2 * c);
    };

    v4f_t acc[4][MMF_MTILES];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < MMF_MTILES; ++b) acc[a][b] = v4f_t{0.0f, 0.0f, 0.0f, 0.0f};

    // Software pipeline, per wave and step j: 3 activation DMAs of step j + 2; at a
    // superblock's step 0 also the code loads of its steps 2-3, 2 min-operand DMAs and the
    // next header, at its step 2 the code loads of the next superblock's steps 0-1. The
    // end-of-step wait leaves only the current step's operations in flight, so step j + 1's
    // operands have landed (and, at the end of step 1, the header issued at step 0). Past
    // the last step the loads repeat it.
    constexpr int VM_ACT = AINS, VM_CODES = AINS + 4, VM_SB = VM_CODES + TINS + 1;
    u4_t codes[2][4];  // slot p holds pair p of the current superblock (16 bytes per tile)
    u4_t hdr = mmf_load16(hres, hoff, 0);
    issue_act(0, 0);
    load_codes(codes[0], 0);
    issue_act(min(1, steps - 1), 1);
    mmf_wait<VM_ACT>(codes[0], hdr);
    MmfRow rnext = F::row(hdr);  // constants of the superblock the next step 0 starts
    write_consts(hdr, rnext, 0);
    float unit_cur = 1.0f;
    __syncthreads();

    int st = 0;  // activation stage of the current step (step % 3)
    for (int sb = 0; sb < nsb; ++sb) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int step = 4 * sb + jj, nx2 = min(step + 2, steps - 1);
            const int st2 = st == 0 ? 2 : st - 1;  // (step + 2) % 3
            // hdr holds superblock sb's header here: its min-term operands, read at the end.
            if (jj == 0) {
                F::min_row(hdr, rnext, &wmin[tid * TROW]);
                unit_cur = rnext.unit;
            }
            issue_act(nx2, st2);
            if (jj == 0) {
                load_codes(codes[1], 2 * sb + 1);
                issue_tmin(sb);
                hdr = mmf_load16(hres, hoff, uint32_t(min(sb + 1, nsb - 1)) * F::SBB);
            } else if (jj == 2) {
                load_codes(codes[0], min(2 * sb + 2, 2 * nsb - 1));
            }

            const uint8_t *as = a16s[st];
            const int cpair = 2 * (jj >> 1) + (g >> 1);  // block pair of this lane group
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                // Weight operands: block 2 cpair + b, positions 16 (g & 1) + 8 (jj & 1) + [0, 8).
                h8_t wf[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const u4_t &pq = codes[jj >> 1][t];
                    const u2_t cq = (jj & 1) ? u2_t{pq.z, pq.w} : u2_t{pq.x, pq.y};
                    const uint32_t kc = reinterpret_cast<const uint32_t *>(&wconst[sb & 1][64 * wave + 16 * t + col][cpair])[b];
                    wf[t] = b == 0 ? F::template frag<0>(cq, kc) : F::template frag<1>(cq, kc);
                }
                const int pc = 16 * ((4 * b + g) ^ swz_col);
#pragma unroll
                for (int a = 0; a < MMF_MTILES; ++a) {
                    const h8_t af = *reinterpret_cast<const h8_t *>(as + (16 * a + col) * MMF_ROWB + pc);
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        acc[t][a] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[t], af, acc[t][a], 0, 0, 0);
                }
            }

            if (jj == 3) {  // superblock end: min terms, then rescale to the next unit
                h8_t mw[4];
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    mw[t] = *reinterpret_cast<const h8_t *>(&wmin[(64 * wave + 16 * t + col) * TROW + 16 * g]);
#pragma unroll
                for (int a = 0; a < MMF_MTILES; ++a) {
                    const h8_t mt = *reinterpret_cast<const h8_t *>(&tmins[(16 * a + col) * TROW + 16 * g]);
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        acc[t][a] = __builtin_amdgcn_mfma_f32_16x16x32_f16(mw[t], mt, acc[t][a], 0, 0, 0);
                }
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const v4f_t rv = *reinterpret_cast<const v4f_t *>(&ratio[64 * wave + 16 * t + 4 * g]);
#pragma unroll
                    for (int a = 0; a < MMF_MTILES; ++a) acc[t][a] *= rv;
                }
            }

            if (jj == 2) {  // the header of superblock sb + 1 landed at the end of step 1
                if (sb + 1 < nsb) {
                    rnext = F::row(hdr);
                    write_consts(hdr, rnext, (sb + 1) & 1);
                    ratio[tid] = unit_cur * __builtin_amdgcn_rcpf(rnext.unit);  // within 2 ulp
                } else {
                    ratio[tid] = unit_cur;
                }
            }
            // Step j + 1's operands have landed; only this step's operations stay in flight.
            if (jj == 0)
                mmf_wait<VM_SB>();
            else if (jj == 1)
                mmf_wait<VM_ACT>(codes[1], hdr);
            else if (jj == 2)
                mmf_wait<VM_CODES>();
            else
                mmf_wait<VM_ACT>(codes[0]);
            __syncthreads();
            st = st == 2 ? 0 : st + 1;
        }
    }
    // No DMA may land in LDS after the workgroup ends.
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // Store Y[m][n .. n+3] = acc * inverse[m]; lane indices re-derived here, not kept
    // live through the loop.
    int ln = lane;
    __asm__ volatile("" : "+v"(ln));
    const int ecol = ln & 15, eg = ln >> 4;
#pragma unroll
    for (int a = 0; a < MMF_MTILES; ++a) {
        const int row = m0 + 16 * a + ecol;
        if (row >= m) continue;
        const float inv = inverse[row];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int c0 = n0 + 64 * wave_u + 16 * t + 4 * eg;
            if (c0 >= n) continue;
            const v4f_t v = acc[t][a] * inv;
            if (dst_bf16) {
                const uint32_t lo = uint32_t(float_to_bf16_bits(v[0])) | (uint32_t(float_to_bf16_bits(v[1])) << 16);
                const uint32_t hi = uint32_t(float_to_bf16_bits(v[2])) | (uint32_t(float_to_bf16_bits(v[3])) << 16);
                *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(dst) + int64_t(row) * stride_dst + c0) = make_uint2(lo, hi);
            } else {
                *reinterpret_cast<v4f_t *>(static_cast<float *>(dst) + int64_t(row) * stride_dst + c0) = v;
            }
        }
    }
}

template <int TYPE>
void launch_mmf_type(const void *weight, int64_t n, int64_t k, int64_t m, const MmfAct &act, void *dst,
                     bool dst_bf16, int64_t stride_dst, hipStream_t stream) {
    const int tiles_m = static_cast<int>((m + MMF_MT - 1) / MMF_MT);
    const int tiles_n = static_cast<int>((n + MMF_NT - 1) / MMF_NT);
    const uint8_t *tmin = mmf_uses_t32(TYPE) ? act.t32 : act.t16;
    if (!tmin) throw Error("fp16-MFMA GEMM: min-term operands were not prepared");
    mmf_kernel<TYPE><<<dim3(unsigned(tiles_m) * unsigned(tiles_n)), dim3(MMF_THREADS), 0, stream>>>(
        static_cast<const uint8_t *>(weight), (k / 256) * MmfW<TYPE>::SBB, static_cast<int>(n),
        static_cast<int>(k), act.a16, tmin, act.inverse, static_cast<int>(m), dst, stride_dst, dst_bf16 ? 1 : 0,
        tiles_m, tiles_n);
}

}  // namespace kai
