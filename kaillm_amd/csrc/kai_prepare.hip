// Q8_1 activation preparation (kernel "prepare"): exact per-row power-of-two
// normalisation followed by Q8_1 quantisation of every 32-value block.
//
// Follows kai_dual::prepare_dual (vllm_gguf_plugin/native/kernels/kai_dual_mmvq.cuh:147-254):
//   amax = max |x| over the row; e = biased exponent of amax;
//   se = clamp(260 - e, 1, 253) when 0 < e < 255, else 127;
//   scale = 2^(se - 127) puts amax into [64, 128); inverse[row] = 2^(127 - se);
//   per block: v = x * scale, a = max|v|, d = a / 127, q = a == 0 ? 0 : roundf(v / d),
//   ds = (half_rn(d), half_rn(d * sum q)).
//   two_pass adds a second block quantising v - half(d) * q (one fused multiply-add).
// Division is IEEE (hipcc's default correctly rounded fp32 divide), so the
// bytes are identical to the CPU restatement.
//
// Launch: workgroups of 256 lanes, four lanes per 32-value block (8 values each), so
// 64 blocks per workgroup and several workgroups per row; every workgroup of a row
// reads the whole row for its maximum (L2-resident, a few KiB), which keeps the row
// scale without a second launch, and the per-block maximum and code sum are quad
// (DPP) reductions. The arithmetic per value is unchanged.
#include "kai_launch.h"

// Every rounding step must be the one the reference spells out. No floating-point
// contraction in this file; see quad_store for the fp16 conversion of d * sum.
#pragma clang fp contract(off)

namespace kai {

constexpr int PREP_MAX_BLOCKS = 1024;  // K <= 32768 (the reference's limit)

// Codes of one 32-value block: q = roundf(v / d) with d = max|v| / 127 (fp32), and the
// stored fp16 d (quad_codes).
struct BlockCodes {
    float d;      // fp32 scale the codes were rounded with
    uint16_t hd;  // its fp16 bits, the block's stored scale
    int isum;     // sum of the codes
};
// Row scale from the row maximum: returns scale, writes inverse through lane 0.
__device__ __forceinline__ float row_scale_from_max(float amax, float *inverse_out, bool writer) {
    const int biased = static_cast<int>((__builtin_bit_cast(uint32_t, amax) >> 23) & 255u);
    int se = 127;
    if (biased != 0 && biased != 255) se = min(max(260 - biased, 1), 253);
    if (writer) *inverse_out = __builtin_bit_cast(float, static_cast<uint32_t>(254 - se) << 23);
    return __builtin_bit_cast(float, static_cast<uint32_t>(se) << 23);
}

// Block-wide maximum over up to 16 waves; all lanes get the result.
__device__ __forceinline__ float block_max(float v, float *lds) {
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    v = wave_max(v);
    if (lane == 0) lds[wave] = v;
    __syncthreads();
    const int nwaves = (blockDim.x + WAVE - 1) / WAVE;
    float m = 0.0f;
    for (int w = 0; w < nwaves; ++w) m = fmaxf(m, lds[w]);
    return m;
}

constexpr int PREP_THREADS = 256;
constexpr int PREP_BLOCKS = PREP_THREADS / 4;  // 32-value blocks per workgroup

// 8 consecutive source values as float.
template <int DTYPE>
__device__ __forceinline__ void load8(const typename Src<DTYPE>::T *p, float (&v)[8]) {
    if constexpr (DTYPE == 0) {
        const float4 a = load_unaligned<float4>(p), b = load_unaligned<float4>(p + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        const uint4 u = load_unaligned<uint4>(p);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = DTYPE == 1 ? bf16_bits_to_float(w[i] & 0xffffu) : half_bits_to_float(w[i] & 0xffffu);
            v[2 * i + 1] = DTYPE == 1 ? bf16_bits_to_float(w[i] >> 16) : half_bits_to_float(w[i] >> 16);
        }
    }
}

// Reductions over the four lanes of a block (every lane gets the same result).
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ float quad_max(float v) {
    v = fmaxf(v, dpp_f32<DPP_QUAD_1032>(v));
    return fmaxf(v, dpp_f32<DPP_QUAD_2301>(v));
}
__device__ __forceinline__ int quad_sum(int v) {
    v += dpp_i32<DPP_QUAD_1032>(v);
    return v + dpp_i32<DPP_QUAD_2301>(v);
}
__device__ __forceinline__ float quad_sum(float v) {
    v += dpp_f32<DPP_QUAD_1032>(v);  // (v0 + v1) + (v2 + v3) in every lane
    return v + dpp_f32<DPP_QUAD_2301>(v);
}

// 8 consecutive source values as loaded (two float4 for fp32, one uint4 of 16-bit values),
// and their conversion to float (load8 split in two, so loads can be issued back to back).
template <int DTYPE>
struct Raw8 {
    uint4 a, b;  // b unused for 16-bit sources
};
template <int DTYPE>
__device__ __forceinline__ void load_raw8(const typename Src<DTYPE>::T *p, Raw8<DTYPE> &r) {
    if constexpr (DTYPE == 0) {
        r.a = load_unaligned<uint4>(p);
        r.b = load_unaligned<uint4>(p + 4);
    } else {
        r.a = load_unaligned<uint4>(p);
    }
}
template <int DTYPE>
__device__ __forceinline__ void convert8(const Raw8<DTYPE> &r, float (&v)[8]) {
    const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
    if constexpr (DTYPE == 0) {
        const uint32_t x[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = __builtin_bit_cast(float, w[i]);
            v[4 + i] = __builtin_bit_cast(float, x[i]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = DTYPE == 1 ? bf16_bits_to_float(w[i] & 0xffffu) : half_bits_to_float(w[i] & 0xffffu);
            v[2 * i + 1] = DTYPE == 1 ? bf16_bits_to_float(w[i] >> 16) : half_bits_to_float(w[i] >> 16);
        }
    }
}

// Maximum |x| of the thread's runs of a row (run p by thread p % PREP_THREADS), ROUND runs
// at a time: the round's loads are issued back to back (indices clamped to the last run,
// whose values are then ignored) before the first maximum. The run with index
// blockIdx.y * PREP_THREADS + threadIdx.x is kept in `own`.
template <int DTYPE, int ROUND>
__device__ __forceinline__ float row_max(const typename Src<DTYPE>::T *xr, int runs, float (&own)[8]) {
    float mx = 0.0f;
    for (int i0 = 0; i0 * PREP_THREADS < runs; i0 += ROUND) {
        Raw8<DTYPE> r[ROUND];
#pragma unroll
        for (int u = 0; u < ROUND; ++u)
            load_raw8<DTYPE>(xr + 8 * min(int(threadIdx.x) + (i0 + u) * PREP_THREADS, runs - 1), r[u]);
#pragma unroll
        for (int u = 0; u < ROUND; ++u) {
            float v[8];
            convert8<DTYPE>(r[u], v);
            if (int(threadIdx.x) + (i0 + u) * PREP_THREADS < runs) {
#pragma unroll
                for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(v[j]));
            }
            if (i0 + u == int(blockIdx.y)) {  // uniform
#pragma unroll
                for (int j = 0; j < 8; ++j) own[j] = v[j];
            }
        }
    }
    return mx;
}

// Scale of a row from its maximum |x|, read by every workgroup of the row. The run this
// workgroup's thread quantises (blockIdx.y * PREP_THREADS + threadIdx.x: 4 lanes per block,
// PREP_BLOCKS blocks per workgroup) is kept in `own`, so the values are read once (when that
// run is past the row end the thread stores nothing). Rows of up to 8192 values take one
// round of 4 runs per thread; longer rows rounds of 12 (one wait on memory up to 24576).
template <int DTYPE>
__device__ __forceinline__ float row_scale(const typename Src<DTYPE>::T *xr, int k, float *lds, float *inverse_out,
                                           bool writer, float (&own)[8]) {
    const int runs = k / 8;
    const float mx = runs <= 4 * PREP_THREADS ? row_max<DTYPE, 4>(xr, runs, own) : row_max<DTYPE, 12>(xr, runs, own);
    return row_scale_from_max(block_max(mx, lds), inverse_out, writer);
}
static_assert(PREP_THREADS == 4 * PREP_BLOCKS, "one run of 8 values per thread and workgroup");

// Codes of the lane's 8 values of one block: d = max|v| / 127 over the block (quad),
// q = roundf(v / d); returns the fp32 d, the stored fp16 bits and the block's code sum.
__device__ __forceinline__ BlockCodes quad_codes(const float (&v)[8], int8_t (&q)[8]) {
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) a = fmaxf(a, fabsf(v[j]));
    a = quad_max(a);
    BlockCodes b;
    b.d = a / 127.0f;
    int s = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        q[j] = static_cast<int8_t>(a == 0.0f ? 0.0f : roundf(v[j] / b.d));
        s += q[j];
    }
    b.isum = quad_sum(s);
    b.hd = float_to_half_bits(b.d);
    return b;
}

// The quad's share of one Q8_1 block: part 0 writes ds = (hd, hs), each part its 8 codes.
__device__ __forceinline__ void quad_write(block_q8_1 *out, int part, uint16_t hd, uint16_t hs, const int8_t (&q)[8]) {
    uint32_t *w = reinterpret_cast<uint32_t *>(out);
    if (part == 0) w[0] = static_cast<uint32_t>(hd) | (static_cast<uint32_t>(hs) << 16);
#pragma unroll
    for (int i = 0; i < 2; ++i)
        w[1 + 2 * part + i] = static_cast<uint32_t>(static_cast<uint8_t>(q[4 * i])) |
                              (static_cast<uint32_t>(static_cast<uint8_t>(q[4 * i + 1])) << 8) |
                              (static_cast<uint32_t>(static_cast<uint8_t>(q[4 * i + 2])) << 16) |
                              (static_cast<uint32_t>(static_cast<uint8_t>(q[4 * i + 3])) << 24);
}

// One Q8_1 block from the four lanes of a quad: part 0 writes (d, d * sum), each part
// its 8 codes. Returns the stored fp16 d.
__device__ __forceinline__ float quad_store(const float (&v)[8], block_q8_1 *out, int part, int8_t (&q)[8]) {
    const BlockCodes b = quad_codes(v, q);
    // half(d * sum) rounds the product to fp32 first, then to fp16 (no fused conversion).
    float prod = b.d * static_cast<float>(b.isum);
    __asm__ volatile("" : "+v"(prod));
    quad_write(out, part, b.hd, float_to_half_bits(prod), q);
    return half_bits_to_float(b.hd);
}

template <int DTYPE, bool TWO_PASS>
__global__ __launch_bounds__(PREP_THREADS) void prepare_q8_1_kernel(
    const typename Src<DTYPE>::T *__restrict__ x, int64_t stride_x, int k, block_q8_1 *__restrict__ y1,
    block_q8_1 *__restrict__ y2, float *__restrict__ inverse) {
    __shared__ float wave_max_lds[PREP_THREADS / WAVE];
    const int row = blockIdx.x;
    const int nblocks = k / QK8_1;
    const int part = threadIdx.x & 3, ib = blockIdx.y * PREP_BLOCKS + (threadIdx.x >> 2);
    const auto *xr = x + static_cast<int64_t>(row) * stride_x;
    float v[8];
    const float scale = row_scale<DTYPE>(xr, k, wave_max_lds, inverse + row, blockIdx.y == 0 && threadIdx.x == 0, v);
    if (ib >= nblocks) return;  // whole quads
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] *= scale;
    int8_t q1[8];
    const float d1h = quad_store(v, y1 + static_cast<int64_t>(row) * nblocks + ib, part, q1);
    if constexpr (TWO_PASS) {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = fmaf(-d1h, static_cast<float>(q1[j]), v[j]);
        int8_t q2[8];
        quad_store(v, y2 + static_cast<int64_t>(row) * nblocks + ib, part, q2);
    }
}

// ---------------------------------------------------------------- legacy activation
// quantize_q8_1 of the legacy _C_gguf ops (vllm_gguf_plugin/csrc/gguf/gguf_kernel.cu:32-69):
// no row normalisation; per 32 values d = max|x| / 127 and q = roundf(x / d) as in
// quad_codes, ds = (half(d), half(sum x)). The reference adds sum x with a 32-lane xor
// butterfly; lane 0's sum is pass h = 16, 8, 4, 2, 1 adding value i + h to value i (i < h).
// Lane `part` of a quad holds values 8 part .. 8 part + 7, so passes 16 and 8 pair it with
// lanes part ^ 2 and part ^ 1 (values i + 16 and i + 8), and passes 4, 2, 1 stay in the
// lane. Every lane of the quad ends with the same sum (fp32 addition is commutative).
__device__ __forceinline__ float legacy_block_sum(const float (&v)[8]) {
    float t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) t[j] = v[j] + dpp_f32<DPP_QUAD_2301>(v[j]);
#pragma unroll
    for (int j = 0; j < 8; ++j) t[j] = t[j] + dpp_f32<DPP_QUAD_1032>(t[j]);
#pragma unroll
    for (int j = 0; j < 4; ++j) t[j] = t[j] + t[j + 4];
    t[0] = t[0] + t[2];
    t[1] = t[1] + t[3];
    return t[0] + t[1];
}

// Legacy block of the quad: codes, fp16 d and fp16 sum x.
struct LegacyBlock {
    int8_t q[8];
    uint16_t hd, hs;
};
__device__ __forceinline__ LegacyBlock legacy_block(const float (&v)[8]) {
    LegacyBlock b;
    b.hd = quad_codes(v, b.q).hd;
    b.hs = float_to_half_bits(legacy_block_sum(v));
    return b;
}

// Launch as prepare_q8_1_kernel; inverse[row] = 1 (no normalisation to undo).
template <int DTYPE>
__global__ __launch_bounds__(PREP_THREADS) void prepare_legacy_kernel(const typename Src<DTYPE>::T *__restrict__ x,
                                                                      int64_t stride_x, int k,
                                                                      block_q8_1 *__restrict__ y,
                                                                      float *__restrict__ inverse) {
    const int row = blockIdx.x;
    const int nblocks = k / QK8_1;
    const int part = threadIdx.x & 3, ib = blockIdx.y * PREP_BLOCKS + (threadIdx.x >> 2);
    if (blockIdx.y == 0 && threadIdx.x == 0) inverse[row] = 1.0f;
    if (ib >= nblocks) return;  // whole quads
    float v[8];
    load8<DTYPE>(x + static_cast<int64_t>(row) * stride_x + QK8_1 * ib + 8 * part, v);
    const LegacyBlock b = legacy_block(v);
    quad_write(y + static_cast<int64_t>(row) * nblocks + ib, part, b.hd, b.hs, b.q);
}

template <int DTYPE>
static void launch_prepare_legacy_dtype(const void *x, int64_t m, int64_t k, int64_t stride_x, const ActLayout &o,
                                        hipStream_t stream) {
    const int64_t nblocks = k / QK8_1;
    const dim3 grid(static_cast<unsigned>(m), static_cast<unsigned>((nblocks + PREP_BLOCKS - 1) / PREP_BLOCKS));
    prepare_legacy_kernel<DTYPE><<<grid, dim3(PREP_THREADS), 0, stream>>>(
        static_cast<const typename Src<DTYPE>::T *>(x), stride_x, static_cast<int>(k), o.y1, o.inverse);
}

void launch_prepare_legacy(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x, const ActLayout &out,
                           hipStream_t stream) {
    if (k <= 0 || k % QK8_1 || k / QK8_1 > int64_t(PREP_BLOCKS) * 65535 || m <= 0 || m > INT_MAX)
        throw Error("Invalid legacy activation shape");
    switch (x_dtype) {
        case 0: launch_prepare_legacy_dtype<0>(x, m, k, stride_x, out, stream); break;
        case 1: launch_prepare_legacy_dtype<1>(x, m, k, stride_x, out, stream); break;
        case 2: launch_prepare_legacy_dtype<2>(x, m, k, stride_x, out, stream); break;
        default: throw Error("Legacy activations must be F32, BF16 or F16");
    }
}

// ---------------------------------------------------------------- batched path (m > 8)
// GGML MMQ quantisation of the normalised row (quantize_scaled,
// current_ggml_direct.cu:1025-1092), per group of G values (G = 32: one quad; G = 64: two
// quads, joined by one lane exchange): amax = max|v|, d_inv = 127 / amax,
// q = roundf(v * d_inv) (NaN -> 0, saturated to int8: the reference's char conversion),
// d = 1 / d_inv. Both divisions are IEEE (correctly rounded). Returns d; q and the lane's
// code sum are written.
__device__ __forceinline__ int mmq_code(float p) {
    const float r = fminf(fmaxf(roundf(p), -128.0f), 127.0f);
    return p != p ? 0 : static_cast<int>(r);
}
template <int G>
__device__ __forceinline__ float mmq_group_codes(const float (&v)[8], int8_t (&q)[8], int &lane_sum) {
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) a = fmaxf(a, fabsf(v[j]));
    a = quad_max(a);
    if constexpr (G == 64) a = fmaxf(a, __shfl_xor(a, 4, WAVE));
    const float d_inv = 127.0f / a;
    int s = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int c = mmq_code(v[j] * d_inv);
        q[j] = static_cast<int8_t>(c);
        s += c;
    }
    lane_sum = s;
    return 1.0f / d_inv;
}
// fp16 bits of d * s, the product rounded to fp32 first (no fused conversion).
__device__ __forceinline__ uint32_t half_of_product(float d, int s) {
    float prod = d * static_cast<float>(s);
    __asm__ volatile("" : "+v"(prod));
    return float_to_half_bits(prod);
}
__device__ __forceinline__ uint2 pack_codes(const int8_t (&q)[8]) {
    uint32_t w[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
        w[i] = static_cast<uint32_t>(static_cast<uint8_t>(q[4 * i])) |
               (static_cast<uint32_t>(static_cast<uint8_t>(q[4 * i + 1])) << 8) |
               (static_cast<uint32_t>(static_cast<uint8_t>(q[4 * i + 2])) << 16) |
               (static_cast<uint32_t>(static_cast<uint8_t>(q[4 * i + 3])) << 24);
    return make_uint2(w[0], w[1]);
}

// Activation planes of the batched path: 128-value blocks of 144 bytes
// (block_q8_1_mmq: 16 header bytes, int8 qs[128]) in [K/128][m] order, K padded to
// MMQ_ROW_PADDING with zero blocks; the header per layout is
//   D4   fp32 d of each 32 values;
//   DS4  half2 (d, d * sum q) of each 32 values;
//   D2S6 half d of each 64 values, then half d * sum q of the 16-value groups 0..5.
// The row scale and inverse are those of prepare_q8_1_kernel (same launch shape, same
// arithmetic), and one launch writes every plane the group needs (null when absent).
// One lane's share of the small-M images (layout in kai_launch.h): octet `part` of block ib
// of row r, quantised as for the planes; lane 0 of the quad (of each 16-value pair for
// D2S6) writes the block's scale and terms, which are the values the planes' headers
// decode to.
__device__ __forceinline__ void mmqs_image_lane(const MmqPlanes &p, int ib, int r, int part, const float (&v)[8]) {
    const size_t step = static_cast<size_t>(ib >> 3);
    const int b = ib & 7;
    const int code_at = (b * 16 + r) * 32 + 8 * (part ^ ((r >> 2) & 3));
    const int word_at = MMQS_CODE_BYTES + (b * 16 + r) * 4;
    if (p.d4 || p.ds4) {
        int8_t q[8];
        int s;
        const float d = mmq_group_codes<32>(v, q, s);
        const uint2 packed = pack_codes(q);
        const int total = quad_sum(s);
        if (p.d4) {
            uint8_t *img = p.d4 + step * mmqs_image_step(MMQ_D4);
            *reinterpret_cast<uint2 *>(img + code_at) = packed;
            if (part == 0) *reinterpret_cast<float *>(img + word_at) = d;
        }
        if (p.ds4) {
            uint8_t *img = p.ds4 + step * mmqs_image_step(MMQ_DS4);
            *reinterpret_cast<uint2 *>(img + code_at) = packed;
            if (part == 0) {
                const float dh = half_bits_to_float(float_to_half_bits(d));
                float *w = reinterpret_cast<float *>(img + word_at);
                w[0] = dh;
                w[MMQS_D8_BYTES / 4] = half_bits_to_float(static_cast<uint16_t>(half_of_product(d, total)));
                w[MMQS_D8_BYTES / 2] = dh * static_cast<float>(total);
            }
        }
    }
    if (p.d2s6) {
        int8_t q[8];
        int s;
        const float d = mmq_group_codes<64>(v, q, s);
        uint8_t *img = p.d2s6 + step * mmqs_image_step(MMQ_D2S6);
        *reinterpret_cast<uint2 *>(img + code_at) = pack_codes(q);
        const int s16 = s + dpp_i32<DPP_QUAD_1032>(s);  // lanes {0,1} and {2,3}: 16 values each
        const float dh = half_bits_to_float(float_to_half_bits(d));
        if (part == 0) *reinterpret_cast<float *>(img + word_at) = dh;
        if ((part & 1) == 0) {
            const int g = 2 * b + (part >> 1);
            const float t = (b & 3) < 3 ? half_bits_to_float(static_cast<uint16_t>(half_of_product(d, s16)))
                                        : dh * static_cast<float>(s16);
            *reinterpret_cast<float *>(img + MMQS_CODE_BYTES + MMQS_D8_BYTES + (g * 16 + r) * 4) = t;
        }
    }
}

// The legacy quantisation (legacy_block) into the D4 / DS4 planes or small-M images, for
// the legacy ops' batched product: D4 holds the stored fp16 d as fp32 (the legacy MMQ reads
// d8 from the block's half2 ds), DS4 the half2 (d, sum x), and the DS4 image's two min-term
// factors (Q4_K, Q4_0) are both the stored half(sum x) (vecdotq.cuh:46-66, :353-377).
__device__ __forceinline__ void legacy_mmq_lane(const MmqPlanes &p, int ib, int row, int m, int part, int k,
                                                const float (&v)[8]) {
    if (p.image && ib >= 8 * static_cast<int>(mmqs_steps(k))) return;  // whole quads
    const LegacyBlock b = legacy_block(v);
    const uint2 packed = pack_codes(b.q);
    const float dh = half_bits_to_float(b.hd);
    if (p.image) {
        const size_t step = static_cast<size_t>(ib >> 3);
        const int bb = ib & 7;
        const int code_at = (bb * 16 + row) * 32 + 8 * (part ^ ((row >> 2) & 3));
        const int word_at = MMQS_CODE_BYTES + (bb * 16 + row) * 4;
        if (p.d4) {
            uint8_t *img = p.d4 + step * mmqs_image_step(MMQ_D4);
            *reinterpret_cast<uint2 *>(img + code_at) = packed;
            if (part == 0) *reinterpret_cast<float *>(img + word_at) = dh;
        }
        if (p.ds4) {
            uint8_t *img = p.ds4 + step * mmqs_image_step(MMQ_DS4);
            *reinterpret_cast<uint2 *>(img + code_at) = packed;
            if (part == 0) {
                float *w = reinterpret_cast<float *>(img + word_at);
                w[0] = dh;
                w[MMQS_D8_BYTES / 4] = half_bits_to_float(b.hs);
                w[MMQS_D8_BYTES / 2] = half_bits_to_float(b.hs);
            }
        }
        return;
    }
    const int sub = ib & 3;
    const size_t blk = (static_cast<size_t>(ib >> 2) * static_cast<size_t>(m) + static_cast<size_t>(row)) * MMQ_BLOCK_BYTES;
    const size_t codes = blk + 16 + 32 * sub + 8 * part;
    if (p.d4) {
        *reinterpret_cast<uint2 *>(p.d4 + codes) = packed;
        if (part == 0) *reinterpret_cast<float *>(p.d4 + blk + 4 * sub) = dh;
    }
    if (p.ds4) {
        *reinterpret_cast<uint2 *>(p.ds4 + codes) = packed;
        if (part == 0)
            *reinterpret_cast<uint32_t *>(p.ds4 + blk + 4 * sub) =
                static_cast<uint32_t>(b.hd) | (static_cast<uint32_t>(b.hs) << 16);
    }
}

// One lane's 8 values of block ib in the fp16 GEMM's image (layout in kai_launch.h): the
// dequantised activation d * q of each code, the product rounded to fp32 then to fp16; 16-value
// group 2 ib + part / 2, half part % 2.
__device__ __forceinline__ void mmqh_codes_lane(const MmqhImage &h, int mpad, int ib, int row, int part,
                                                const int8_t (&q)[8], float d) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = half_of_product(d, q[2 * i]) | (half_of_product(d, q[2 * i + 1]) << 16);
    const size_t at = ((static_cast<size_t>(2 * ib + (part >> 1)) * mpad + row) * 16 + 8 * (part & 1)) * 2;
    *reinterpret_cast<uint4 *>(h.codes + at) = make_uint4(w[0], w[1], w[2], w[3]);
}
// high and low fp16 parts of an fp32 value: hi = half(v), lo = half(v - hi)
__device__ __forceinline__ uint32_t half_hi(float v) { return float_to_half_bits(v); }
__device__ __forceinline__ uint32_t half_lo(float v) { return float_to_half_bits(v - half_bits_to_float(half_hi(v))); }

// LEGACY: the legacy ops' quantisation (no row normalisation, inverse 1, legacy_mmq_lane).
// One chunk's share of a lane: block ib of the row, values 8 part .. 8 part + 7 (v, before the
// row scale), into every plane and image the group reads.
template <bool LEGACY>
__device__ __forceinline__ void prepare_mmq_chunk(const MmqPlanes &p, float (&v)[8], float scale, int ib, int row,
                                                  int part, int k, int m, int nblocks, int kpad_blocks, int hblocks,
                                                  int mpad) {
    if (ib >= kpad_blocks) return;  // whole groups of 8 lanes (kpad_blocks is a multiple of 16)
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = ib < nblocks ? v[j] * scale : 0.0f;
    if constexpr (LEGACY) {
        legacy_mmq_lane(p, ib, row, m, part, k, v);
        return;
    }
    if (p.image) {
        if (ib >= 8 * static_cast<int>(mmqs_steps(k))) return;  // whole groups of 8 lanes
        mmqs_image_lane(p, ib, row, part, v);
        return;
    }
    const int sub = ib & 3;  // 32-value block within the 128-value block
    const size_t blk = (static_cast<size_t>(ib >> 2) * static_cast<size_t>(m) + static_cast<size_t>(row)) * MMQ_BLOCK_BYTES;
    const size_t codes = blk + 16 + 32 * sub + 8 * part;
    const bool plane_row = row < m;  // rows past m exist only in the fp16 images (zeros)
    // fp16 images: codes and scale records to K padded to 64, min operands to whole superblocks
    const bool h_block = ib < hblocks, h_min = ib < 8 * ((k + 255) / 256);
    if (p.d4 || p.ds4 || p.h[MMQ_D4].codes || p.h[MMQ_DS4].codes) {
        int8_t q[8];
        int s;
        const float d = mmq_group_codes<32>(v, q, s);
        const uint2 packed = pack_codes(q);
        const int total = quad_sum(s);
        if (p.d4 && plane_row) {
            *reinterpret_cast<uint2 *>(p.d4 + codes) = packed;
            if (part == 0) *reinterpret_cast<float *>(p.d4 + blk + 4 * sub) = d;
        }
        if (p.ds4 && plane_row) {
            *reinterpret_cast<uint2 *>(p.ds4 + codes) = packed;
            if (part == 0)
                *reinterpret_cast<uint32_t *>(p.ds4 + blk + 4 * sub) =
                    static_cast<uint32_t>(float_to_half_bits(d)) | (half_of_product(d, total) << 16);
        }
        if (const MmqhImage &h = p.h[MMQ_DS4]; h.codes && h_min && part == 0) {
            // [S_0..7 | Xhi_0..7 | Xlo_0..7 | 0 x 8]: the stored sum, and the exact sum half(d) * sum q
            uint16_t *mn = reinterpret_cast<uint16_t *>(h.mins + (static_cast<size_t>(ib >> 3) * mpad + row) * 64);
            const float x = half_bits_to_float(float_to_half_bits(d)) * static_cast<float>(total);
            mn[ib & 7] = static_cast<uint16_t>(half_of_product(d, total));
            mn[8 + (ib & 7)] = static_cast<uint16_t>(half_hi(x));
            mn[16 + (ib & 7)] = static_cast<uint16_t>(half_lo(x));
            mn[24 + (ib & 7)] = 0;
        }
        if (h_block) {
            if (const MmqhImage &h = p.h[MMQ_D4]; h.codes) mmqh_codes_lane(h, mpad, ib, row, part, q, d);
            if (const MmqhImage &h = p.h[MMQ_DS4]; h.codes)
                mmqh_codes_lane(h, mpad, ib, row, part, q, half_bits_to_float(float_to_half_bits(d)));
        }
    }
    if (p.d2s6 || p.h[MMQ_D2S6].codes) {
        int8_t q[8];
        int s;
        const float d = mmq_group_codes<64>(v, q, s);
        const int s16 = s + dpp_i32<DPP_QUAD_1032>(s);  // lanes {0,1} and {2,3}: 16 values each
        const int slot = 2 * sub + (part >> 1);
        if (p.d2s6 && plane_row) {
            *reinterpret_cast<uint2 *>(p.d2s6 + codes) = pack_codes(q);
            uint16_t *hdr = reinterpret_cast<uint16_t *>(p.d2s6 + blk);
            if ((part & 1) == 0 && slot < 6) hdr[2 + slot] = static_cast<uint16_t>(half_of_product(d, s16));
            if ((sub & 1) == 0 && part == 0) hdr[sub >> 1] = float_to_half_bits(d);
        }
        if (const MmqhImage &h = p.h[MMQ_D2S6]; h.codes) {
            const float dh = half_bits_to_float(float_to_half_bits(d));
            if (h_block) mmqh_codes_lane(h, mpad, ib, row, part, q, dh);
            if (h_min && (part & 1) == 0) {
                // [Shi | Slo | Xhi | Xlo] per 16-value group: the stored half sums (d * sum q for the
                // last 32 values of each 128), and the exact sums half(d) * sum q
                const float sum = slot < 6 ? half_bits_to_float(half_of_product(d, s16)) : dh * static_cast<float>(s16);
                const float x = dh * static_cast<float>(s16);
                uint16_t *mn = reinterpret_cast<uint16_t *>(h.mins + (static_cast<size_t>(ib >> 3) * mpad + row) * 128);
                const int g = 2 * (ib & 7) + (part >> 1);
                mn[g] = static_cast<uint16_t>(half_hi(sum));
                mn[16 + g] = static_cast<uint16_t>(half_lo(sum));
                mn[32 + g] = static_cast<uint16_t>(half_hi(x));
                mn[48 + g] = static_cast<uint16_t>(half_lo(x));
            }
        }
    }
}

// One workgroup per row (many rows): the thread loads its R runs of the row at once (run u
// of thread t is run t + 256 u, the thread's run of chunk u), takes the row maximum from
// them (and from the rest of a row longer than 2048 R values) and converts each chunk from
// the kept values, so the row is read once (the runs of chunks from R on are read again).
template <int DTYPE, bool LEGACY, int R>
__device__ __forceinline__ void prepare_whole_row(const typename Src<DTYPE>::T *xr, int k, int m, int row, int chunks,
                                                  float *lds, const MmqPlanes &p, int kpad_blocks, int hblocks,
                                                  int mpad) {
    const int runs = k / 8, nblocks = k / QK8_1, part = threadIdx.x & 3, t = threadIdx.x;
    Raw8<DTYPE> keep[R];
    float mx = 0.0f;
    if (row < m) {  // uniform over the workgroup
#pragma unroll
        for (int u = 0; u < R; ++u) load_raw8<DTYPE>(xr + 8 * min(t + u * PREP_THREADS, runs - 1), keep[u]);
        if constexpr (!LEGACY) {
#pragma unroll
            for (int u = 0; u < R; ++u) {
                float v[8];
                convert8<DTYPE>(keep[u], v);
                if (t + u * PREP_THREADS < runs) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(v[j]));
                }
            }
            // the runs past the kept ones (rows longer than 2048 R values), four at a time
            for (int u0 = R; u0 * PREP_THREADS < runs; u0 += 4) {
                Raw8<DTYPE> r[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) load_raw8<DTYPE>(xr + 8 * min(t + (u0 + u) * PREP_THREADS, runs - 1), r[u]);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    float v[8];
                    convert8<DTYPE>(r[u], v);
                    if (t + (u0 + u) * PREP_THREADS < runs) {
#pragma unroll
                        for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(v[j]));
                    }
                }
            }
        }
    }
    float scale = 1.0f;
    if constexpr (LEGACY) {
        if (row < m && t == 0) p.inverse[row] = 1.0f;
    } else {
        scale = row < m ? row_scale_from_max(block_max(mx, lds), p.inverse + row, t == 0) : 0.0f;
    }
#pragma clang loop unroll(full)  // keep[] stays in registers only with constant indices
    for (int c = 0; c < R; ++c) {
        if (c < chunks) {  // uniform
            const int ib = c * PREP_BLOCKS + (t >> 2);
            float v[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
            if (row < m && ib < nblocks) convert8<DTYPE>(keep[c], v);
            prepare_mmq_chunk<LEGACY>(p, v, scale, ib, row, part, k, m, nblocks, kpad_blocks, hblocks, mpad);
        }
    }
    for (int c = R; c < chunks; ++c) {
        const int ib = c * PREP_BLOCKS + (t >> 2);
        float v[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        if (row < m && ib < nblocks) load8<DTYPE>(xr + QK8_1 * ib + 8 * part, v);
        prepare_mmq_chunk<LEGACY>(p, v, scale, ib, row, part, k, m, nblocks, kpad_blocks, hblocks, mpad);
    }
}

template <int DTYPE, bool LEGACY>
__global__ __launch_bounds__(PREP_THREADS) void prepare_mmq_kernel(
    const typename Src<DTYPE>::T *__restrict__ x, int64_t stride_x, int k, int m, int kpad_blocks, int hblocks, int mpad,
    MmqPlanes p, int chunks) {
    __shared__ float wave_max_lds[PREP_THREADS / WAVE];
    // images: rows m..15 (m..mpad) are written as zeros. Workgroups are dealt round-robin over
    // the 8 XCDs: each XCD takes a contiguous range of rows, so the rows that share a line of
    // the images and planes (32-byte pieces of adjacent rows at one K position) are written
    // into one L2, where the pieces merge before the line goes to HBM.
    const int row = gridDim.x % 8 ? blockIdx.x : (blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8;
    const int nblocks = k / QK8_1;
    const int part = threadIdx.x & 3;
    const auto *xr = x + static_cast<int64_t>(row) * stride_x;
    if (chunks > 1) {  // one workgroup per row, all its chunks (uniform over the grid)
        if (k <= 4 * 8 * PREP_THREADS)
            prepare_whole_row<DTYPE, LEGACY, 4>(xr, k, m, row, chunks, wave_max_lds, p, kpad_blocks, hblocks, mpad);
        else
            prepare_whole_row<DTYPE, LEGACY, 12>(xr, k, m, row, chunks, wave_max_lds, p, kpad_blocks, hblocks, mpad);
        return;
    }
    float own[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    float scale = 0.0f;
    if constexpr (LEGACY) {
        if (row < m && blockIdx.y == 0 && threadIdx.x == 0) p.inverse[row] = 1.0f;
        scale = 1.0f;
    } else if (row < m) {  // uniform over the workgroup
        scale = row_scale<DTYPE>(xr, k, wave_max_lds, p.inverse + row, blockIdx.y == 0 && threadIdx.x == 0, own);
    }
    // the workgroup's chunk of PREP_BLOCKS blocks, from the row maximum's pass (own)
    const int ib = blockIdx.y * PREP_BLOCKS + (threadIdx.x >> 2);
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = own[j];
    if (LEGACY) {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = 0.0f;
        if (row < m && ib < nblocks) load8<DTYPE>(xr + QK8_1 * ib + 8 * part, v);
    }
    prepare_mmq_chunk<LEGACY>(p, v, scale, ib, row, part, k, m, nblocks, kpad_blocks, hblocks, mpad);
}

template <int DTYPE>
static void launch_prepare_dtype(const void *x, int64_t m, int64_t k, int64_t stride_x, const ActLayout &o,
                                 hipStream_t stream) {
    const int nblocks = static_cast<int>(k / QK8_1);
    const dim3 grid(static_cast<unsigned>(m), static_cast<unsigned>((nblocks + PREP_BLOCKS - 1) / PREP_BLOCKS));
    const auto *src = static_cast<const typename Src<DTYPE>::T *>(x);
    if (o.y2) {
        prepare_q8_1_kernel<DTYPE, true><<<grid, dim3(PREP_THREADS), 0, stream>>>(
            src, stride_x, static_cast<int>(k), o.y1, o.y2, o.inverse);
    } else {
        prepare_q8_1_kernel<DTYPE, false><<<grid, dim3(PREP_THREADS), 0, stream>>>(
            src, stride_x, static_cast<int>(k), o.y1, o.y2, o.inverse);
    }
}

void launch_prepare(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x, const ActLayout &out,
                    hipStream_t stream) {
    if (k / QK8_1 > PREP_MAX_BLOCKS) throw Error("Fused activation preparation supports K <= 32768");
    switch (x_dtype) {
        case 0: launch_prepare_dtype<0>(x, m, k, stride_x, out, stream); break;
        case 1: launch_prepare_dtype<1>(x, m, k, stride_x, out, stream); break;
        case 2: launch_prepare_dtype<2>(x, m, k, stride_x, out, stream); break;
        default: throw Error("Fused activations must be F32, BF16 or F16");
    }
}

template <int DTYPE>
static void launch_prepare_mmq_dtype(const void *x, int64_t m, int64_t k, int64_t stride_x, const MmqPlanes &p,
                                     hipStream_t stream) {
    const int kpad_blocks = static_cast<int>(mmq_blocks128(k) * 4);
    const bool any_h = p.h[0].codes || p.h[1].codes || p.h[2].codes;
    // images: the zero rows too (small-M images to 16 rows, fp16 images to mmqh_mpad(m))
    const int64_t rows = p.image ? MMQS_MAX_ROWS : any_h ? mmqh_mpad(m) : m;
    const int hblocks = static_cast<int>(mmqh_kpad(k) / QK8_1), mpad = static_cast<int>(mmqh_mpad(m));
    // Many rows: one workgroup per row walks all its chunks, so the row maximum is read once per
    // row instead of once per chunk (at 2048 rows of K = 17408, nine times)
    const int all_chunks = (kpad_blocks + PREP_BLOCKS - 1) / PREP_BLOCKS;
    const int chunks = rows >= 256 ? all_chunks : 1;
    const dim3 grid(static_cast<unsigned>(rows), static_cast<unsigned>((all_chunks + chunks - 1) / chunks));
    const auto *src = static_cast<const typename Src<DTYPE>::T *>(x);
    if (p.legacy)
        prepare_mmq_kernel<DTYPE, true><<<grid, dim3(PREP_THREADS), 0, stream>>>(
            src, stride_x, static_cast<int>(k), static_cast<int>(m), kpad_blocks, hblocks, mpad, p, chunks);
    else
        prepare_mmq_kernel<DTYPE, false><<<grid, dim3(PREP_THREADS), 0, stream>>>(
            src, stride_x, static_cast<int>(k), static_cast<int>(m), kpad_blocks, hblocks, mpad, p, chunks);
}

void launch_prepare_mmq(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x, const MmqPlanes &planes,
                        hipStream_t stream) {
    if (k % QK8_1 || k <= 0 || m <= 0 || m > INT_MAX || mmq_blocks128(k) * 4 > INT_MAX)
        throw Error("Invalid batched activation shape");
    if (planes.image && m > MMQS_MAX_ROWS) throw Error("Small-M images hold at most 16 activation rows");
    if (planes.legacy && planes.d2s6) throw Error("The legacy quantisation has no D2S6 layout");
    if ((planes.legacy || planes.image) && (planes.h[0].codes || planes.h[1].codes || planes.h[2].codes))
        throw Error("The fp16 GEMM's images take the batched quantisation above 16 rows");
    switch (x_dtype) {
        case 0: launch_prepare_mmq_dtype<0>(x, m, k, stride_x, planes, stream); break;
        case 1: launch_prepare_mmq_dtype<1>(x, m, k, stride_x, planes, stream); break;
        case 2: launch_prepare_mmq_dtype<2>(x, m, k, stride_x, planes, stream); break;
        default: throw Error("Fused MMQ activations must be F32, BF16 or F16");
    }
}

// ---------------------------------------------------------------- fused producers
// Producers of the single-pass Q8_1 activation from a transformed input, so the consumer
// GEMV needs no separate preparation (the reference's kai_prepare_ext.cuh:121-251, entry
// points current_ggml_direct.cu:883-944):
//   view   stored column c reads x column ((c/s)%a)*b*s + (c/(a*s))*s + c%s;
//   swiglu act[c] = rd(rd(silu(g[c])) * u[c]) from a merged [gate | up] row, rd rounding to
//          the input dtype, silu(g) = g / (1 + exp(-g));
//   norm   v = x (+ r, written to the fp32 residual stream), y = bf16(v * rstd * w32) with
//          rstd = 1 / sqrt(sum(v^2) / k + eps); the activation quantises the stored y.
// One workgroup of PRODUCE_THREADS per row; run r of 8 values belongs to thread
// r % PRODUCE_THREADS, so the four runs of a 32-value block sit in one quad. Every
// reduction whose order could change a bit has a fixed order that the CPU oracle repeats:
// sum(v^2) accumulates each thread's runs in order with fused multiply-adds, then a binary
// tree over the 64 lanes of a wave, then the waves in order.
constexpr int PRODUCE_THREADS = 512;
constexpr int PRODUCE_RUNS = 8;  // k <= 32768

// exp for the SwiGLU producer (the platform exp is not specified to the bit): Cody-Waite
// reduction x = n ln2 + r with a two-part ln2, the degree-7 Taylor polynomial of e^r by
// Horner in fused multiply-adds, and 2^n by ldexp. Each step is one IEEE operation, so the
// oracle's copy of these lines returns the same bits; within 2 ulp of e^x.
__device__ __forceinline__ float produce_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return __builtin_inff();
    if (x < -103.97208404541015625f) return 0.0f;
    const float n = rintf(x * 1.44269502162933349609375f);
    float r = fmaf(-n, 0.693145751953125f, x);
    r = fmaf(-n, 1.42860682030941723212e-6f, r);
    float p = 1.98412698e-4f;
    p = fmaf(p, r, 1.38888889e-3f);
    p = fmaf(p, r, 8.33333333e-3f);
    p = fmaf(p, r, 4.16666667e-2f);
    p = fmaf(p, r, 1.66666667e-1f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, static_cast<int>(n));
}

template <int DTYPE>
__device__ __forceinline__ float round_to_src(float v) {
    if constexpr (DTYPE == 1) return bf16_bits_to_float(float_to_bf16_bits(v));
    else if constexpr (DTYPE == 2) return half_bits_to_float(float_to_half_bits(v));
    else return v;
}

enum ProduceMode { PRODUCE_VIEW = 0, PRODUCE_SWIGLU = 1, PRODUCE_NORM = 2 };

struct ProduceArgs {
    const void *x;  // view: x; swiglu: [gate | up]; norm: x
    int64_t stride_x;
    const void *res;  // norm: residual or null
    int64_t stride_r;
    float *res_out;  // norm: fp32 residual stream [m][k]
    const float *w32;
    float eps;
    uint16_t *y;  // norm: bf16 output [m][k]
    int a, b, s;  // view
    int k;
    block_q8_1 *y1;
    float *inverse;
};

// Sum over the workgroup in the fixed order described above (every lane gets it).
__device__ __forceinline__ float produce_sum(float v, float *lds) {
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    v = wave_sum(v);  // binary tree over the lanes (pairs, quads, 8, 16, 32, 64)
    if (lane == 0) lds[wave] = v;
    __syncthreads();
    float s = lds[0];
    for (int w = 1; w < PRODUCE_THREADS / WAVE; ++w) s += lds[w];
    return s;
}

template <int MODE, int XT, int RT>
__global__ __launch_bounds__(PRODUCE_THREADS) void produce_kernel(ProduceArgs p) {
    __shared__ float max_lds[PRODUCE_THREADS / WAVE];
    __shared__ float sum_lds[PRODUCE_THREADS / WAVE];
    using XS = typename Src<XT>::T;
    const int row = blockIdx.x, t = threadIdx.x, k = p.k, nruns = k / 8;
    const XS *xr = static_cast<const XS *>(p.x) + static_cast<int64_t>(row) * p.stride_x;
    float v[PRODUCE_RUNS][8];
    float amax = 0.0f, ss = 0.0f;
#pragma unroll
    for (int i = 0; i < PRODUCE_RUNS; ++i) {
        const int r = t + PRODUCE_THREADS * i, c = 8 * r;
        if (r >= nruns) continue;
        if constexpr (MODE == PRODUCE_VIEW) {
            load8<XT>(xr + ((c / p.s) % p.a) * p.b * p.s + (c / (p.a * p.s)) * p.s + c % p.s, v[i]);
        } else if constexpr (MODE == PRODUCE_SWIGLU) {
            float u[8];
            load8<XT>(xr + c, v[i]);
            load8<XT>(xr + k + c, u);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float g = v[i][j];
                v[i][j] = round_to_src<XT>(round_to_src<XT>(g / (1.0f + produce_expf(-g))) * u[j]);
            }
        } else {
            load8<XT>(xr + c, v[i]);
            if (p.res) {
                float rv[8];
                load8<RT>(static_cast<const typename Src<RT>::T *>(p.res) + static_cast<int64_t>(row) * p.stride_r + c, rv);
#pragma unroll
                for (int j = 0; j < 8; ++j) v[i][j] += rv[j];
                float4 *ro = reinterpret_cast<float4 *>(p.res_out + static_cast<int64_t>(row) * k + c);
                ro[0] = make_float4(v[i][0], v[i][1], v[i][2], v[i][3]);
                ro[1] = make_float4(v[i][4], v[i][5], v[i][6], v[i][7]);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) ss = fmaf(v[i][j], v[i][j], ss);
        }
        if constexpr (MODE != PRODUCE_NORM) {
#pragma unroll
            for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[i][j]));
        }
    }
    if constexpr (MODE == PRODUCE_NORM) {
        const float total = produce_sum(ss, sum_lds);
        const float rstd = 1.0f / sqrtf(total / static_cast<float>(k) + p.eps);
#pragma unroll
        for (int i = 0; i < PRODUCE_RUNS; ++i) {
            const int r = t + PRODUCE_THREADS * i, c = 8 * r;
            if (r >= nruns) continue;
            uint32_t packed[4];
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                const uint16_t h0 = float_to_bf16_bits(v[i][j] * rstd * p.w32[c + j]);
                const uint16_t h1 = float_to_bf16_bits(v[i][j + 1] * rstd * p.w32[c + j + 1]);
                v[i][j] = bf16_bits_to_float(h0);
                v[i][j + 1] = bf16_bits_to_float(h1);
                packed[j / 2] = static_cast<uint32_t>(h0) | (static_cast<uint32_t>(h1) << 16);
                amax = fmaxf(amax, fmaxf(fabsf(v[i][j]), fabsf(v[i][j + 1])));
            }
            *reinterpret_cast<uint4 *>(p.y + static_cast<int64_t>(row) * k + c) =
                make_uint4(packed[0], packed[1], packed[2], packed[3]);
        }
    }
    const float scale = row_scale_from_max(block_max(amax, max_lds), p.inverse + row, t == 0);
#pragma unroll
    for (int i = 0; i < PRODUCE_RUNS; ++i) {
        const int r = t + PRODUCE_THREADS * i;
        if (r >= nruns) continue;  // whole quads: nruns is a multiple of 4
#pragma unroll
        for (int j = 0; j < 8; ++j) v[i][j] *= scale;
        int8_t q[8];
        quad_store(v[i], p.y1 + static_cast<int64_t>(row) * (k / QK8_1) + r / 4, r & 3, q);
    }
}

template <int MODE, int XT, int RT>
static void launch_produce(const ProduceArgs &a, int64_t m, hipStream_t stream) {
    produce_kernel<MODE, XT, RT><<<dim3(static_cast<unsigned>(m)), dim3(PRODUCE_THREADS), 0, stream>>>(a);
}

static ProduceArgs produce_args(int64_t k, const ActLayout &out) {
    ProduceArgs a{};
    a.k = static_cast<int>(k);
    a.y1 = out.y1;
    a.inverse = out.inverse;
    return a;
}

void launch_prepare_view(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x, int64_t a, int64_t b,
                         int64_t s, const ActLayout &out, hipStream_t stream) {
    if (k / 8 > PRODUCE_THREADS * PRODUCE_RUNS) throw Error("Fused activation preparation supports K <= 32768");
    ProduceArgs p = produce_args(k, out);
    p.x = x;
    p.stride_x = stride_x;
    p.a = static_cast<int>(a);
    p.b = static_cast<int>(b);
    p.s = static_cast<int>(s);
    switch (x_dtype) {
        case 0: launch_produce<PRODUCE_VIEW, 0, 0>(p, m, stream); break;
        case 1: launch_produce<PRODUCE_VIEW, 1, 0>(p, m, stream); break;
        case 2: launch_produce<PRODUCE_VIEW, 2, 0>(p, m, stream); break;
        default: throw Error("Fused activations must be F32, BF16 or F16");
    }
}

void launch_prepare_swiglu(const void *gate_up, int dtype, int64_t m, int64_t k, int64_t stride, const ActLayout &out,
                           hipStream_t stream) {
    if (k / 8 > PRODUCE_THREADS * PRODUCE_RUNS) throw Error("Fused activation preparation supports K <= 32768");
    ProduceArgs p = produce_args(k, out);
    p.x = gate_up;
    p.stride_x = stride;
    switch (dtype) {
        case 0: launch_produce<PRODUCE_SWIGLU, 0, 0>(p, m, stream); break;
        case 1: launch_produce<PRODUCE_SWIGLU, 1, 0>(p, m, stream); break;
        case 2: launch_produce<PRODUCE_SWIGLU, 2, 0>(p, m, stream); break;
        default: throw Error("Fused activations must be F32, BF16 or F16");
    }
}

void launch_norm_prepare(const void *x, int x_dtype, int64_t stride_x, const void *residual, int residual_dtype,
                         int64_t stride_r, float *residual_out, const float *weight32, float eps, void *y, int64_t m,
                         int64_t k, const ActLayout &out, hipStream_t stream) {
    if (k / 8 > PRODUCE_THREADS * PRODUCE_RUNS) throw Error("Fused activation preparation supports K <= 32768");
    ProduceArgs p = produce_args(k, out);
    p.x = x;
    p.stride_x = stride_x;
    p.res = residual;
    p.stride_r = stride_r;
    p.res_out = residual_out;
    p.w32 = weight32;
    p.eps = eps;
    p.y = static_cast<uint16_t *>(y);
    switch (x_dtype * 4 + (residual ? residual_dtype : 0)) {
        case 0 * 4 + 0: launch_produce<PRODUCE_NORM, 0, 0>(p, m, stream); break;
        case 0 * 4 + 1: launch_produce<PRODUCE_NORM, 0, 1>(p, m, stream); break;
        case 1 * 4 + 0: launch_produce<PRODUCE_NORM, 1, 0>(p, m, stream); break;
        case 1 * 4 + 1: launch_produce<PRODUCE_NORM, 1, 1>(p, m, stream); break;
        default: throw Error("Fused norm inputs must be BF16 or F32 (residual BF16 or F32)");
    }
}

}  // namespace kai
