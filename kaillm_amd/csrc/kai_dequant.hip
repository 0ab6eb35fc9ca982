// Dequantisation of GGUF wire blocks to F32 / BF16 / F16: the reference's legacy
// ggml_dequantize op (csrc/gguf/gguf_kernel.cu:87-102, dispatch quantization/linear.py:55-59),
// which its non-fused layers and embedding loaders call.
//
// One thread per run of 8 consecutive output values; a run never straddles a block (every
// block holds a multiple of 8 values). The thread reads the few header and code bytes of
// its run straight from global memory (the block's other runs hit the same cache lines) and
// writes 16 or 32 contiguous bytes. The kernel is HBM-bound on the output: per value it
// moves 0.56 B (Q4_K) .. 1.06 B (Q8_0) of weights in and 2 or 4 B out.
//
// Each value is the format's published formula in fp32 with every product and difference
// rounded separately (no fused multiply-add), in the order gguf-py's quants.py evaluates it,
// then rounded to the output type to nearest even.
#include "kai_device.h"
#include "kai_formats.h"
#include "kai_iq3s_grid.h"
#include "kai_launch.h"

namespace kai {
namespace {

constexpr int DQ_THREADS = 256;

static __device__ const uint32_t dq_iq3s_grid[512] = {KAI_IQ3S_GRID_VALUES};

__device__ __forceinline__ float ld_half(const uint8_t *p) { return half_bits_to_float(p[0] | (p[1] << 8)); }

// Values e0 .. e0 + 7 of the block at b (e0 a multiple of 8).
template <int TYPE>
__device__ __forceinline__ void dequant_run(const uint8_t *__restrict__ b, int e0, float (&v)[8]) {
#pragma clang fp contract(off)
    if constexpr (TYPE == Q8_0) {  // quants.py:397-402: d * q
        const float d = ld_half(b);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = d * static_cast<float>(static_cast<int8_t>(b[2 + e0 + j]));
    } else if constexpr (TYPE == Q4_0) {  // quants.py:242-252: d * (nibble - 8); low nibbles first
        const float d = ld_half(b);
        const int shift = e0 < 16 ? 0 : 4, base = 2 + (e0 & 15);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = d * static_cast<float>(((b[base + j] >> shift) & 15) - 8);
    } else if constexpr (TYPE == Q4_K) {  // quants.py:480-523: (d * sc) * q - dmin * m
        const float d = ld_half(b), dmin = ld_half(b + 2);
        const int i = e0 / 32, l0 = e0 % 32;
        const uint8_t *s = b + 4;
        const int sc = i < 4 ? (s[i] & 63) : ((s[4 + i] & 15) | ((s[i - 4] >> 2) & 48));
        const int mn = i < 4 ? (s[4 + i] & 63) : ((s[4 + i] >> 4) | ((s[i] >> 2) & 48));
        const float dsc = d * static_cast<float>(sc), dmn = dmin * static_cast<float>(mn);
        const uint8_t *q = b + 16 + 32 * (i / 2) + l0;
        const int shift = 4 * (i % 2);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = dsc * static_cast<float>((q[j] >> shift) & 15) - dmn;
    } else if constexpr (TYPE == Q6_K) {  // quants.py:553-573: (d * sc) * (q - 32)
        const float d = ld_half(b + 208);
        const int h = e0 / 128, sub = (e0 % 128) / 32, l0 = e0 % 32;
        const float dsc = d * static_cast<float>(static_cast<int8_t>(b[192 + e0 / 16]));
        const uint8_t *ql = b + 64 * h + 32 * (sub % 2) + l0, *qh = b + 128 + 32 * h + l0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int lo = (ql[j] >> (4 * (sub / 2))) & 15, hi = (qh[j] >> (2 * sub)) & 3;
            v[j] = dsc * static_cast<float>((lo | (hi << 4)) - 32);
        }
    } else if constexpr (TYPE == Q2_K) {  // quants.py:407-429: (d * sc) * q - dmin * m
        const float d = ld_half(b + 80), dmin = ld_half(b + 82);
        const int s = b[e0 / 16], h = e0 / 128, sub = (e0 % 128) / 32, l0 = e0 % 32;
        const float dsc = d * static_cast<float>(s & 15), dmn = dmin * static_cast<float>(s >> 4);
        const uint8_t *q = b + 16 + 32 * h + l0;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = dsc * static_cast<float>((q[j] >> (2 * sub)) & 3) - dmn;
    } else {  // IQ3_S, quants.py:1097-1125: (d * (1 + 2 sc)) * level * sign
        const float d = ld_half(b);
        const int g = e0 / 32, t0 = e0 % 32;
        const float dsc = d * static_cast<float>(1 + 2 * ((b[106 + g / 2] >> (4 * (g % 2))) & 15));
        const int signs = b[74 + 4 * g + t0 / 8];
#pragma unroll
        for (int half = 0; half < 2; ++half) {  // two grid entries of 4 values
            const int i = t0 / 4 + half;
            const int idx = b[2 + 8 * g + i] | (((b[66 + g] >> i) & 1) << 8);
            const uint32_t levels = dq_iq3s_grid[idx];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int level = (levels >> (8 * j)) & 255;
                const int value = ((signs >> (4 * half + j)) & 1) ? -level : level;
                v[4 * half + j] = dsc * static_cast<float>(value);
            }
        }
    }
}

template <int TYPE, int OUT>
__global__ __launch_bounds__(DQ_THREADS) void dequant_kernel(const uint8_t *__restrict__ w, int64_t runs,
                                                             void *__restrict__ out) {
    constexpr int QK = block_elems(TYPE), BB = block_bytes(TYPE);
    const int64_t r = static_cast<int64_t>(blockIdx.x) * DQ_THREADS + threadIdx.x;
    if (r >= runs) return;
    const int64_t e = 8 * r;
    float v[8];
    dequant_run<TYPE>(w + (e / QK) * BB, static_cast<int>(e % QK), v);
    if constexpr (OUT == 0) {
        float4 *o = reinterpret_cast<float4 *>(static_cast<float *>(out) + e);
        o[0] = make_float4(v[0], v[1], v[2], v[3]);
        o[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else {
        // The fp32 values are materialised before rounding: otherwise the compiler folds a
        // product and its conversion into one mixed-precision fused multiply-add with a +0
        // addend, which turns a -0 product into +0.
#pragma unroll
        for (int j = 0; j < 8; ++j) asm volatile("" : "+v"(v[j]));
        uint32_t p[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t lo = OUT == 1 ? float_to_bf16_bits(v[2 * j]) : float_to_half_bits(v[2 * j]);
            const uint32_t hi = OUT == 1 ? float_to_bf16_bits(v[2 * j + 1]) : float_to_half_bits(v[2 * j + 1]);
            p[j] = lo | (hi << 16);
        }
        *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(out) + e) = make_uint4(p[0], p[1], p[2], p[3]);
    }
}

template <int TYPE>
void launch_dequant_type(const void *w, int64_t values, void *out, int out_dtype, hipStream_t stream) {
    const int64_t runs = values / 8;
    const dim3 grid(static_cast<unsigned>((runs + DQ_THREADS - 1) / DQ_THREADS));
    const auto *src = static_cast<const uint8_t *>(w);
    switch (out_dtype) {
        case 0: dequant_kernel<TYPE, 0><<<grid, DQ_THREADS, 0, stream>>>(src, runs, out); break;
        case 1: dequant_kernel<TYPE, 1><<<grid, DQ_THREADS, 0, stream>>>(src, runs, out); break;
        case 2: dequant_kernel<TYPE, 2><<<grid, DQ_THREADS, 0, stream>>>(src, runs, out); break;
        default: throw Error("Dequantized output must be F32, BF16 or F16");
    }
}

}  // namespace

void launch_dequantize(const void *w, int type, int64_t values, void *out, int out_dtype, hipStream_t stream) {
    if (values <= 0) return;
    if (values / 8 > static_cast<int64_t>(DQ_THREADS) * 0xffffffffLL) throw Error("Dequantization too large");
    switch (type) {
        case Q8_0: launch_dequant_type<Q8_0>(w, values, out, out_dtype, stream); break;
        case Q4_0: launch_dequant_type<Q4_0>(w, values, out, out_dtype, stream); break;
        case Q4_K: launch_dequant_type<Q4_K>(w, values, out, out_dtype, stream); break;
        case Q6_K: launch_dequant_type<Q6_K>(w, values, out, out_dtype, stream); break;
        case Q2_K: launch_dequant_type<Q2_K>(w, values, out, out_dtype, stream); break;
        case IQ3_S: launch_dequant_type<IQ3_S>(w, values, out, out_dtype, stream); break;
        default: throw Error("Unsupported GGML weight type");
    }
}

}  // namespace kai
