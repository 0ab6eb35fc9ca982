// Measurement kernels: the MFMA rate, the LDS read rate and a STREAM-style HBM copy of this
// device, each timed by the caller (bench.py --peaks) to set the roofline's measured ceilings
// beside the published ones. No counterpart in the reference.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/kai_peaks.h"
#include "kai_launch.h"

namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef float f16_t __attribute__((ext_vector_type(16)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef int i4_t __attribute__((ext_vector_type(4)));
typedef int i16_t __attribute__((ext_vector_type(16)));

// CHAINS independent accumulators per wave, ITERS rounds: the MFMA pipe of each SIMD never waits
// on a result. Operands come from the lane id (their values do not change the rate).
constexpr int CHAINS = 4;
template <int KIND>
__global__ __launch_bounds__(1024) void peak_mfma_kernel(int64_t iters, float *out) {
    const int l = threadIdx.x;
    if constexpr (KIND == KAI_PEAK_F16_32X32X16 || KIND == KAI_PEAK_F16_16X16X32 || KIND == KAI_PEAK_F16_32X32X8) {
        const _Float16 v = static_cast<_Float16>(static_cast<float>(l & 7) * 0.125f);
        const h8_t a8 = {v, v, v, v, v, v, v, v};
        const h4_t a4 = {v, v, v, v};
        if constexpr (KIND == KAI_PEAK_F16_16X16X32) {
            f4_t acc[CHAINS] = {};
            for (int64_t i = 0; i < iters; ++i)
#pragma unroll
                for (int c = 0; c < CHAINS; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a8, a8, acc[c], 0, 0, 0);
            float s = 0.0f;
#pragma unroll
            for (int c = 0; c < CHAINS; ++c) s += acc[c][0];
            if (s == 1234.5f) out[l] = s;
        } else {
            f16_t acc[CHAINS] = {};
            for (int64_t i = 0; i < iters; ++i)
#pragma unroll
                for (int c = 0; c < CHAINS; ++c) {
                    if constexpr (KIND == KAI_PEAK_F16_32X32X16)
                        acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a8, a8, acc[c], 0, 0, 0);
                    else
                        acc[c] = __builtin_amdgcn_mfma_f32_32x32x8f16(a4, a4, acc[c], 0, 0, 0);
                }
            float s = 0.0f;
#pragma unroll
            for (int c = 0; c < CHAINS; ++c) s += acc[c][0];
            if (s == 1234.5f) out[l] = s;
        }
    } else {
        const int v = (l & 7) * 0x01010101;
        const i4_t a = {v, v, v, v};
        if constexpr (KIND == KAI_PEAK_I8_16X16X64) {
            i4_t acc[CHAINS] = {};
            for (int64_t i = 0; i < iters; ++i)
#pragma unroll
                for (int c = 0; c < CHAINS; ++c) acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, a, acc[c], 0, 0, 0);
            int s = 0;
#pragma unroll
            for (int c = 0; c < CHAINS; ++c) s += acc[c][0];
            if (s == 12345) out[l] = static_cast<float>(s);
        } else {
            i16_t acc[CHAINS] = {};
            for (int64_t i = 0; i < iters; ++i)
#pragma unroll
                for (int c = 0; c < CHAINS; ++c) acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, a, acc[c], 0, 0, 0);
            int s = 0;
#pragma unroll
            for (int c = 0; c < CHAINS; ++c) s += acc[c][0];
            if (s == 12345) out[l] = static_cast<float>(s);
        }
    }
}

// Each lane reads 16 bytes per round from a 64 KiB LDS block (lane-consecutive addresses,
// no bank conflicts), four reads in flight.
__global__ __launch_bounds__(1024) void peak_lds_kernel(int64_t iters, float *out) {
    __shared__ __align__(16) uint4 buf[4096];
    for (int i = threadIdx.x; i < 4096; i += blockDim.x) buf[i] = make_uint4(i, i + 1, i + 2, i + 3);
    __syncthreads();
    uint4 x = make_uint4(0, 0, 0, 0);
    const int base = threadIdx.x % 1024;
    for (int64_t i = 0; i < iters; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint4 v = buf[(base + 1024 * r + static_cast<int>(i & 0)) & 4095];
            x.x ^= v.x, x.y += v.y, x.z ^= v.z, x.w += v.w;
        }
        asm volatile("" : "+v"(x.x), "+v"(x.y), "+v"(x.z), "+v"(x.w));
    }
    if (x.x == 0x12345 && x.y == 7) out[threadIdx.x] = 1.0f;
}

// dst = src, 16 bytes per lane per step, grid-stride; each step's loads are all issued first.
typedef unsigned u4v_t __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void peak_copy_kernel(const u4v_t *__restrict__ src, u4v_t *__restrict__ dst,
                                                         int64_t n16) {
    constexpr int U = 4;
    const int64_t stride = int64_t(gridDim.x) * blockDim.x;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += U * stride) {
        u4v_t v[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (i + u * stride < n16) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (i + u * stride < n16) __builtin_nontemporal_store(v[u], dst + i + u * stride);
    }
}

}  // namespace

namespace kai {

void launch_peak_mfma(int kind, int64_t iters, int blocks, int threads, float *out, hipStream_t s) {
    if (iters <= 0 || blocks <= 0 || threads <= 0 || threads > 1024 || threads % 64 || !out)
        throw Error("Invalid MFMA peak launch");
    switch (kind) {
#define KAI_K(K) \
    case K: peak_mfma_kernel<K><<<blocks, threads, 0, s>>>(iters, out); break;
        KAI_K(KAI_PEAK_F16_32X32X16) KAI_K(KAI_PEAK_F16_16X16X32) KAI_K(KAI_PEAK_F16_32X32X8)
        KAI_K(KAI_PEAK_I8_32X32X32) KAI_K(KAI_PEAK_I8_16X16X64)
#undef KAI_K
        default: throw Error("Unknown MFMA kind");
    }
}

int64_t peak_mfma_ops(int kind) {
    switch (kind) {
        case KAI_PEAK_F16_32X32X16: return 2LL * 32 * 32 * 16;
        case KAI_PEAK_F16_16X16X32: return 2LL * 16 * 16 * 32;
        case KAI_PEAK_F16_32X32X8: return 2LL * 32 * 32 * 8;
        case KAI_PEAK_I8_32X32X32: return 2LL * 32 * 32 * 32;
        case KAI_PEAK_I8_16X16X64: return 2LL * 16 * 16 * 64;
        default: return 0;
    }
}

void launch_peak_lds(int64_t iters, int blocks, int threads, float *out, hipStream_t s) {
    if (iters <= 0 || blocks <= 0 || threads <= 0 || threads > 1024 || threads % 64 || !out)
        throw Error("Invalid LDS peak launch");
    peak_lds_kernel<<<blocks, threads, 0, s>>>(iters, out);
}

void launch_peak_copy(const void *src, void *dst, int64_t bytes, int blocks, hipStream_t s) {
    if (!src || !dst || bytes <= 0 || bytes % 16 || blocks <= 0) throw Error("Invalid copy peak launch");
    peak_copy_kernel<<<blocks, 256, 0, s>>>(static_cast<const u4v_t *>(src), static_cast<u4v_t *>(dst), bytes / 16);
}

}  // namespace kai
