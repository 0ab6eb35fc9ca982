// The fp16 GEMM (kai_mmqh.cuh): its split-K reduction and the dispatch by weight type (the
// kernels are instantiated in kai_mmq_<type>.hip).
#include "kai_mmqh.cuh"

namespace kai {

// out[i][j] = inverse[i] * (sum of the splits' partial sums, in split order).
__global__ __launch_bounds__(256) void mmqh_reduce_kernel(const float *__restrict__ partial, int splits, int m, int n,
                                                          const float *__restrict__ inverse, void *__restrict__ dst,
                                                          int64_t stride_dst, int dst_bf16) {
    const int64_t total = int64_t(m) * n;
    const int64_t e0 = (int64_t(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (n % 4 == 0) {  // the four elements share a row: 16-byte loads of every split, in split order
        if (e0 >= total) return;
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int z = 0; z < splits; ++z) {
            const float4 p = *reinterpret_cast<const float4 *>(partial + int64_t(z) * total + e0);
            v.x += p.x;
            v.y += p.y;
            v.z += p.z;
            v.w += p.w;
        }
        const int i = static_cast<int>(e0 / n), j = static_cast<int>(e0 % n);
        const float inv = inverse[i];
        v.x *= inv;
        v.y *= inv;
        v.z *= inv;
        v.w *= inv;
        const int64_t idx = int64_t(i) * stride_dst + j;
        if (dst_bf16) {
            const uint32_t lo = float_to_bf16_bits(v.x) | (uint32_t(float_to_bf16_bits(v.y)) << 16),
                           hi = float_to_bf16_bits(v.z) | (uint32_t(float_to_bf16_bits(v.w)) << 16);
            uint16_t *d = static_cast<uint16_t *>(dst) + idx;
            if ((reinterpret_cast<uintptr_t>(d) & 7) == 0) {
                *reinterpret_cast<uint2 *>(d) = make_uint2(lo, hi);
            } else {
                d[0] = lo & 0xffffu, d[1] = lo >> 16, d[2] = hi & 0xffffu, d[3] = hi >> 16;
            }
        } else {
            float *d = static_cast<float *>(dst) + idx;
            if ((reinterpret_cast<uintptr_t>(d) & 15) == 0) {
                *reinterpret_cast<float4 *>(d) = v;
            } else {
                d[0] = v.x, d[1] = v.y, d[2] = v.z, d[3] = v.w;
            }
        }
        return;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int64_t e = e0 + q;
        if (e >= total) return;
        float v = 0.0f;
        for (int z = 0; z < splits; ++z) v += partial[int64_t(z) * total + e];
        const int i = static_cast<int>(e / n), j = static_cast<int>(e % n);
        v *= inverse[i];
        const int64_t idx = int64_t(i) * stride_dst + j;
        if (dst_bf16) static_cast<uint16_t *>(dst)[idx] = float_to_bf16_bits(v);
        else static_cast<float *>(dst)[idx] = v;
    }
}

#define KAI_EXTERN(T) \
    extern template void launch_mmqh<T>(const void *, int64_t, int64_t, int64_t, const MmqhArgs &, const float *, \
                                        float *, size_t, void *, bool, int64_t, hipStream_t);
KAI_EXTERN(Q8_0) KAI_EXTERN(Q4_0) KAI_EXTERN(Q4_K) KAI_EXTERN(Q2_K) KAI_EXTERN(IQ3_S)
#undef KAI_EXTERN

void launch_mmq_h(int type, const void *weight, int64_t n, int64_t k, int64_t m, const MmqhImage &image,
                  const float *inverse, float *partial, size_t partial_bytes, void *dst, bool dst_bf16,
                  int64_t stride_dst, hipStream_t stream) {
    if (!image.codes || (mmq_layout(type) != MMQ_D4 && !image.mins))
        throw Error("The fp16 GEMM's activation image is missing");
    if (m > INT_MAX || mmqh_mpad(m) > INT_MAX) throw Error("Too many activation rows");
    const MmqhArgs a{image.codes, image.mins, static_cast<int>(mmqh_mpad(m))};
    switch (type) {
#define KAI_T(T) \
    case T: launch_mmqh<T>(weight, n, k, m, a, inverse, partial, partial_bytes, dst, dst_bf16, stride_dst, stream); return;
        KAI_T(Q8_0) KAI_T(Q4_0) KAI_T(Q4_K) KAI_T(Q2_K) KAI_T(IQ3_S)
#undef KAI_T
        default: throw Error("The fp16 GEMM takes Q8_0, Q4_0, Q4_K, Q2_K and IQ3_S");
    }
}

size_t mmqh_partial_bytes_of(int type, int64_t m, int64_t n, int64_t k) {
    switch (type) {
#define KAI_T(T) case T: return mmqh_partial_bytes(mmqh_plan<T>(n, k, m), m, n);
        KAI_T(Q8_0) KAI_T(Q4_0) KAI_T(Q4_K) KAI_T(Q2_K) KAI_T(IQ3_S)
#undef KAI_T
        default: return 0;
    }
}

}  // namespace kai
