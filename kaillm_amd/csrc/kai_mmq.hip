// MMQ dispatch by weight type (instantiations live in kai_mmq_<type>.hip).
#include "kai_mmqs.cuh"

namespace kai {

template <bool PLANES>
static void dispatch(int type, const void *weight, int64_t n, int64_t k, int64_t m, const void *act,
                     const float *inverse, void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream) {
    switch (type) {
#define KAI_T(T) \
    case T: launch_mmq_type<T, PLANES>(weight, n, k, m, act, inverse, dst, dst_bf16, stride_dst, stream); break;
        KAI_T(Q8_0) KAI_T(Q4_0) KAI_T(Q4_K) KAI_T(Q6_K) KAI_T(Q2_K) KAI_T(IQ3_S)
#undef KAI_T
        default: throw Error("Unsupported fused MMQ weight type");
    }
}

void launch_mmq(int type, const void *weight, int64_t n, int64_t k, int64_t m, const block_q8_1 *y,
                const float *inverse, void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream) {
    dispatch<false>(type, weight, n, k, m, y, inverse, dst, dst_bf16, stride_dst, stream);
}

void launch_mmq_planes(int type, const void *weight, int64_t n, int64_t k, int64_t m, const uint8_t *plane,
                       const float *inverse, float *partial, size_t partial_bytes, void *dst, bool dst_bf16,
                       int64_t stride_dst, hipStream_t stream) {
    if (m <= MMQS_MAX_ROWS) {
        switch (type) {
#define KAI_T(T) \
    case T: launch_mmqs<T>(weight, n, k, m, plane, inverse, partial, partial_bytes, dst, dst_bf16, stride_dst, stream); return;
            KAI_T(Q8_0) KAI_T(Q4_0) KAI_T(Q4_K) KAI_T(Q6_K) KAI_T(Q2_K) KAI_T(IQ3_S)
#undef KAI_T
            default: throw Error("Unsupported fused MMQ weight type");
        }
    }
    dispatch<true>(type, weight, n, k, m, plane, inverse, dst, dst_bf16, stride_dst, stream);
}

size_t mmq_partial_bytes(int type, int64_t m, int64_t n, int64_t k) {
    switch (type) {
#define KAI_T(T) case T: return mmqs_partial_bytes<T>(m, n, k);
        KAI_T(Q8_0) KAI_T(Q4_0) KAI_T(Q4_K) KAI_T(Q6_K) KAI_T(Q2_K) KAI_T(IQ3_S)
#undef KAI_T
        default: return 0;
    }
}

}  // namespace kai
