// MMQ dispatch by weight type (instantiations live in kai_mmq_<type>.hip).
#include "kai_launch.h"

namespace kai {

template <int TYPE, bool PLANES>
void launch_mmq_type(const void *weight, int64_t n, int64_t k, int64_t m, const void *act, const float *inverse,
                     void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream);

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
                       const float *inverse, void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream) {
    dispatch<true>(type, weight, n, k, m, plane, inverse, dst, dst_bf16, stride_dst, stream);
}

}  // namespace kai
