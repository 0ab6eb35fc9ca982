// MMQ dispatch by weight type (instantiations live in kai_mmq_<type>.hip).
#include "kai_mmqd.cuh"

namespace kai {

// The kernels are compiled in the per-type files; this file only dispatches.
#define KAI_EXTERN(T) \
    extern template void launch_mmq_type<T, false>(const void *, int64_t, int64_t, int64_t, const void *, \
                                                   const float *, void *, bool, int64_t, hipStream_t); \
    extern template void launch_mmq_type<T, true>(const void *, int64_t, int64_t, int64_t, const void *, \
                                                  const float *, void *, bool, int64_t, hipStream_t); \
    extern template void launch_mmqs<T>(const void *, int64_t, int64_t, int64_t, const uint8_t *, const float *, \
                                        float *, size_t, void *, bool, int64_t, hipStream_t); \
    extern template void launch_mmqd<T>(const void *, int64_t, int64_t, int64_t, const block_q8_1 *, const float *, \
                                        void *, bool, int64_t, hipStream_t); \
    extern template void launch_mmqd_image<T>(const void *, int64_t, int64_t, int64_t, const uint8_t *, const float *, \
                                              void *, bool, int64_t, hipStream_t);
KAI_EXTERN(Q8_0) KAI_EXTERN(Q4_0) KAI_EXTERN(Q4_K) KAI_EXTERN(Q6_K) KAI_EXTERN(Q2_K) KAI_EXTERN(IQ3_S)
#undef KAI_EXTERN
extern template void launch_mmq_type<Q4_K, true, true>(const void *, int64_t, int64_t, int64_t, const void *,
                                                       const float *, void *, bool, int64_t, hipStream_t);
extern template void launch_mmqs<Q4_K, true>(const void *, int64_t, int64_t, int64_t, const uint8_t *, const float *,
                                             float *, size_t, void *, bool, int64_t, hipStream_t);
extern template void launch_mmqd_image<Q4_K, true>(const void *, int64_t, int64_t, int64_t, const uint8_t *,
                                                   const float *, void *, bool, int64_t, hipStream_t);

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

bool mmq_decode_persistent(int type, int64_t n, int64_t k) {
    switch (type) {
#define KAI_T(T) case T: return mmqd_suits<T, false>(n, k, device_cu_count());
        KAI_T(Q8_0) KAI_T(Q4_0) KAI_T(Q4_K) KAI_T(Q6_K) KAI_T(Q2_K) KAI_T(IQ3_S)
#undef KAI_T
        default: return false;
    }
}

void launch_mmq_decode(int type, const void *weight, int64_t n, int64_t k, int64_t m, const block_q8_1 *y,
                       const float *inverse, void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream) {
    switch (type) {
#define KAI_T(T) case T: launch_mmqd<T>(weight, n, k, m, y, inverse, dst, dst_bf16, stride_dst, stream); break;
        KAI_T(Q8_0) KAI_T(Q4_0) KAI_T(Q4_K) KAI_T(Q6_K) KAI_T(Q2_K) KAI_T(IQ3_S)
#undef KAI_T
        default: throw Error("Unsupported fused MMQ weight type");
    }
}

// Whether up to MMQS_MAX_ROWS rows of this matrix run on the persistent GEMM over the image
// (no partial sums) rather than the small-M GEMM.
static bool image_persistent(int type, int64_t n, int64_t k) {
    switch (type) {
#define KAI_T(T) case T: return mmqd_suits<T, true>(n, k, device_cu_count());
        KAI_T(Q8_0) KAI_T(Q4_0) KAI_T(Q4_K) KAI_T(Q6_K) KAI_T(Q2_K) KAI_T(IQ3_S)
#undef KAI_T
        default: return false;
    }
}

void launch_mmq_planes(int type, const void *weight, int64_t n, int64_t k, int64_t m, const uint8_t *plane,
                       const float *inverse, float *partial, size_t partial_bytes, void *dst, bool dst_bf16,
                       int64_t stride_dst, hipStream_t stream, bool exact) {
    const bool small = m <= MMQS_MAX_ROWS, persistent = small && image_persistent(type, n, k);
    if (exact && type == Q4_K) {  // the only format whose batched weight arithmetic rounds
        if (persistent)
            launch_mmqd_image<Q4_K, true>(weight, n, k, m, plane, inverse, dst, dst_bf16, stride_dst, stream);
        else if (small)
            launch_mmqs<Q4_K, true>(weight, n, k, m, plane, inverse, partial, partial_bytes, dst, dst_bf16, stride_dst,
                                    stream);
        else
            launch_mmq_type<Q4_K, true, true>(weight, n, k, m, plane, inverse, dst, dst_bf16, stride_dst, stream);
        return;
    }
    if (exact && type != Q8_0 && type != Q6_K) throw Error("Exact batched arithmetic covers Q4_K, Q8_0 and Q6_K");
    if (small) {
        switch (type) {
#define KAI_T(T) \
    case T: \
        if (persistent) launch_mmqd_image<T>(weight, n, k, m, plane, inverse, dst, dst_bf16, stride_dst, stream); \
        else launch_mmqs<T>(weight, n, k, m, plane, inverse, partial, partial_bytes, dst, dst_bf16, stride_dst, stream); \
        return;
            KAI_T(Q8_0) KAI_T(Q4_0) KAI_T(Q4_K) KAI_T(Q6_K) KAI_T(Q2_K) KAI_T(IQ3_S)
#undef KAI_T
            default: throw Error("Unsupported fused MMQ weight type");
        }
    }
    dispatch<true>(type, weight, n, k, m, plane, inverse, dst, dst_bf16, stride_dst, stream);
}

size_t mmqh_partial_bytes_of(int type, int64_t m, int64_t n, int64_t k);  // kai_mmqh.hip

// The small-M GEMM's partial sums, whichever GEMM the launch picks: the scratch query takes no
// device, and a matrix the persistent GEMM takes leaves them unused. h: the fp16 GEMM's
// split-K sums.
size_t mmq_partial_bytes(int type, int64_t m, int64_t n, int64_t k, bool h) {
    if (h) return mmqh_partial_bytes_of(type, m, n, k);
    switch (type) {
#define KAI_T(T) case T: return mmqs_partial_bytes<T>(m, n, k);
        KAI_T(Q8_0) KAI_T(Q4_0) KAI_T(Q4_K) KAI_T(Q6_K) KAI_T(Q2_K) KAI_T(IQ3_S)
#undef KAI_T
        default: return 0;
    }
}

}  // namespace kai
