// MMQ instantiations for Q6_K (kernel templates in kai_mmq.cuh, kai_mmqs.cuh
// and kai_mmqd.cuh).
#include "kai_mmqd.cuh"

namespace kai {
template void launch_mmq_type<Q6_K, false>(const void *, int64_t, int64_t, int64_t, const void *, const float *, void *,
                                       bool, int64_t, hipStream_t);
template void launch_mmq_type<Q6_K, true>(const void *, int64_t, int64_t, int64_t, const void *, const float *, void *,
                                      bool, int64_t, hipStream_t);
template void launch_mmqs<Q6_K>(const void *, int64_t, int64_t, int64_t, const uint8_t *, const float *, float *,
                             size_t, void *, bool, int64_t, hipStream_t);
template void launch_mmqd<Q6_K>(const void *, int64_t, int64_t, int64_t, const block_q8_1 *, const float *, void *,
                             bool, int64_t, hipStream_t);
template void launch_mmqd_image<Q6_K>(const void *, int64_t, int64_t, int64_t, const uint8_t *, const float *,
                                    void *, bool, int64_t, hipStream_t);
}  // namespace kai
