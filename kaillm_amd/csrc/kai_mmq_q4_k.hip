// MMQ instantiations for Q4_K (kernel templates in kai_mmq.cuh, kai_mmqs.cuh,
// kai_mmqd.cuh and kai_mmqh.cuh).
#include "kai_mmqd.cuh"
#include "kai_mmqh.cuh"

namespace kai {
template void launch_mmq_type<Q4_K, false>(const void *, int64_t, int64_t, int64_t, const void *, const float *, void *,
                                       bool, int64_t, hipStream_t);
template void launch_mmq_type<Q4_K, true>(const void *, int64_t, int64_t, int64_t, const void *, const float *, void *,
                                      bool, int64_t, hipStream_t);
template void launch_mmqs<Q4_K>(const void *, int64_t, int64_t, int64_t, const uint8_t *, const float *, float *,
                             size_t, void *, bool, int64_t, hipStream_t);
// the legacy ops' exact weight products
template void launch_mmq_type<Q4_K, true, true>(const void *, int64_t, int64_t, int64_t, const void *, const float *,
                                                void *, bool, int64_t, hipStream_t);
template void launch_mmqs<Q4_K, true>(const void *, int64_t, int64_t, int64_t, const uint8_t *, const float *, float *,
                                      size_t, void *, bool, int64_t, hipStream_t);
template void launch_mmqd<Q4_K>(const void *, int64_t, int64_t, int64_t, const block_q8_1 *, const float *, void *,
                             bool, int64_t, hipStream_t);
template void launch_mmqd_image<Q4_K>(const void *, int64_t, int64_t, int64_t, const uint8_t *, const float *,
                                    void *, bool, int64_t, hipStream_t);
template void launch_mmqd_image<Q4_K, true>(const void *, int64_t, int64_t, int64_t, const uint8_t *,
                                            const float *, void *, bool, int64_t, hipStream_t);
template void launch_mmqh<Q4_K>(const void *, int64_t, int64_t, int64_t, const MmqhArgs &, const float *, float *,
                              size_t, void *, bool, int64_t, hipStream_t);
}  // namespace kai
