// MMQ instantiations for IQ3_S (kernel template in kai_mmq.cuh).
#include "kai_mmq.cuh"

namespace kai {
template void launch_mmq_type<IQ3_S, false>(const void *, int64_t, int64_t, int64_t, const void *, const float *, void *,
                                       bool, int64_t, hipStream_t);
template void launch_mmq_type<IQ3_S, true>(const void *, int64_t, int64_t, int64_t, const void *, const float *, void *,
                                      bool, int64_t, hipStream_t);
}  // namespace kai
