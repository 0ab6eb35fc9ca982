// MMQ instantiations for IQ3_S (kernel template in kai_mmq.cuh).
#include "kai_mmq.cuh"

namespace kai {
template void launch_mmq_type<IQ3_S>(const void *, int64_t, int64_t, int64_t, const block_q8_1 *, const float *, void *,
                                  bool, int64_t, hipStream_t);
}  // namespace kai
