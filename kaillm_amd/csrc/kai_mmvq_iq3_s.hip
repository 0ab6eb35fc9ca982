// GEMV instantiations for IQ3_S (kernel template in kai_mmvq.cuh).
#include "kai_mmvq.cuh"

namespace kai {
template void launch_mmvq_type<IQ3_S>(const void *, int64_t, int64_t, int64_t, const block_q8_1 *, const block_q8_1 *,
                                   const float *, void *, bool, int64_t, hipStream_t);
}  // namespace kai
