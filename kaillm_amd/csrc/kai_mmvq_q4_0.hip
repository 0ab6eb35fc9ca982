// GEMV instantiations for Q4_0 (kernel template in kai_mmvq.cuh).
#include "kai_mmvq.cuh"

namespace kai {
template void launch_mmvq_type<Q4_0>(const void *, int64_t, int64_t, int64_t, const block_q8_1 *, const block_q8_1 *,
                                   const float *, void *, bool, int64_t, hipStream_t);
}  // namespace kai
