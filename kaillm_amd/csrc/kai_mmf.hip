// fp16-MFMA prefill GEMM: dispatch by weight type (kernel template in kai_mmf.cuh).
#include "kai_mmf.cuh"

namespace kai {

bool mmf_supported(int type) { return type == Q4_K; }

void launch_mmf(int type, const void *weight, int64_t n, int64_t k, int64_t m, const MmfAct &act, void *dst,
                bool dst_bf16, int64_t stride_dst, hipStream_t stream) {
    if (k % 256 || n % 4 || m < 1 || m * k * 2 > INT32_MAX || n > INT32_MAX || !mmf_weight_fits(type, n, k))
        throw Error("fp16-MFMA GEMM: K must be a multiple of 256, N of 4, M*K*2 below 2^31 and the weight below 4 GiB");
    switch (type) {
        case Q4_K: launch_mmf_type<Q4_K>(weight, n, k, m, act, dst, dst_bf16, stride_dst, stream); break;
        default: throw Error("Unsupported weight type for the fp16-MFMA GEMM");
    }
}

}  // namespace kai
