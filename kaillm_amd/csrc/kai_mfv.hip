// fp16-MFMA small-M GEMM: dispatch by weight type (kernel template in kai_mfv.cuh).
#include "kai_mfv.cuh"

namespace kai {

bool mfv_supported(int type) { return type == Q4_K; }

void launch_mfv(int type, const void *weight, int64_t n, int64_t k, int64_t m, const MmfAct &act, float *partial,
                void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream) {
    if (k % 256 || m < 1 || m > MFV_MAX_ROWS || n > INT32_MAX || !mmf_weight_fits(type, n, k))
        throw Error("fp16-MFMA small-M GEMM: K must be a multiple of 256, M at most 16 and the weight below 4 GiB");
    switch (type) {
        case Q4_K: launch_mfv_type<Q4_K>(weight, n, k, m, act, partial, dst, dst_bf16, stride_dst, stream); break;
        default: throw Error("Unsupported weight type for the fp16-MFMA small-M GEMM");
    }
}

}  // namespace kai
