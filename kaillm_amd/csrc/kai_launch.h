// Host-side launcher declarations shared by the kernel translation units and
// the C ABI (kai_abi.hip). Launchers validate what their kernels assume and
// throw kai::Error; the ABI turns that into a -1 status and a message.
#pragma once

#include <hip/hip_runtime.h>
#include <algorithm>
#include <stdexcept>
#include <string>

#include "kai_device.h"
#include "kai_formats.h"

namespace kai {

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

constexpr int MMVQ_MAX_ROWS = 16;  // activation rows the GEMV kernel is built for

// Compute units of the current device (cached per device).
int device_cu_count();

// Activation buffer layout (the reference's, byte for byte): [pass1: m*(k/32) Q8_1 blocks,
// 256-aligned][pass2 when two_pass][inverse: m floats, 256-aligned].
inline size_t align256(size_t bytes) { return (bytes + 255) & ~size_t(255); }
inline size_t q8_1_pass_bytes(int64_t m, int64_t k) {
    return align256(size_t(m) * size_t(k / QK8_1) * sizeof(block_q8_1));
}

// Where each region of an activation buffer starts.
struct ActLayout {
    block_q8_1 *y1;
    block_q8_1 *y2;  // null unless two_pass
    float *inverse;
};
inline size_t activation_bytes(int64_t m, int64_t k, int two_pass) {
    return q8_1_pass_bytes(m, k) * (two_pass ? 2 : 1) + align256(size_t(m) * sizeof(float));
}
inline ActLayout activation_layout(void *activation, int64_t m, int64_t k, int two_pass) {
    char *base = static_cast<char *>(activation);
    const size_t pass = q8_1_pass_bytes(m, k);
    return {reinterpret_cast<block_q8_1 *>(base), two_pass ? reinterpret_cast<block_q8_1 *>(base + pass) : nullptr,
            reinterpret_cast<float *>(base + pass * (two_pass ? 2 : 1))};
}

void launch_prepare(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x, const ActLayout &out,
                    hipStream_t stream);

// GEMV: dst[j*stride_dst + r] = inverse[j] * sum_b dot(W[r, b], y[j, b]) for j < m <= 16.
void launch_mmvq(int type, const void *weight, int64_t n, int64_t k, int64_t m, const block_q8_1 *y1,
                 const block_q8_1 *y2, const float *inverse, void *dst, bool dst_bf16, int64_t stride_dst,
                 hipStream_t stream);

// Batched GEMM (int8 MFMA), k % 256 == 0: dst[j*stride_dst + r] as above. kai_fused_mmvq uses
// it from MMQ_MIN_ROWS rows on (below that the v_dot4 GEMV streams faster).
constexpr int MMQ_MIN_ROWS = 3;
void launch_mmq(int type, const void *weight, int64_t n, int64_t k, int64_t m, const block_q8_1 *y,
                const float *inverse, void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream);

}  // namespace kai
