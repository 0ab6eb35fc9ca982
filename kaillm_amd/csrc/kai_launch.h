// Host-side launcher declarations shared by the kernel translation units and
// the C ABI (kai_abi.hip). Launchers validate what their kernels assume and
// throw kai::Error; the ABI turns that into a -1 status and a message.
#pragma once

#include <hip/hip_runtime.h>
#include <algorithm>
#include <atomic>
#include <climits>
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

// Devices (bit per index below 64) on which a kernel's dynamic LDS limit is raised.
using DeviceFlags = std::atomic<uint64_t>;
// Raise `kernel`'s dynamic LDS limit to `bytes` on the current device the first time it
// launches there. Callable from any host thread: the flags are atomic and the attribute
// call is idempotent, so threads racing on a device's first launch both set it; devices
// from index 64 on set it every launch.
inline void raise_dynamic_lds(const void *kernel, size_t bytes, DeviceFlags &done, const char *what) {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) throw Error("No HIP device");
    const uint64_t bit = device < 64 ? uint64_t(1) << device : 0;
    if (bit && (done.load(std::memory_order_acquire) & bit)) return;
    if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes)) != hipSuccess)
        throw Error(what);
    done.fetch_or(bit, std::memory_order_release);
}

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

// Destination row r of dst = source row row_order[r] (or r) of the tensor at file_offset of
// the file at path, with destination block j = source block block_order[j] (or j) within
// each row; returns once the copies on `stream` have completed.
void upload_rows(const char *path, int64_t file_offset, int64_t src_rows, int64_t row_bytes, const int64_t *row_order,
                 int64_t rows, int64_t block_bytes, const int64_t *block_order, void *dst, hipStream_t stream);

// `values` weight values (a whole number of blocks, rows back to back) to F32 (0), BF16 (1)
// or F16 (2) in row-major order.
void launch_dequantize(const void *w, int type, int64_t values, void *out, int out_dtype, hipStream_t stream);

void launch_prepare(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x, const ActLayout &out,
                    hipStream_t stream);
// Fused producers of the single-pass activation (kai_prepare.hip): x[..., view], silu(gate)
// * up from a merged [gate | up] row, and Gemma RMSNorm (+ residual) writing bf16 y.
// The legacy _C_gguf ops' Q8_1 activation (no row normalisation, ds = (half(d), half(sum x)),
// inverse 1) into the single-pass layout.
void launch_prepare_legacy(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x, const ActLayout &out,
                           hipStream_t stream);
void launch_prepare_view(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x, int64_t a, int64_t b,
                         int64_t s, const ActLayout &out, hipStream_t stream);
void launch_prepare_swiglu(const void *gate_up, int dtype, int64_t m, int64_t k, int64_t stride, const ActLayout &out,
                           hipStream_t stream);
void launch_norm_prepare(const void *x, int x_dtype, int64_t stride_x, const void *residual, int residual_dtype,
                         int64_t stride_r, float *residual_out, const float *weight32, float eps, void *y, int64_t m,
                         int64_t k, const ActLayout &out, hipStream_t stream);

// GEMV: dst[j*stride_dst + r] = inverse[j] * sum_b dot(W[r, b], y[j, b]) for j < m <= 16.
void launch_mmvq(int type, const void *weight, int64_t n, int64_t k, int64_t m, const block_q8_1 *y1,
                 const block_q8_1 *y2, const float *inverse, void *dst, bool dst_bf16, int64_t stride_dst,
                 hipStream_t stream);

// Products of more decode rows than the GEMV takes (k % 256 == 0), on int8 MFMA with the
// paired tile's arithmetic (two 32-value blocks per MFMA): the persistent paired GEMM
// (kai_mmqd.cuh: the activation staged once per workgroup, no scratch) where
// mmq_decode_persistent(type, n, k), the tiled paired kernel (launch_mmq) elsewhere.
// kai_fused_mmvq keeps the v_dot4 GEMV up to gemv_max_rows(type, k) rows before the tiled
// kernel and up to gemv_rows_before_persistent(type, k) before the persistent one. Measured on
// MI355X for every format at 1 to 8 rows on the BASELINE shapes: against the tiled kernel,
// IQ3_S 5120x17408 at 5-6 rows takes 103-116 us on the GEMV, 39 us tiled; Q6_K 5120x17408 at 4
// rows 40.8 / 37.4, but 5120x6144 16.1 / 16.4; Q4_K 7168x5120 at 4 rows 11.2 / 12.1. Against the
// persistent kernel (34816x5120): Q4_K at 3 / 4 rows 28.4 / 31.8 us on the GEMV, 28.5 / 28.6
// persistent; Q2_K at 2 / 3 rows 27.5 / 33.7, 28.2 / 28.3; IQ3_S at 4 / 5 rows 39.6 / 57.6,
// 43.4 / 42.8; Q4_0 16384x2048 at 6 / 8 rows 12.2 / 17.3, 14.7 / 15.0, 2048x8192 14.3 / 27.9,
// 15.3 / 15.7.
inline int gemv_max_rows(int type, int64_t k) {
    switch (type) {
        case Q4_0: case Q8_0: return 8;
        case Q6_K: return k >= 12288 ? 3 : 4;
        case Q4_K: case IQ3_S: return 4;
        default: return 3;
    }
}
// n: matrix rows, cus: compute units. Q4_0 on a matrix of fewer 16-row sets than CUs (where the
// persistent GEMM leaves CUs idle) keeps the GEMV, with its K split, up to 8 rows: measured on
// MI355X at 8 rows 2048x8192 17.27 -> 15.54 us and 3072x2048 10.41 -> 9.19 us (whole calls), but
// 16384x2048 16.31 -> 18.20 us.
inline int gemv_rows_before_persistent(int type, int64_t k, int64_t n, int cus) {
    switch (type) {
        case Q4_0: return (n + 15) / 16 < cus ? 8 : 6;
        case Q8_0: return 6;
        case Q4_K: return 3;
        case Q2_K: return 2;
        default: return gemv_max_rows(type, k);
    }
}
// Whether m activation rows fit the GEMV's LDS staging in one launch (more rows are split
// into launches that each stream the weights again).
inline bool gemv_one_launch(int64_t m, int64_t k, int two_pass) {
    return m * (two_pass ? 2 : 1) * (k / QK8_1) * 40 <= 160 * 1024 - 4096;
}
// dst[j*stride_dst + r] = inverse[j] * sum_b dot(W[r, b], y[j, b]) for j < m <= 8, k % 256 == 0.
void launch_mmq(int type, const void *weight, int64_t n, int64_t k, int64_t m, const block_q8_1 *y,
                const float *inverse, void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream);
bool mmq_decode_persistent(int type, int64_t n, int64_t k);
void launch_mmq_decode(int type, const void *weight, int64_t n, int64_t k, int64_t m, const block_q8_1 *y,
                       const float *inverse, void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream);
// A batched product over the batched path's activation of the type's layout (any k that
// is a whole number of the type's blocks): up to MMQS_MAX_ROWS rows on the small-M GEMM
// (kai_mmqs.cuh) reading the layout's small-M image, which may need
// mmq_partial_bytes(type, m, n, k) of scratch for K-chunk partial sums; more rows on the
// tiled int8 GEMM (kai_mmq.cuh) reading the plane. exact: the legacy MMQ's weight arithmetic
// (d * sc and dmin * m in fp32; differs from GGML MMQ's fp16 roundings for Q4_K only).
void launch_mmq_planes(int type, const void *weight, int64_t n, int64_t k, int64_t m, const uint8_t *plane,
                       const float *inverse, float *partial, size_t partial_bytes, void *dst, bool dst_bf16,
                       int64_t stride_dst, hipStream_t stream, bool exact = false);
// Partial-sum scratch of an m-row product: the small-M GEMM's (m <= 16), or with h the fp16
// GEMM's split-K sums.
size_t mmq_partial_bytes(int type, int64_t m, int64_t n, int64_t k, bool h = false);

// Batched path (kai_fused_mmq_run): activation planes of GGML's MMQ quantisation, one per
// layout a matrix of the group reads (D4: Q8_0, Q6_K, IQ3_S; DS4: Q4_0, Q4_K; D2S6: Q2_K).
// A plane holds 128-value blocks of MMQ_BLOCK_BYTES (16 header bytes, int8 qs[128]) in
// [K/128][m] order, K padded to a multiple of MMQ_ROW_PADDING with zero blocks (the
// reference's block_q8_1_mmq layout and padding, current_ggml_direct.cu:1025-1092,1136).
constexpr int MMQ_BLOCK_BYTES = 144, MMQ_ROW_PADDING = 512;
enum MmqLayout : int { MMQ_D4 = 0, MMQ_DS4 = 1, MMQ_D2S6 = 2 };
constexpr int mmq_layout(int type) {
    return type == Q4_0 || type == Q4_K ? MMQ_DS4 : type == Q2_K ? MMQ_D2S6 : MMQ_D4;
}
inline int64_t mmq_blocks128(int64_t k) { return (k + MMQ_ROW_PADDING - 1) / MMQ_ROW_PADDING * (MMQ_ROW_PADDING / 128); }
inline size_t mmq_plane_bytes(int64_t m, int64_t k) {
    return size_t(mmq_blocks128(k)) * size_t(m) * MMQ_BLOCK_BYTES;
}
// Up to MMQS_MAX_ROWS activation rows the preparation writes, in place of each plane, the
// small-M GEMM's LDS image of the same quantisation (kai_mmqs.cuh copies it as is). Per K
// step of 256 values (mmqs_image_step bytes): codes [block 8][row 16][32 bytes], octet o of
// row r at byte 8 * (o ^ ((r >> 2) & 3)); the activation scales d8 [8][16] fp32 (D4: d, DS4
// and D2S6: the stored fp16 d); then the min-term factors, fp32: DS4 [8][16] the stored fp16
// d * sum q (Q4_K) followed by [8][16] d8 * sum q (Q4_0); D2S6 [16][16] one per 16 values
// (the stored fp16 sums, d8 * sum q for the last 32 values of each 128). Rows past m and
// blocks past K are zero.
constexpr int MMQS_MAX_ROWS = 16;
constexpr int MMQS_CODE_BYTES = 8 * 16 * 32, MMQS_D8_BYTES = 8 * 16 * 4;
constexpr int mmqs_image_step(int layout) {
    return MMQS_CODE_BYTES + MMQS_D8_BYTES + (layout == MMQ_D4 ? 0 : 2 * MMQS_D8_BYTES);
}
__host__ __device__ inline int64_t mmqs_steps(int64_t k) { return (k + 255) / 256; }
inline size_t mmqs_image_bytes(int layout, int64_t k) { return size_t(mmqs_steps(k)) * mmqs_image_step(layout); }

// Above MMQS_MAX_ROWS rows the fp16 GEMM (kai_mmqh.cuh: Q4_K, Q4_0, Q8_0, IQ3_S and Q2_K) reads,
// per layout, an fp16 image of the same quantisation, rows padded to mmqh_mpad(m) with zeros
// and K to mmqh_kpad(k), laid out as the GEMM's MFMA operands:
//   codes  fp16 [kpad / 16][mpad][16]: each code times its block's scale, d * q rounded to fp32
//          then to fp16, with d the scale the reference's block dot takes (D4: fp32 d; DS4 and
//          D2S6: the stored fp16 d);
//   mins   the min-pass operands per superblock (none for D4): DS4 fp16 [ceil(k / 256)][mpad][32]
//          = [S_0..7 | Xhi_0..7 | Xlo_0..7 | 0 x 8], S the stored half(d * sum q) of the 8
//          blocks and X = half(d) * sum q the exact block sums as high and low fp16 parts
//          (hi = half(X), lo = half(X - hi)); D2S6 [..][mpad][64] = [Shi | Slo | Xhi | Xlo] over
//          the 16 groups of 16 values, S the stored half sums (d * sum q for the last 32 values of
//          each 128).
inline int64_t mmqh_mpad(int64_t m) { return (m + 31) / 32 * 32; }
inline int64_t mmqh_kpad(int64_t k) { return (k + 255) / 256 * 256; }  // whole 256-value steps
inline size_t mmqh_codes_bytes(int64_t m, int64_t k) { return size_t(mmqh_kpad(k)) * size_t(mmqh_mpad(m)) * 2; }
inline size_t mmqh_mins_bytes(int layout, int64_t m, int64_t k) {
    return layout == MMQ_D4 ? 0 : size_t((k + 255) / 256) * size_t(mmqh_mpad(m)) * (layout == MMQ_DS4 ? 64 : 128);
}
struct MmqhImage {
    uint8_t *codes = nullptr, *mins = nullptr;
};

struct MmqPlanes {
    uint8_t *d4, *ds4, *d2s6;  // null when no matrix of the group reads that layout
    float *inverse;
    bool image;          // small-M images (m <= MMQS_MAX_ROWS) instead of planes
    bool legacy = false;  // the legacy ops' quantisation (launch_prepare_legacy's), D4 / DS4 only
    MmqhImage h[3] = {};  // the fp16 GEMM's images per layout (null codes when not read)
};
// Whether kai_fused_mmq_run's m-row product of an n-row matrix with this type runs on the fp16
// GEMM (reading the layout's fp16 image) rather than the int8 kernels (reading the plane): above
// 16 rows, every format but Q6_K. Measured at 80 rows (whole calls): Q4_K 34816 x 5120 111.7 us
// on the int8 tile kernel, 107.0 us on the fp16 GEMM; 5120 x 17408 90 / 53 us. (n is the
// matrix's rows, for the rule's callers.)
inline bool mmq_uses_h(int type, int64_t m, int64_t n) {
    (void)n;
    return m > MMQS_MAX_ROWS &&
           (type == Q4_K || type == Q4_0 || type == Q8_0 || type == IQ3_S || type == Q2_K);
}
void launch_mmq_h(int type, const void *weight, int64_t n, int64_t k, int64_t m, const MmqhImage &image,
                  const float *inverse, float *partial, size_t partial_bytes, void *dst, bool dst_bf16,
                  int64_t stride_dst, hipStream_t stream);

void launch_prepare_mmq(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x, const MmqPlanes &planes,
                        hipStream_t stream);

// Measurement kernels (kai_peaks.hip): the MFMA rate of one instruction kind, the LDS read
// rate and a streaming copy; kinds are the KAI_PEAK_* codes of include/kai_peaks.h.
void launch_peak_mfma(int kind, int64_t iters, int blocks, int threads, float *out, hipStream_t stream);
int64_t peak_mfma_ops(int kind);
void launch_peak_lds(int64_t iters, int blocks, int threads, float *out, hipStream_t stream);
void launch_peak_copy(const void *src, void *dst, int64_t bytes, int blocks, hipStream_t stream);

}  // namespace kai
