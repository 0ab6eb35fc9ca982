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

// Batched GEMM (int8 MFMA), k % 256 == 0: dst[j*stride_dst + r] as above. kai_fused_mmvq uses
// it above gemv_max_rows(type) rows; up to there the v_dot4 GEMV is faster (measured on
// MI355X for every format at 3 to 8 rows on the BASELINE shapes, against the paired 8-row
// MMQ tile: IQ3_S 5120x17408 at 5-6 rows takes 103-116 us on the GEMV, 65 us on MMQ).
inline int gemv_max_rows(int type) {
    switch (type) {
        case Q4_0: case Q8_0: return 8;
        case Q4_K: case Q6_K: case IQ3_S: return 4;
        default: return 3;
    }
}
// Whether m activation rows fit the GEMV's LDS staging in one launch (more rows are split
// into launches that each stream the weights again).
inline bool gemv_one_launch(int64_t m, int64_t k, int two_pass) {
    return m * (two_pass ? 2 : 1) * (k / QK8_1) * 40 <= 160 * 1024 - 4096;
}
void launch_mmq(int type, const void *weight, int64_t n, int64_t k, int64_t m, const block_q8_1 *y,
                const float *inverse, void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream);

// Prefill GEMM on fp16 MFMA (kai_mmf.cuh) for K-quant weights from MMF_MIN_ROWS rows on.
// Its activation operands, one region each, 256-aligned: a16 [m][k] fp16 = half(d8 * q8) of
// the row's Q8_1 blocks, in the GEMM's K order (mmf_a16_run); t32 [m][k/256][64 bytes] and
// t16 [m][k/256][96 bytes], the min-term operands of 32- and 16-value sums (present when a
// matrix of the group needs them); inverse [m] fp32.
// Tiles of the fp16-MFMA GEMM (kai_mmf.cuh: 256 weight rows x 96 activation rows); below
// MMF_MIN_TILES workgroups it fills too little of the chip and the int8 kernel is faster
// (measured crossover on MI355X at 120-170 tiles).
constexpr int MMF_TILE_N = 256, MMF_TILE_M = 96, MMF_MIN_TILES = 160;
constexpr int MMF_MIN_ROWS = 128;
// K order of a16 within a superblock, in runs of 8 values: the GEMM's step j (64 values)
// holds at run 8 j + 4 h + g, for lane group g and half h, block 4 (j / 2) + 2 (g / 2) + h
// at positions 16 (g % 2) + 8 (j % 2) + [0, 8). Every step then takes, per weight row and
// lane group, 8 code bytes of one 16-byte run of the Q4_K superblock (a pair of steps
// shares it), so a lane loads its codes as one 16-byte piece per two steps. Returns the
// run of block `block` (0..7) positions [8 run, 8 run + 8).
__host__ __device__ inline int mmf_a16_run(int block, int run) {
    const int j = 2 * (block >> 2) + (run & 1), g = 2 * ((block >> 1) & 1) + (run >> 1), h = block & 1;
    return 8 * j + 4 * h + g;
}
struct MmfAct {
    uint16_t *a16;
    uint8_t *t32;
    uint8_t *t16;
    float *inverse;
};
bool mmf_supported(int type);
inline bool mmf_uses_t32(int type) { return type == Q4_K; }
inline bool mmf_uses_t16(int type) { return type == Q2_K; }
// Whether an m-row product with this matrix runs on the fp16-MFMA GEMM (its weight is
// addressed through one buffer descriptor: below 4 GiB).
inline bool mmf_weight_fits(int type, int64_t n, int64_t k) {
    return n * (k / 256) * block_bytes(type) <= int64_t(UINT32_MAX);
}
inline bool mmf_route(int type, int64_t m, int64_t n, int64_t k) {
    const int64_t tiles = ((m + MMF_TILE_M - 1) / MMF_TILE_M) * ((n + MMF_TILE_N - 1) / MMF_TILE_N);
    return mmf_supported(type) && m >= MMF_MIN_ROWS && tiles >= MMF_MIN_TILES && k % 256 == 0 &&
           m * k * 2 <= INT32_MAX && n % 4 == 0 && mmf_weight_fits(type, n, k);
}
inline size_t mmf_bytes(int64_t m, int64_t k, bool t32, bool t16) {
    return align256(size_t(m) * size_t(k) * 2) + (t32 ? align256(size_t(m) * size_t(k / 256) * 64) : 0) +
           (t16 ? align256(size_t(m) * size_t(k / 256) * 96) : 0) + align256(size_t(m) * sizeof(float));
}
inline MmfAct mmf_layout(void *base, int64_t m, int64_t k, bool t32, bool t16) {
    char *p = static_cast<char *>(base);
    MmfAct a{};
    a.a16 = reinterpret_cast<uint16_t *>(p);
    p += align256(size_t(m) * size_t(k) * 2);
    if (t32) {
        a.t32 = reinterpret_cast<uint8_t *>(p);
        p += align256(size_t(m) * size_t(k / 256) * 64);
    }
    if (t16) {
        a.t16 = reinterpret_cast<uint8_t *>(p);
        p += align256(size_t(m) * size_t(k / 256) * 96);
    }
    a.inverse = reinterpret_cast<float *>(p);
    return a;
}
void launch_prepare_mmf(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x, const MmfAct &out,
                        hipStream_t stream);

// Small-M GEMM on fp16 MFMA (kai_mfv.cuh), up to MFV_MAX_ROWS activation rows, on the
// operands of launch_prepare_mmf. Workgroups of 64 weight rows; K is split over
// mfv_splits(n, k) workgroups (doubling while there are fewer than two workgroups per CU of
// a 256-CU device and every split keeps at least 4 superblocks), whose fp32 partial sums
// ([splits][m][n], mfv_partial_bytes) are added by a second kernel.
constexpr int MFV_MAX_ROWS = 16;
inline int mfv_splits(int64_t n, int64_t k) {
    const int64_t wgs = (n + 63) / 64, nsb = k / 256;
    int ks = 1;
    while (ks < 8 && wgs * ks < 512 && nsb / (2 * ks) >= 4) ks *= 2;
    return ks;
}
inline size_t mfv_partial_bytes(int64_t m, int64_t n, int64_t k) {
    const int ks = mfv_splits(n, k);
    return ks > 1 ? align256(size_t(ks) * size_t(m) * size_t(n) * sizeof(float)) : 0;
}
bool mfv_supported(int type);
inline bool mfv_route(int type, int64_t m, int64_t n, int64_t k) {
    return mfv_supported(type) && m >= 1 && m <= MFV_MAX_ROWS && k % 256 == 0 && n <= INT32_MAX &&
           mmf_weight_fits(type, n, k);
}
// Whether an m-row product with this matrix runs on one of the fp16-MFMA kernels.
inline bool fp16_route(int type, int64_t m, int64_t n, int64_t k) {
    return mmf_route(type, m, n, k) || mfv_route(type, m, n, k);
}
void launch_mfv(int type, const void *weight, int64_t n, int64_t k, int64_t m, const MmfAct &act, float *partial,
                void *dst, bool dst_bf16, int64_t stride_dst, hipStream_t stream);
void launch_mmf(int type, const void *weight, int64_t n, int64_t k, int64_t m, const MmfAct &act, void *dst,
                bool dst_bf16, int64_t stride_dst, hipStream_t stream);

}  // namespace kai
