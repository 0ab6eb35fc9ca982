/*
 * CPU oracle for the GGUF dequant-fused quantized linear path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or, for the baseline, as the timed CPU restatement). The product library
 * (kaillm_amd/libkai_hip.so) never links or calls it.
 *
 * It restates, in plain C with IEEE float arithmetic, what the reference path
 * computes:
 *   - Q8_1 activation preparation of kai_dual::prepare_dual
 *     (vllm_gguf_plugin/native/kernels/kai_dual_mmvq.cuh:147-254) and the
 *     activation buffer layout of current_ggml_direct.cu:808-839;
 *   - the per-format block dot products vec_dot_{q8_0,q4_0,q4_K,q6_K,q2_K,iq3_s}_q8_1
 *     (llama.cpp @0c1e570, not vendored; in-tree text csrc/gguf/vecdotq.cuh), evaluated
 *     as exact integer block sums times the stored fp16 scales, accumulated in FP64;
 *   - the GEMV epilogue y[j, r] = inverse[j] * sum_b dot(W[r, b], q8[j, b])
 *     (kai_dual_mmvq.cuh:258-327);
 *   - the batched path of kai_fused_mmq_run (current_ggml_direct.cu:967-1265): row_scale,
 *     GGML's MMQ activation quantisation quantize_scaled with its D4 / DS4 / D2S6 layouts
 *     (:978-1092), and GGML MMQ's block arithmetic per format (upstream ggml mmq.cuh
 *     @0c1e570, not vendored: restated from its published tile loaders and MMA dots);
 *   - block dequantization per gguf-py quants.py (:242-252, :397-402, :407-429,
 *     :476-523, :553-573, :1097-1125);
 *   - the fused activation producers kai_dual::prepare_view / prepare_swiglu /
 *     norm_prepare (kai_prepare_ext.cuh:121-251), with their two unspecified steps (exp,
 *     and the order of the norm's sum of squares) fixed as the HIP kernels fix them;
 *   - the legacy _C_gguf ops: quantize_q8_1 and the legacy MMVQ / MMQ block forms
 *     (csrc/gguf/gguf_kernel.cu:32-290, vecdotq.cuh).
 * Each function names the reference lines it follows.
 *
 * Pinning (tests/test_oracle_*.py): fp16/bf16 conversion against numpy; Q8_1
 * preparation against closed-form special cases and invariants; dequantization
 * against hand-assembled known-answer blocks; the block dots against
 * dequantize-then-dot in FP64 (an independent route through the layout); the
 * IQ3_S grid against the older vendored table (tests/golden/gen_iq3s_grid.py); the
 * producers against FP64 references (exp within 2 ulp of libm's double exp, RMSNorm
 * within bf16 rounding), the view as a transposed copy prepared by oracle_prepare, and
 * the SwiGLU dtype roundings against numpy's own conversions; the legacy quantiser against
 * closed forms (ties, signed zero, fp16 overflow / underflow, the butterfly's grouping) and
 * the legacy products against dense FP64 routes (tests/test_oracle_legacy.py).
 */
#ifndef KAI_ORACLE_H
#define KAI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORACLE_Q4_0 = 2,
    ORACLE_Q8_0 = 8,
    ORACLE_Q8_1 = 9,
    ORACLE_Q2_K = 10,
    ORACLE_Q4_K = 12,
    ORACLE_Q6_K = 14,
    ORACLE_IQ3_S = 21,
};

/* Elements and bytes per block; 0 for an unsupported type. */
int oracle_block_elems(int type);
int oracle_block_bytes(int type);

/* IEEE half <-> float (round to nearest even), bf16 -> float. */
float oracle_half_to_float(uint16_t h);
uint16_t oracle_float_to_half(float f);
float oracle_bf16_to_float(uint16_t b);

/* Activation buffer bytes: [pass1 m*(k/32)*36, 256-aligned][pass2][inverse m*4, 256-aligned]. */
size_t oracle_activation_bytes(int64_t m, int64_t k, int two_pass);

/* Q8_1 activation preparation. x_dtype: 0 f32, 1 bf16, 2 f16. Returns 0 or -1. */
int oracle_prepare(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x,
                   void *activation, int two_pass);

/* float -> bf16 bits (round to nearest even, NaN kept quiet). */
uint16_t oracle_float_to_bf16(float f);

/* e^x by the fixed operation sequence of the HIP SwiGLU producer (Cody-Waite + degree-7
 * Taylor); within 2 ulp of e^x. */
float oracle_expf(float x);

/* Fused producers of the single-pass activation (returns 0 or -1):
 * view (stored column c reads x column ((c/s)%a)*b*s + (c/(a*s))*s + c%s), SwiGLU of a
 * merged [gate | up] row, and Gemma RMSNorm (+ residual) writing bf16 y and the fp32
 * residual stream. The norm's sum of squares follows the HIP kernel's fixed order. */
int oracle_prepare_view(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x,
                        void *activation, int64_t a, int64_t b, int64_t s);
int oracle_prepare_swiglu(const void *gate_up, int dtype, int64_t m, int64_t k, int64_t stride,
                          void *activation);
int oracle_norm_prepare(const void *x, int x_dtype, int64_t stride_x, const void *residual,
                        int residual_dtype, int64_t stride_r, float *residual_out,
                        const float *weight32, float eps, uint16_t *y, int64_t m, int64_t k,
                        void *activation);

/* Dequantize one row of k elements. Returns 0 or -1. */
int oracle_dequantize_row(int type, const uint8_t *row, int64_t k, float *out);

/* Block dot of weight row r (n rows, k columns) with activation row j, FP64.
 * out[j * n + r] = inverse[j] * sum_b dot(...) (+ pass 2 when two_pass). */
int oracle_mul_mat(int type, const uint8_t *weight, int64_t n, int64_t k, int64_t m,
                   const void *activation, int two_pass, double *out, int threads);

/* Same arithmetic as oracle_mul_mat, written to float out with stride. Used as the
 * CPU baseline timing leg. */
int oracle_mul_mat_f32(int type, const uint8_t *weight, int64_t n, int64_t k, int64_t m,
                       const void *activation, int two_pass, float *out, int64_t stride_out,
                       int threads);

/* ---- Batched path (kai_fused_mmq_run, more than 8 rows; current_ggml_direct.cu:967-1265).
 *
 * Activation: the same power-of-two row normalisation (row_scale, :978-1022), then GGML's
 * MMQ quantisation of the normalised row (quantize_scaled, :1025-1092) into one "plane"
 * per layout: 128-value blocks of 144 bytes {16 bytes of scales/sums; int8 qs[128]} in
 * [K/128][m] order, K padded to a multiple of 512 with zero blocks (:1136). Per group of
 * G values (G = 64 for D2S6, else 32): amax = max|v|, d_inv = 127/amax, q = roundf(v*d_inv)
 * (NaN -> 0, saturated to int8), d = 1/d_inv. The 16 header bytes hold
 *   D4   (Q8_0, Q6_K, IQ3_S): fp32 d per 32 values;
 *   DS4  (Q4_0, Q4_K):        half2 (d, d*sum q) per 32 values;
 *   D2S6 (Q2_K):              half d per 64 values (2), then half d*sum q per 16 values for
 *                             the first 96 values (6); the last 32 carry no stored sum. */
enum { ORACLE_MMQ_D4 = 0, ORACLE_MMQ_DS4 = 1, ORACLE_MMQ_D2S6 = 2 };

/* Layout a weight type's MMQ reads (-1 if unsupported); 128-value blocks per row; bytes
 * of one plane. */
int oracle_mmq_layout(int type);
int64_t oracle_mmq_blocks128(int64_t k);
size_t oracle_mmq_plane_bytes(int64_t m, int64_t k);

/* row_scale + quantize_scaled for one layout: writes inverse[m] and the plane. */
int oracle_prepare_mmq(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x,
                       int layout, uint8_t *plane, float *inverse);

/* GGML MMQ over a plane of the type's layout, in FP64 from exact integer block dots:
 * out[j * n + r] = inverse[j] * sum over blocks. Weight-side scales are those GGML's
 * MMQ tile loaders form (half(d*sc), half(dmin*m) for Q4_K and Q2_K). */
int oracle_mul_mat_mmq(int type, const uint8_t *weight, int64_t n, int64_t k, int64_t m,
                       const uint8_t *plane, const float *inverse, double *out, int threads);

/* ---- Legacy _C_gguf ops (csrc/gguf/gguf_kernel.cu:32-290, bound as torch ops
 * ggml_mul_mat_vec_a8 / ggml_mul_mat_a8 at csrc/torch_bindings.cpp:22-53).
 *
 * Activation: quantize_q8_1 (gguf_kernel.cu:32-69), per 32-value block with no row
 * normalisation: amax = max|x|, d = amax / 127, q = amax == 0 ? 0 : roundf(x / d),
 * ds = (half(d), half(sum x)), the sum being the kernel's 32-lane xor butterfly (masks 16,
 * 8, 4, 2, 1; lane 0 ends with ((x0 + x16) + (x8 + x24)) + ... in that grouping). Written
 * in oracle_prepare's single-pass layout with inverse[row] = 1. The reference spaces its
 * rows K padded to 512 (:74); the padding blocks are zero and no product reads them, so
 * the dense layout carries the same products. */
int oracle_prepare_legacy(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x,
                          void *activation);

/* Products over a legacy activation, FP64 from exact integer block dots.
 * batched = 0: ggml_mul_mat_vec_a8's MMVQ block dots (mmvq.cuh:2-39), the same
 * formulas as oracle_mul_mat. batched = 1: ggml_mul_mat_a8's MMQ block dots (mmq.cuh);
 * they differ from the MMVQ ones only for Q4_K, whose min term takes the stored
 * half(sum x) (vecdotq.cuh:353-377: sumf_m += ds8.y * m) where MMVQ takes d8 * sum q
 * (:328-351). out[j * n + r]. */
int oracle_mul_mat_legacy(int type, const uint8_t *weight, int64_t n, int64_t k, int64_t m,
                          const void *activation, int batched, double *out, int threads);

/* Library identity string (build flags), for reports. */
const char *oracle_build_info(void);

#ifdef __cplusplus
}
#endif
#endif
