/*
 * kai_hip: C ABI of the MI355X (gfx950) GGUF dequant-fused quantized linear.
 *
 * Drop-in for the exports that the reference's Python bridge binds with ctypes
 * (vllm_gguf_plugin/quantization/native_fused.py:52-85) from its CUDA library
 * (vllm_gguf_plugin/native/kernels/current_ggml_direct.cu). Same names, argument
 * order and meaning, status conventions:
 *   - every pointer is device memory owned by the caller (PyTorch); the library
 *     performs no allocation, copy or synchronisation on these entry points;
 *   - `stream` is a hipStream_t passed as uintptr_t; 0 is the null stream;
 *   - activation dtype codes: 0 = f32, 1 = bf16, 2 = f16;
 *   - int entry points return 0 on success and -1 on error, size queries return
 *     0 on error; the message is kept per host thread (current_direct_error);
 *   - weight types are GGML ids: Q4_0 = 2, Q8_0 = 8, Q2_K = 10, Q4_K = 12,
 *     Q6_K = 14, IQ3_S = 21; weights are the unchanged GGUF wire bytes, row-major
 *     [n, (k / qk) * block_bytes];
 *   - the activation buffer is [pass1: m*(k/32) Q8_1 blocks of 36 bytes, padded to
 *     256][pass2 when two_pass][inverse: m floats, padded to 256].
 */
#ifndef KAI_HIP_H
#define KAI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Last error message of the calling thread ("" after a successful call).
 * Replaces current_direct_error (current_ggml_direct.cu:174). */
const char *current_direct_error(void);

/* 1 when kai_fused_mmvq can run this shape: supported type, 1 <= m <= 8,
 * k % 32 == 0, k / 32 <= 1024, k % qk == 0, 0 < n <= INT_MAX; else 0.
 * Replaces kai_fused_supported (current_ggml_direct.cu:826-835). */
int kai_fused_supported(int type, int64_t n, int64_t k, int64_t m);

/* Bytes of the activation buffer for m rows of k values.
 * Replaces kai_fused_activation_bytes (current_ggml_direct.cu:837-839). */
size_t kai_fused_activation_bytes(int64_t m, int64_t k, int two_pass);

/* Q8_1 activation preparation of x [m, k] (row stride stride_x elements) into
 * `activation`: exact power-of-two row normalisation, then per-32-value Q8_1.
 * Replaces kai_fused_prepare (current_ggml_direct.cu:841-863; kernel
 * kai_dual_mmvq.cuh:147-254). */
int kai_fused_prepare(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x,
                      void *activation, int two_pass, uintptr_t stream);

/* Single-pass activation of x[..., view] for m <= 8 rows: stored column c reads x column
 * ((c/s)%a)*b*s + (c/(a*s))*s + c%s, i.e. x as [a][b][s] stored as [b][a][s]; s % 32 == 0,
 * a*b*s == k. Same buffer layout and arithmetic as kai_fused_prepare with two_pass = 0.
 * Replaces kai_fused_prepare_view (current_ggml_direct.cu:883-901; kernel
 * kai_prepare_ext.cuh:121-140). */
int kai_fused_prepare_view(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x,
                           void *activation, int64_t a, int64_t b, int64_t s, uintptr_t stream);

/* Single-pass activation of act[c] = rd(rd(silu(g[c])) * u[c]) for m <= 8 rows of a merged
 * [m, 2k] gate_up input (row stride `stride` >= 2k; gate = columns [0, k), up = [k, 2k)), rd
 * rounding to the input dtype, silu(g) = g / (1 + exp(-g)) with exp evaluated by a fixed
 * sequence of IEEE operations (within 2 ulp). Replaces kai_fused_prepare_swiglu
 * (current_ggml_direct.cu:903-919; kernel kai_prepare_ext.cuh:142-183). */
int kai_fused_prepare_swiglu(const void *gate_up, int dtype, int64_t m, int64_t k, int64_t stride,
                             void *activation, uintptr_t stream);

/* Gemma RMSNorm for m <= 8 rows: v = x (+ residual; then v is written to residual_out, fp32
 * [m, k]); y = bf16(v * rstd * weight32) with rstd = 1 / sqrt(sum(v^2) / k + eps) (IEEE divide
 * and square root), written to y (bf16 [m, k]); the activation quantises the stored y. x and
 * residual are F32 (0) or BF16 (1); y and residual_out are 16-byte aligned. Replaces
 * kai_fused_norm_prepare (current_ggml_direct.cu:921-944; kernel kai_prepare_ext.cuh:185-251). */
int kai_fused_norm_prepare(const void *x, int x_dtype, int64_t stride_x, const void *residual,
                           int residual_dtype, int64_t stride_r, float *residual_out,
                           const float *weight32, float eps, void *y, int64_t m, int64_t k,
                           void *activation, uintptr_t stream);

/* Dequantise `rows` contiguous rows of `cols` values (GGUF wire bytes, cols a multiple of
 * the block size) to out [rows, cols] as F32 (0), BF16 (1) or F16 (2), out 16-byte aligned.
 * Each value is the format's formula in fp32 (gguf-py quants.py order, no fused
 * multiply-add), rounded to nearest even. Replaces the torch op ggml_dequantize
 * (csrc/gguf/gguf_kernel.cu:87-102), which has no C entry point in the reference. */
int kai_dequantize(const void *weight, int type, int64_t rows, int64_t cols, void *out, int out_dtype,
                   uintptr_t stream);

/* The legacy _C_gguf ops. The reference binds them as torch ops (schema
 * csrc/torch_bindings.cpp:22-53) with no C entry points; these are their C form.
 *
 * kai_ggml_quantize_q8_1: the legacy Q8_1 activation of x [m, k] (row stride stride_x) in
 * kai_fused_prepare's single-pass layout (kai_fused_activation_bytes(m, k, 0) bytes): per 32
 * values with no row normalisation, d = max|x| / 127, q = max|x| == 0 ? 0 : roundf(x / d),
 * ds = (half(d), half(sum x)) with sum x grouped as a 32-lane xor butterfly (masks 16, 8, 4,
 * 2, 1), inverse[row] = 1. Replaces quantize_row_q8_1_cuda (csrc/gguf/gguf_kernel.cu:32-85),
 * which spaces its rows K padded to 512 with zero blocks that no product reads. */
int kai_ggml_quantize_q8_1(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x, void *activation,
                           uintptr_t stream);

/* Scratch bytes of one kai_ggml_mul_mat_vec_a8 (batched = 0) or kai_ggml_mul_mat_a8
 * (batched = 1) call; 0 with a message when the call would be rejected. */
size_t kai_ggml_a8_workspace(int type, int64_t row, int64_t k, int64_t vecs, int batched);

/* y [vecs, row] (dense; F32, or BF16 when y_bf16) = x [vecs, k] @ W^T over the legacy
 * activation (kai_ggml_quantize_q8_1's arithmetic), W the GGUF wire bytes [row, k / qk *
 * block_bytes]; k <= 32768.
 * kai_ggml_mul_mat_vec_a8 takes the legacy MMVQ block dots (Q4_0's offset from the stored
 * half(sum x); Q4_K and Q2_K mins from d8 * sum q). Replaces ggml_mul_mat_vec_a8
 * (csrc/gguf/gguf_kernel.cu:104-218).
 * kai_ggml_mul_mat_a8 takes the legacy MMQ block dots, which differ only in Q4_K's min term
 * (the stored half(sum x)); every type but IQ3_S (the reference has no such kernel), any row
 * count. Replaces ggml_mul_mat_a8
 * (csrc/gguf/gguf_kernel.cu:220-290). */
int kai_ggml_mul_mat_vec_a8(const void *weight, int type, int64_t row, const void *x, int x_dtype, int64_t vecs,
                            int64_t k, int64_t stride_x, void *y, int y_bf16, void *scratch, size_t scratch_bytes,
                            uintptr_t stream);
int kai_ggml_mul_mat_a8(const void *weight, int type, int64_t row, const void *x, int x_dtype, int64_t vecs,
                        int64_t k, int64_t stride_x, void *y, int y_bf16, void *scratch, size_t scratch_bytes,
                        uintptr_t stream);

/* Copy a GGUF tensor's rows from the model file at `path` into device memory, bytes
 * unchanged: the tensor starts at file_offset and holds src_rows rows of row_bytes. dst row r
 * (r < rows) receives source row row_order[r] (row_order NULL: row r); with block_order,
 * block j (block_bytes each) of every dst row receives the source row's block block_order[j].
 * Reads go through pinned staging buffers and hipMemcpyAsync on `stream`; returns when the
 * copies are complete. Replaces the reference's read-then-permute of stored tensors
 * (gguf-reader/gguf/gguf_reader.py:116-390 memory-mapped reads, then
 * quantization/yaqa_linear.py:102-127 _permute_stored on the host copy), which has no C entry
 * point in the reference. */
int kai_upload_rows(const char *path, int64_t file_offset, int64_t src_rows, int64_t row_bytes,
                    const int64_t *row_order, int64_t rows, int64_t block_bytes,
                    const int64_t *block_order, void *dst, uintptr_t stream);

/* GEMV: dst[j * stride_dst + r] = inverse[j] * sum_b dot(W[r, b], q8[j, b]) for
 * r < n, j < m <= 8; F32 or BF16 (dst_bf16) output. Takes no scratch; on long rows of
 * matrices with few 16-row sets it splits K across workgroups through a library-owned
 * device array of 4 slots rotated per launch, so at most 4 such launches may overlap on
 * one GPU (more race).
 * Replaces kai_fused_mmvq (current_ggml_direct.cu:946-965; kernel kai_dual_mmvq.cuh:258-397). */
int kai_fused_mmvq(const void *weight, int type, int64_t n, int64_t k, int64_t m,
                   const void *activation, int two_pass, void *dst, int dst_bf16,
                   int64_t stride_dst, uintptr_t stream);

/* Scratch bytes kai_fused_mmq_run needs for `count` matrices (types[i], rows[i])
 * sharing k, at m > 8 activation rows: [inverse: m floats][one int8 activation region per
 * layout read by a matrix on the int8 kernels, D4 then DS4 then D2S6][one fp16 image
 * (codes, then min-pass sums) per layout read by a matrix on the fp16 GEMM][the fp32
 * partial sums of a kernel that splits K, or of the K pieces the fp16 GEMM runs its last
 * tiles in (at most 32 MiB)], each region padded to 256 bytes. Up to 16 rows
 * the int8 region is the small-M image (the GGML MMQ quantisation laid out for the small-M
 * GEMM's LDS, 4608 bytes (D4) or 5632 bytes (DS4, D2S6) per 256 values of k) and the
 * partial sums the small-M GEMM's (16 x 16 values per piece of a 16-row set). Above 16 rows
 * a matrix runs on the fp16 GEMM when mmq_uses_h(type, m, rows) holds (every type but
 * Q6_K), reading the fp16 image: codes
 * half(d * q) as [k padded to 256 / 16][m padded to 32][16], and per 256 values of k and row
 * 64 (DS4) or 128 (D2S6) bytes of min-pass sums (none for D4); the others read a plane:
 * 128-value blocks of 144 bytes in [k/128][m] order with k padded to 512. The size is not
 * monotonic in m. direct_f32 is accepted for signature compatibility (outputs are always
 * stored in place). Replaces kai_fused_mmq_workspace (current_ggml_direct.cu:1196-1205). */
size_t kai_fused_mmq_workspace(int device, const int *types, const int64_t *rows, int count,
                               int64_t k, int64_t m, int direct_f32);

/* Batched projection group for m > 8 rows (multi-sequence decode, spec-verify,
 * prefill): one activation preparation (the power-of-two row normalisation, then GGML's
 * MMQ quantisation of each layout the group reads: D4 for Q8_0/Q6_K/IQ3_S, DS4 for
 * Q4_0/Q4_K, D2S6 for Q2_K), then every matrix writes its column slice of dst
 * [m, sum rows] (row stride stride_dst, or sum rows when 0); F32 or BF16. k is a whole
 * number of each type's blocks and a multiple of 4; the sum of rows is a multiple of 4.
 * Replaces kai_fused_mmq_run (current_ggml_direct.cu:1207-1265). */
int kai_fused_mmq_run(const void *const *weights, const int *types, const int64_t *rows, int count,
                      const void *x, int x_dtype, int64_t stride_x, int64_t k, int64_t m,
                      void *dst, int dst_bf16, int64_t stride_dst, void *scratch, size_t scratch_bytes,
                      int device, uintptr_t stream);

/* Largest scratch kai_fused_mmq_run_noalloc can use on one device (16 MiB), and the
 * function that reports it. */
#define KAI_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
size_t kai_fused_mmq_noalloc_capacity(void);

/* kai_fused_mmq_run without the scratch arguments: the same arithmetic and kernels, with
 * the scratch in a device array the library holds per GPU (KAI_NOALLOC_SCRATCH_BYTES, kept
 * until the process ends). It allocates nothing, so callers that cannot allocate (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc) can use it.
 * Returns -1 with a message when kai_fused_mmq_workspace(...) for the call exceeds the
 * capacity. Every call on one GPU uses that GPU's array: calls that overlap on one GPU
 * (two streams, or two host threads) race and must be ordered by the caller. No
 * counterpart in the reference. */
int kai_fused_mmq_run_noalloc(const void *const *weights, const int *types, const int64_t *rows, int count,
                              const void *x, int x_dtype, int64_t stride_x, int64_t k, int64_t m,
                              void *dst, int dst_bf16, int64_t stride_dst, int device, uintptr_t stream);

#ifdef __cplusplus
}
#endif
#endif
