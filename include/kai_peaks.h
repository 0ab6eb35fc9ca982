/*
 * kai_peaks: measurement entry points of libkai_hip (no counterpart in the reference).
 *
 * They run fixed kernels that bench.py --peaks times with HIP events to measure this
 * device's ceilings: the dense MFMA rate per instruction kind, the LDS read rate and a
 * STREAM-style HBM copy. Same conventions as kai_hip.h: device pointers, stream as
 * uintptr_t, 0 on success, -1 with current_direct_error() on error.
 */
#ifndef KAI_PEAKS_H
#define KAI_PEAKS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* MFMA instruction kinds */
#define KAI_PEAK_F16_32X32X16 0 /* v_mfma_f32_32x32x16_f16 */
#define KAI_PEAK_F16_16X16X32 1 /* v_mfma_f32_16x16x32_f16 */
#define KAI_PEAK_F16_32X32X8 2  /* v_mfma_f32_32x32x8_f16 */
#define KAI_PEAK_I8_32X32X32 3  /* v_mfma_i32_32x32x32_i8 */
#define KAI_PEAK_I8_16X16X64 4  /* v_mfma_i32_16x16x64_i8 */

/* blocks x threads lanes each issue iters x 4 independent MFMAs of `kind` (out: a guard
 * buffer of `threads` floats, written only on an impossible sum). */
int kai_peak_mfma(int kind, int64_t iters, int blocks, int threads, float *out, uintptr_t stream);
/* Operations (2 x multiply-adds) of one MFMA of `kind`; 0 for an unknown kind. */
int64_t kai_peak_mfma_ops(int kind);
/* blocks x threads lanes each read iters x 4 x 16 bytes of LDS. */
int kai_peak_lds(int64_t iters, int blocks, int threads, float *out, uintptr_t stream);
/* dst = src over `bytes` (a multiple of 16) with `blocks` workgroups of 256 lanes. */
int kai_peak_copy(const void *src, void *dst, int64_t bytes, int blocks, uintptr_t stream);

#ifdef __cplusplus
}
#endif

#endif
