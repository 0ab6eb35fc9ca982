/*
 * Host-side GGUF weight quantizers (tooling in libkai_hip.so, no GPU involved).
 *
 * No counterpart in the reference's native library: the reference quantizes on
 * the host with gguf-py (runtime-source/gguf-reader/gguf/quants.py), which this
 * replaces for building synthetic weights in tests and benchmarks. Not on the
 * hot path.
 */
#ifndef KAI_QUANTIZE_H
#define KAI_QUANTIZE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Quantize n rows of k floats (host memory, row-major) into GGUF wire blocks of
 * `type` (Q4_0 = 2, Q8_0 = 8, Q2_K = 10, Q4_K = 12, Q6_K = 14, IQ3_S = 21) at dst
 * (host memory, n * (k / qk) * block_bytes). threads <= 1 runs on the caller's
 * thread. Returns 0, or -1 for an unsupported type, k % qk != 0 or null pointers. */
int kai_quantize_rows(int type, const float *src, int64_t n, int64_t k, void *dst, int threads);

#ifdef __cplusplus
}
#endif
#endif
