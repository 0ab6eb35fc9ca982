"""GGUF block formats carried by the fused linear, and host-side quantization.

Type ids are GGML's (vllm_gguf_plugin/triton/gemm/utils.py:5-24); geometry
(bits, group, block elements, block bytes) follows
vllm_gguf_plugin/quantization/gguf_repack.py:18-34 for the formats this path runs.
"""
import ctypes

import numpy as np

from .native import check, library

Q4_0, Q8_0, Q8_1, Q2_K, Q4_K, Q6_K, IQ3_S = 2, 8, 9, 10, 12, 14, 21

# type -> (bits, values per scale group, values per block, bytes per block)
FORMATS = {
    Q4_0: (4, 32, 32, 18),
    Q8_0: (8, 32, 32, 34),
    Q8_1: (8, 32, 32, 36),
    Q2_K: (2, 16, 256, 84),
    Q4_K: (4, 32, 256, 144),
    Q6_K: (6, 16, 256, 210),
    IQ3_S: (3, 32, 256, 110),
}
NAMES = {Q4_0: "Q4_0", Q8_0: "Q8_0", Q8_1: "Q8_1", Q2_K: "Q2_K", Q4_K: "Q4_K", Q6_K: "Q6_K", IQ3_S: "IQ3_S"}
WEIGHT_TYPES = (Q4_0, Q8_0, Q2_K, Q4_K, Q6_K, IQ3_S)


def block_elems(qtype: int) -> int:
    return FORMATS[qtype][2]


def block_bytes(qtype: int) -> int:
    return FORMATS[qtype][3]


def row_bytes(qtype: int, k: int) -> int:
    qk, bb = FORMATS[qtype][2:]
    if k % qk:
        raise ValueError(f"k={k} is not a multiple of the {NAMES[qtype]} block ({qk})")
    return k // qk * bb


def weight_bytes(qtype: int, n: int, k: int) -> int:
    return n * row_bytes(qtype, k)


def quantize(weights: np.ndarray, qtype: int, threads: int = 0) -> np.ndarray:
    """Quantize float rows [n, k] into wire bytes uint8 [n, (k/qk)*block_bytes]."""
    if qtype not in WEIGHT_TYPES:
        raise ValueError(f"unsupported weight type {qtype}")
    w = np.ascontiguousarray(weights, dtype=np.float32)
    if w.ndim != 2:
        raise ValueError("weights must be two-dimensional")
    n, k = w.shape
    out = np.empty((n, row_bytes(qtype, k)), dtype=np.uint8)
    lib = library()
    threads = threads or min(16, __import__("os").cpu_count() or 1)
    status = lib.kai_quantize_rows(qtype, w.ctypes.data_as(ctypes.c_void_p), n, k,
                                   out.ctypes.data_as(ctypes.c_void_p), threads)
    if status:
        raise ValueError(f"kai_quantize_rows failed for type {qtype}, shape {w.shape}")
    return out
