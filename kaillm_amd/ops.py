"""The legacy GGUF op surface on the gfx950 kernels.

Mirrors the reference's ``vllm_gguf_plugin/ops.py:180-215`` (``ggml_dequantize``,
``ggml_mul_mat_vec_a8``, ``ggml_mul_mat_a8`` over ``csrc/gguf/gguf_kernel.cu:87-290``) and
the dispatch of its non-compact layers, ``_fused_mul_mat_gguf``
(``quantization/linear.py:40-63``), as torch custom ops with fake implementations:

  * ``ggml_dequantize(W, type, m, n, dtype)`` -> ``[m, n]`` in ``dtype`` (F16 by default),
    the HIP dequantisation kernel (``kai_dequantize``);
  * ``ggml_mul_mat_vec_a8`` / ``ggml_mul_mat_a8(W, X, type, row)`` -> ``X @ dequant(W).T`` as
    ``[X rows, row]`` in X's dtype, through the fused projection kernels (GEMV up to 8 rows,
    the batched kernels beyond);
  * ``fused_mul_mat_gguf(x, qweight, type)`` with the reference's row thresholds.

The activation is quantised by the fused path's single-pass preparation. Its block codes
are those of the legacy per-block Q8_1 (the power-of-two row scale cancels in q = x / d);
the stored block sum is ``half(d * sum(q))`` where the legacy kernel stores ``half(sum(x))``,
so the min terms of Q4_K/Q2_K differ within the activation's quantisation error. Unlike
the reference's legacy MMQ, the batched kernels take IQ3_S too.
"""
import torch

from . import native, native_fused
from .formats import FORMATS, WEIGHT_TYPES

F32, F16, BF16 = 0, 1, 30
UNQUANTIZED_TYPES = (F32, F16, BF16)
IMATRIX_QUANT_TYPES = (21,)
MMVQ_QUANT_TYPES = WEIGHT_TYPES
MMQ_QUANT_TYPES = WEIGHT_TYPES
DEQUANT_TYPES = WEIGHT_TYPES
_OUT_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def _dequantize(W, quant_type, m, n, dtype):
    dtype = torch.float16 if dtype is None else dtype
    if dtype not in _OUT_CODES:
        raise TypeError(f"ggml_dequantize cannot produce {dtype}")
    if quant_type not in WEIGHT_TYPES:
        raise NotImplementedError(f"Unsupported GGUF quantization type: {quant_type}")
    W = W.contiguous()
    _, _, qk, bb = FORMATS[quant_type]
    if n % qk or W.numel() < m * (n // qk) * bb:
        raise ValueError("ggml_dequantize: W holds fewer blocks than m x n values")
    out = torch.empty((m, n), dtype=dtype, device=W.device)
    lib = native.library()
    native.check(lib, lib.kai_dequantize(W.data_ptr(), quant_type, m, n, out.data_ptr(), _OUT_CODES[dtype],
                                         torch.cuda.current_stream(W.device).cuda_stream))
    return out


@torch.library.custom_op("kaillm::ggml_dequantize", mutates_args=())
def ggml_dequantize(W: torch.Tensor, quant_type: int, m: int, n: int, dtype: torch.dtype | None) -> torch.Tensor:
    return _dequantize(W, quant_type, m, n, dtype)


@ggml_dequantize.register_fake
def _fake_dequantize(W, quant_type, m, n, dtype):
    return W.new_empty((m, n), dtype=torch.float16 if dtype is None else dtype)


def _mul_mat(W, X, quant_type, row):
    if X.dim() != 2:
        raise ValueError("X must be [rows, K]")
    m, k = X.shape
    if m == 0:
        return X.new_empty((0, row))
    if X.dtype not in _OUT_CODES:
        raise TypeError(f"Unsupported activation dtype {X.dtype}")
    W = W.contiguous()
    _, _, qk, bb = FORMATS[quant_type]
    if W.shape[0] != row or W.numel() != row * (k // qk) * bb or k % qk:
        raise ValueError("W must be [row, K / block * block_bytes] wire bytes")
    X = X.contiguous()
    out_f32 = X.dtype != torch.bfloat16
    if m <= native_fused.MAX_ROWS:
        y = native_fused.fused_mmvq(X, [W], [quant_type], [row], 0, out_f32)
    else:
        y = native_fused.fused_mmq(X, [W], [quant_type], [row], out_f32)
    return y if y.dtype == X.dtype else y.to(X.dtype)


@torch.library.custom_op("kaillm::ggml_mul_mat_vec_a8", mutates_args=())
def ggml_mul_mat_vec_a8(W: torch.Tensor, X: torch.Tensor, quant_type: int, row: int) -> torch.Tensor:
    return _mul_mat(W, X, quant_type, row)


@ggml_mul_mat_vec_a8.register_fake
def _fake_vec(W, X, quant_type, row):
    return X.new_empty((X.shape[0], row))


@torch.library.custom_op("kaillm::ggml_mul_mat_a8", mutates_args=())
def ggml_mul_mat_a8(W: torch.Tensor, X: torch.Tensor, quant_type: int, row: int) -> torch.Tensor:
    return _mul_mat(W, X, quant_type, row)


@ggml_mul_mat_a8.register_fake
def _fake_a8(W, X, quant_type, row):
    return X.new_empty((X.shape[0], row))


def _fused_supported(qweight, x, quant_type):
    """The fused kernels take this shape (K within the preparation's 32768 limit)."""
    lib = native.library()
    return bool(lib.kai_fused_supported(quant_type, qweight.shape[0], x.shape[1], 1))


@torch.library.custom_op("kaillm::fused_mul_mat_gguf", mutates_args=())
def fused_mul_mat_gguf(x: torch.Tensor, qweight: torch.Tensor, qweight_type: int) -> torch.Tensor:
    """x @ W.T for one GGUF matrix, dispatched as quantization/linear.py:40-63 does."""
    if qweight_type in IMATRIX_QUANT_TYPES:
        mmvq_safe = 8 if qweight.shape[0] > 5120 else 16
    else:
        mmvq_safe = 2 if qweight.shape[0] > 5120 else 6
    if x.shape[0] == 0:
        return torch.empty(x.shape[0], qweight.shape[0], dtype=x.dtype, device=x.device)
    if qweight_type in UNQUANTIZED_TYPES:
        return x @ qweight.T
    if qweight_type not in WEIGHT_TYPES:
        raise NotImplementedError(f"Unsupported GGUF quantization type: {qweight_type}")
    if _fused_supported(qweight, x, qweight_type):
        if x.shape[0] <= mmvq_safe and qweight_type in MMVQ_QUANT_TYPES:
            return _mul_mat(qweight, x, qweight_type, qweight.shape[0])
        if qweight_type in MMQ_QUANT_TYPES:
            return _mul_mat(qweight, x, qweight_type, qweight.shape[0])
    _, _, qk, bb = FORMATS[qweight_type]
    weight = _dequantize(qweight, qweight_type, qweight.shape[0], qweight.shape[1] // bb * qk, x.dtype)
    return x @ weight.T


@fused_mul_mat_gguf.register_fake
def _fake_fused(x, qweight, qweight_type):
    return torch.empty(x.shape[0], qweight.shape[0], dtype=x.dtype, device=x.device)
