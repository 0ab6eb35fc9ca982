"""The legacy GGUF op surface on the gfx950 kernels.

Mirrors the reference's ``vllm_gguf_plugin/ops.py:181-208`` (``ggml_dequantize``,
``ggml_mul_mat_vec_a8``, ``ggml_mul_mat_a8``: the ``_C_gguf`` ops of
``csrc/gguf/gguf_kernel.cu:32-290``, schema ``csrc/torch_bindings.cpp:22-53``) and the
dispatch of its non-compact layers, ``_fused_mul_mat_gguf`` (``quantization/linear.py:40-63``),
as torch custom ops with fake implementations:

  * ``ggml_dequantize(W, type, m, n, dtype)`` -> ``[m, n]`` in ``dtype`` (F16 by default),
    the HIP dequantisation kernel (``kai_dequantize``);
  * ``ggml_mul_mat_vec_a8`` / ``ggml_mul_mat_a8(W, X, type, row)`` -> ``X @ dequant(W).T`` as
    ``[X rows, row]`` in X's dtype, with the legacy arithmetic (``kai_ggml_mul_mat_vec_a8`` /
    ``kai_ggml_mul_mat_a8``): X quantised per 32 values with no row normalisation and the
    block sum stored as ``half(sum x)`` (``quantize_q8_1``, gguf_kernel.cu:32-69), then the
    legacy MMVQ block dots, or for ``ggml_mul_mat_a8`` the legacy MMQ ones (Q4_K's min term
    from the stored sum);
  * ``fused_mul_mat_gguf(x, qweight, type)`` with the reference's row thresholds and type sets.

``ggml_mul_mat_a8`` on IQ3_S has no ``_C_gguf`` kernel; the reference's Python op then runs its
Triton GEMM of x with the dequantised weight (ops.py:200-208, triton/gemm/iq_quant/iq3_s.py),
here ``X @ ggml_dequantize(W, X.dtype).T``. K above 32768 takes the dequantising route too.
"""
import torch

from . import native
from .formats import FORMATS, WEIGHT_TYPES

F32, F16, BF16 = 0, 1, 30
UNQUANTIZED_TYPES = (F32, F16, BF16)
IMATRIX_QUANT_TYPES = (21,)
MMVQ_QUANT_TYPES = WEIGHT_TYPES
MMQ_QUANT_TYPES = tuple(t for t in WEIGHT_TYPES if t not in IMATRIX_QUANT_TYPES)  # quantization/utils.py:74-75
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


def _legacy_workspace(quant_type, row, k, m, batched):
    return native.library().kai_ggml_a8_workspace(quant_type, row, k, m, int(batched))


def _mul_mat(W, X, quant_type, row, batched):
    if X.dim() != 2:
        raise ValueError("X must be [rows, K]")
    m, k = X.shape
    if m == 0:
        return X.new_empty((0, row))
    if X.dtype not in _OUT_CODES:
        raise TypeError(f"Unsupported activation dtype {X.dtype}")
    if quant_type not in WEIGHT_TYPES:
        raise NotImplementedError(f"Unsupported GGUF quantization type: {quant_type}")
    W = W.contiguous()
    _, _, qk, bb = FORMATS[quant_type]
    if W.shape[0] != row or k % qk or W.numel() != row * (k // qk) * bb:
        raise ValueError("W must be [row, K / block * block_bytes] wire bytes")
    lib = native.library()
    need = _legacy_workspace(quant_type, row, k, m, batched)
    if need == 0 and ((batched and quant_type not in MMQ_QUANT_TYPES) or k > 32768):
        return X @ _dequantize(W, quant_type, row, k, X.dtype).T
    if need == 0:
        raise RuntimeError(lib.current_direct_error().decode() or "GGUF legacy product failed")
    X = X.contiguous()
    out_bf16 = X.dtype == torch.bfloat16
    y = torch.empty((m, row), dtype=torch.bfloat16 if out_bf16 else torch.float32, device=X.device)
    scratch = torch.empty(need, dtype=torch.uint8, device=X.device)
    fn = lib.kai_ggml_mul_mat_a8 if batched else lib.kai_ggml_mul_mat_vec_a8
    native.check(lib, fn(W.data_ptr(), quant_type, row, X.data_ptr(), _OUT_CODES[X.dtype], m, k, k, y.data_ptr(),
                         int(out_bf16), scratch.data_ptr(), need, torch.cuda.current_stream(X.device).cuda_stream))
    return y if y.dtype == X.dtype else y.to(X.dtype)


@torch.library.custom_op("kaillm::ggml_mul_mat_vec_a8", mutates_args=())
def ggml_mul_mat_vec_a8(W: torch.Tensor, X: torch.Tensor, quant_type: int, row: int) -> torch.Tensor:
    return _mul_mat(W, X, quant_type, row, False)


@ggml_mul_mat_vec_a8.register_fake
def _fake_vec(W, X, quant_type, row):
    return X.new_empty((X.shape[0], row))


@torch.library.custom_op("kaillm::ggml_mul_mat_a8", mutates_args=())
def ggml_mul_mat_a8(W: torch.Tensor, X: torch.Tensor, quant_type: int, row: int) -> torch.Tensor:
    return _mul_mat(W, X, quant_type, row, True)


@ggml_mul_mat_a8.register_fake
def _fake_a8(W, X, quant_type, row):
    return X.new_empty((X.shape[0], row))


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
    if x.shape[0] <= mmvq_safe and qweight_type in MMVQ_QUANT_TYPES:
        return _mul_mat(qweight, x, qweight_type, qweight.shape[0], False)
    if qweight_type in MMQ_QUANT_TYPES:
        return _mul_mat(qweight, x, qweight_type, qweight.shape[0], True)
    if qweight_type in DEQUANT_TYPES:
        _, _, qk, bb = FORMATS[qweight_type]
        weight = _dequantize(qweight, qweight_type, qweight.shape[0], qweight.shape[1] // bb * qk, x.dtype)
        return x @ weight.T
    raise NotImplementedError(f"Unsupported GGUF quantization type: {qweight_type}")


@fused_mul_mat_gguf.register_fake
def _fake_fused(x, qweight, qweight_type):
    return torch.empty(x.shape[0], qweight.shape[0], dtype=x.dtype, device=x.device)
