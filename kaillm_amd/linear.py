"""The quantized-linear ``apply()`` surface over packed GGUF wire bytes.

Mirrors, for the fused path, the reference's
  * ``PackedGGUFLinear`` (vllm_gguf_plugin/quantization/compact.py:189-315): one
    original GGUF matrix held as its unchanged wire bytes ``uint8 [N, K/qk*bytes]``
    with ``weight``, ``weight_type``, ``dtype``, ``shape``, ``is_quantized``; unlike
    the reference (compact.py:235-236) it accepts ROCm tensors;
  * ``GGUFLinearMethod.apply`` / ``YAQAMixedLinearMethod.apply``
    (quantization/linear.py:341-363, quantization/yaqa_linear.py:308-367): the
    layer's parts are grouped once into a ``FusedProjection`` and every call runs it,
    adding the bias afterwards.
The reference falls back to per-part Triton kernels when the fused path cannot run
a shape; this build has no fallback and raises instead.
"""
import torch

from . import native_fused
from .formats import FORMATS, WEIGHT_TYPES


class PackedGGUFLinear(torch.nn.Module):
    """One GGUF matrix as contiguous row-major wire bytes on the GPU."""

    def __init__(self, data: torch.Tensor, weight_type: int, dtype: torch.dtype):
        super().__init__()
        self.weight_type = int(weight_type)
        self.dtype = dtype
        if dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError("Compact GGUF requires FP16, BF16, or FP32 activations")
        if data.ndim != 2:
            raise ValueError("Compact GGUF weights must be a two-dimensional tensor")
        if self.weight_type not in WEIGHT_TYPES:
            raise ValueError(f"Unsupported compact GGUF type: {self.weight_type}")
        if data.dtype != torch.uint8:
            raise ValueError("Quantized GGUF data must contain uint8 wire bytes")
        _, _, block_elements, block_bytes = FORMATS[self.weight_type]
        if data.shape[1] == 0 or data.shape[1] % block_bytes:
            raise ValueError("GGUF row width must be a whole number of wire blocks")
        self.is_quantized = True
        self.shape = (data.shape[0], data.shape[1] // block_bytes * block_elements)
        self.register_buffer("weight", data.detach().contiguous())

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        fused = native_fused.prepare([self])
        if not fused or not fused.supports(x):
            raise RuntimeError(f"fused GGUF path cannot run x{tuple(x.shape)} {x.dtype} on {self.shape}")
        return fused(x)


class GGUFLinearMethod:
    """``apply(layer, x, bias)`` for a layer whose ``gguf_compact`` lists its parts."""

    def apply(self, layer: torch.nn.Module, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        fused = getattr(layer, "_kai_fused", None)
        if fused is None:
            fused = native_fused.prepare(list(layer.gguf_compact)) or False
            layer._kai_fused = fused
        if not fused or not fused.supports(x):
            raise RuntimeError(f"fused GGUF path cannot run x{tuple(x.shape)} {x.dtype} for this layer")
        out = fused(x)
        return out if bias is None else out + bias
