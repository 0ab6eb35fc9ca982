"""The quantized-linear ``apply()`` surface over packed GGUF wire bytes.

Mirrors, for the fused path, the reference's
  * ``PackedGGUFLinear`` (vllm_gguf_plugin/quantization/compact.py:189-315): one
    original GGUF matrix held as its unchanged wire bytes ``uint8 [N, K/qk*bytes]``
    with ``weight``, ``weight_type``, ``dtype``, ``shape``, ``is_quantized``; unlike
    the reference (compact.py:235-236) it accepts ROCm tensors;
  * ``GGUFLinearMethod.apply`` / ``YAQAMixedLinearMethod.apply``
    (quantization/linear.py:341-363, quantization/yaqa_linear.py:308-367): the
    layer's parts are grouped once into a ``FusedProjection`` and every call runs it,
    adding the bias afterwards; ``apply_swiglu`` (yaqa_linear.py:341-347) and the
    input-view path (yaqa_linear.py:348-361) use the fused activation producers.
The reference falls back to per-part Triton kernels when the fused path cannot run
a shape; this build has no fallback and raises instead.
"""
import os

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
    """``apply(layer, x, bias)`` for a layer whose ``gguf_compact`` lists its parts.

    Optional layer attributes, as the reference's loader sets them
    (yaqa_linear.py:265-266, weights_adapter/qwen35.py:181):
      ``_kai_input_gather`` column index applied to x before the projection, and
      ``_kai_input_view`` (a, b, s) when that index is the segment transpose
      [a][b][s] -> [b][a][s]; up to 8 rows then read x through the view with no copy;
      ``_kai_act_producer`` the id of a norm whose output this layer consumes
      (``native_fused.norm_prepare``), registered once in ``native_fused.CONSUMER_OF``.
    """

    def _fused(self, layer):
        fused = getattr(layer, "_kai_fused", None)
        if fused is None:
            fused = native_fused.prepare(list(layer.gguf_compact)) or False
            layer._kai_fused = fused
            producer = layer.__dict__.get("_kai_act_producer")
            if fused and producer is not None:
                native_fused.CONSUMER_OF[fused.weights[0].data_ptr()] = producer
        return fused

    def _ext_rows(self, layer, x, width):
        """The projection when x (width columns) has 1..8 rows the producers can take."""
        fused = self._fused(layer)
        rows = x.numel() // x.shape[-1] if x.shape[-1] else 0
        if not fused or not x.is_cuda or x.shape[-1] != width(fused) or rows not in fused._supported:
            return None
        if x.dtype not in (torch.bfloat16, torch.float16, torch.float32) or not native_fused.ext_available():
            return None
        return fused

    def apply_swiglu(self, layer: torch.nn.Module, gate_up: torch.Tensor, act_fn) -> torch.Tensor:
        """down_proj(silu(gate) * up): up to 8 rows prepare the activation straight from
        gate_up (yaqa_linear.py:341-347); other shapes apply act_fn first."""
        if getattr(layer, "_kai_input_gather", None) is None and os.getenv("KAILLM_FUSED_SWIGLU", "1") == "1":
            fused = self._ext_rows(layer, gate_up, lambda f: 2 * f.k)
            if fused is not None:
                return fused.call_swiglu(gate_up)
        return self.apply(layer, act_fn(gate_up))

    def apply(self, layer: torch.nn.Module, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        gather = getattr(layer, "_kai_input_gather", None)
        view = getattr(layer, "_kai_input_view", None)
        if gather is not None and view is not None and bias is None:
            fused = self._ext_rows(layer, x, lambda f: f.k)
            if fused is not None:
                return fused.call_view(x, view)
        if gather is not None:
            if view is not None:
                x = x.unflatten(-1, tuple(view)).transpose(-3, -2).flatten(-3)
            else:
                x = x.index_select(-1, gather)
        fused = self._fused(layer)
        if not fused or not fused.supports(x):
            raise RuntimeError(f"fused GGUF path cannot run x{tuple(x.shape)} {x.dtype} for this layer")
        out = fused(x)
        return out if bias is None else out + bias
