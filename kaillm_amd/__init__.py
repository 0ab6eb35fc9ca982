"""kaillm_amd: MI355X-native GGUF dequant-fused quantized linear.

The hot path of the reference's vllm_gguf_plugin (fused Q8_1 activation
preparation + GEMV / batched GEMM over unchanged GGUF wire blocks), rebuilt as
hand-written gfx950 HIP kernels behind the reference's C ABI (include/kai_hip.h)
and its Python/torch operator surface (native_fused, linear).
"""
from . import formats, native  # noqa: F401

__all__ = ["formats", "native"]
