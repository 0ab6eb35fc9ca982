"""ctypes binding of libkai_hip.so (include/kai_hip.h, include/kai_quantize.h).

Mirrors the reference's loader (vllm_gguf_plugin/quantization/native_fused.py:52-108):
the same exported names and argument types, ``_check`` raising RuntimeError with
``current_direct_error()``. The library is the in-tree build
(kaillm_amd/libkai_hip.so) unless KAI_HIP_LIBRARY names another file. There is no
fallback: when the library is missing every entry point raises.
"""
import ctypes
import os
from functools import lru_cache
from pathlib import Path

LIBRARY_ENV = "KAI_HIP_LIBRARY"
DEFAULT_PATH = Path(__file__).resolve().parent / "libkai_hip.so"


def library_path() -> Path:
    env = os.getenv(LIBRARY_ENV)
    return Path(env) if env else DEFAULT_PATH


@lru_cache(maxsize=4)
def _load(path: str):
    lib = ctypes.CDLL(path)
    i64, ptr, c_int, u64 = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64
    arr = ctypes.POINTER
    lib.current_direct_error.restype = ctypes.c_char_p
    lib.current_direct_error.argtypes = []
    lib.kai_fused_supported.argtypes = [c_int, i64, i64, i64]
    lib.kai_fused_supported.restype = c_int
    lib.kai_fused_activation_bytes.argtypes = [i64, i64, c_int]
    lib.kai_fused_activation_bytes.restype = ctypes.c_size_t
    lib.kai_fused_prepare.argtypes = [ptr, c_int, i64, i64, i64, ptr, c_int, u64]
    lib.kai_fused_prepare.restype = c_int
    lib.kai_fused_prepare_view.argtypes = [ptr, c_int, i64, i64, i64, ptr, i64, i64, i64, u64]
    lib.kai_fused_prepare_view.restype = c_int
    lib.kai_fused_prepare_swiglu.argtypes = [ptr, c_int, i64, i64, i64, ptr, u64]
    lib.kai_fused_prepare_swiglu.restype = c_int
    lib.kai_fused_norm_prepare.argtypes = [ptr, c_int, i64, ptr, c_int, i64, ptr, ptr, ctypes.c_float, ptr, i64,
                                           i64, ptr, u64]
    lib.kai_fused_norm_prepare.restype = c_int
    lib.kai_fused_mmvq.argtypes = [ptr, c_int, i64, i64, i64, ptr, c_int, ptr, c_int, i64, u64]
    lib.kai_fused_mmvq.restype = c_int
    lib.kai_fused_mmq_workspace.argtypes = [c_int, arr(c_int), arr(i64), c_int, i64, i64, c_int]
    lib.kai_fused_mmq_workspace.restype = ctypes.c_size_t
    lib.kai_fused_mmq_run.argtypes = [arr(ptr), arr(c_int), arr(i64), c_int, ptr, c_int, i64, i64, i64, ptr,
                                      c_int, i64, ptr, ctypes.c_size_t, c_int, u64]
    lib.kai_fused_mmq_run.restype = c_int
    lib.kai_fused_mmq_noalloc_capacity.argtypes = []
    lib.kai_fused_mmq_noalloc_capacity.restype = ctypes.c_size_t
    lib.kai_fused_mmq_run_noalloc.argtypes = [arr(ptr), arr(c_int), arr(i64), c_int, ptr, c_int, i64, i64, i64, ptr,
                                              c_int, i64, c_int, u64]
    lib.kai_fused_mmq_run_noalloc.restype = c_int
    lib.kai_upload_rows.argtypes = [ctypes.c_char_p, i64, i64, i64, ptr, i64, i64, ptr, ptr, u64]
    lib.kai_upload_rows.restype = c_int
    lib.kai_dequantize.argtypes = [ptr, c_int, i64, i64, ptr, c_int, u64]
    lib.kai_dequantize.restype = c_int
    lib.kai_ggml_quantize_q8_1.argtypes = [ptr, c_int, i64, i64, i64, ptr, u64]
    lib.kai_ggml_quantize_q8_1.restype = c_int
    lib.kai_ggml_a8_workspace.argtypes = [c_int, i64, i64, i64, c_int]
    lib.kai_ggml_a8_workspace.restype = ctypes.c_size_t
    for name in ("kai_ggml_mul_mat_vec_a8", "kai_ggml_mul_mat_a8"):
        getattr(lib, name).argtypes = [ptr, c_int, i64, ptr, c_int, i64, i64, i64, ptr, c_int, ptr, ctypes.c_size_t,
                                       u64]
        getattr(lib, name).restype = c_int
    lib.kai_quantize_rows.argtypes = [c_int, ptr, i64, i64, ptr, c_int]
    lib.kai_quantize_rows.restype = c_int
    # measurement entry points (include/kai_peaks.h)
    lib.kai_peak_mfma.argtypes = [c_int, i64, c_int, c_int, ptr, u64]
    lib.kai_peak_mfma.restype = c_int
    lib.kai_peak_mfma_ops.argtypes = [c_int]
    lib.kai_peak_mfma_ops.restype = i64
    lib.kai_peak_lds.argtypes = [i64, c_int, c_int, ptr, u64]
    lib.kai_peak_lds.restype = c_int
    lib.kai_peak_copy.argtypes = [ptr, ptr, i64, c_int, u64]
    lib.kai_peak_copy.restype = c_int
    return lib


def library():
    """The loaded libkai_hip.so; raises when it has not been built."""
    path = library_path()
    if not path.is_file():
        raise RuntimeError(
            f"{path} is missing: build it with kaillm_amd._build.build() (or __graft_entry__.build())"
        )
    return _load(str(path))


def check(lib, status):
    """Raise RuntimeError(current_direct_error()) for a nonzero status (native_fused.py:106-108)."""
    if status:
        raise RuntimeError(lib.current_direct_error().decode())
