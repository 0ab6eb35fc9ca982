"""Fused GGUF projections on MI355X: torch custom ops over libkai_hip.so.

Host-side mirror of the reference's bridge
(vllm_gguf_plugin/quantization/native_fused.py): the same module-level names
(``ENV``, ``MAX_ROWS``, ``TYPES``, ``mode()``, ``mmq_mode()``, ``library()``,
``FusedProjection``, ``prepare(parts)``), the same torch custom op schemas
(``kaillm::fused_mmvq``, ``kaillm::fused_mmq``) with fake implementations, and the
same call sequence: one Q8_1 activation preparation per projection group, then
one GEMV launch per matrix writing its column slice of the merged output.

The fused producers (native_fused.py:105-200 of the reference) are here too:
``kaillm::fused_mmvq_view`` and ``kaillm::fused_mmvq_swiglu`` prepare the activation
from a column-permuted input or from a merged gate_up output, and ``norm_prepare``
runs a Gemma RMSNorm that stashes its output's activation for registered consumer
projections (``CONSUMER_OF``, ``STASH``).

Rows 1..8 run ``kai_fused_mmvq`` (native_fused.py:337-347 of the reference); more
rows run ``kai_fused_mmq_run``. Every launch goes to the gfx950 kernels; there is
no CPU or PyTorch fallback, and a missing library raises.

KAILLM_FUSED_MMVQ: "0" disabled, "1" single pass (default), "2" two passes.
KAILLM_FUSED_MMQ: "0" disables the >8-row path, "1" (default) enables it.
"""
import ctypes
import os

import torch

from . import native
from .formats import WEIGHT_TYPES

ENV = "KAILLM_FUSED_MMVQ"
MAX_ROWS = 8
TYPES = WEIGHT_TYPES
MMQ_TYPES = WEIGHT_TYPES
_DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def mode():
    value = os.getenv(ENV, "1")
    if value not in ("0", "1", "2"):
        raise ValueError(ENV + " must be 0, 1 or 2")
    return int(value)


def mmq_mode():
    value = os.getenv("KAILLM_FUSED_MMQ", "1")
    if value not in ("0", "1"):
        raise ValueError("KAILLM_FUSED_MMQ must be 0 or 1")
    return value == "1"


def library():
    """The gfx950 fused library (raises when it is not built)."""
    return native.library()


def _check(lib, status):
    native.check(lib, status)


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _out(m, total, out_f32, device):
    return torch.empty((m, total), dtype=torch.float32 if out_f32 else torch.bfloat16, device=device)


def _mmvq_into(lib, activation, weights, types, rows_out, m, k, two_pass, out_f32, device):
    """One GEMV launch per matrix, each writing its column slice of the merged output."""
    total = sum(rows_out)
    out = _out(m, total, out_f32, device)
    stream = _stream(device)
    offset = 0
    element = out.element_size()
    for weight, qtype, n in zip(weights, types, rows_out):
        _check(lib, lib.kai_fused_mmvq(weight.data_ptr(), qtype, n, k, m, activation.data_ptr(), two_pass,
                                       out.data_ptr() + offset * element, 0 if out_f32 else 1, total, stream))
        offset += n
    return out


def _new_activation(lib, m, k, two_pass, device):
    return torch.empty(lib.kai_fused_activation_bytes(m, k, two_pass), dtype=torch.uint8, device=device)


# Activation producers (native_fused.py:107-110 of the reference): a norm that feeds
# registered consumer projections stores the activation of its output under its producer
# id; a consumer (keyed by its first weight pointer) whose input is that output uses it
# instead of preparing its own.
CONSUMER_OF = {}
STASH = {}


def ext_available():
    """The producer entry points are there and the single-pass activation is in use."""
    lib = library()
    return hasattr(lib, "kai_fused_norm_prepare") and mode() == 1


def _key(x):
    return (x.data_ptr(), x.shape[0], x.shape[1], x.stride(0), x.dtype, x.device)


def norm_prepare(producer, x, residual, weight32, eps):
    """Gemma RMSNorm of <= 8 rows that also prepares its output's activation.

    Returns (y bf16, fp32 residual stream or None), or None when the inputs are not
    eligible (the caller then runs its own norm). y's activation is stashed for the
    consumers of ``producer``; the stash holds y itself, so its storage cannot be
    reused by another tensor that would match the key.
    """
    if not ext_available() or x.dim() != 2 or not 0 < x.shape[0] <= MAX_ROWS or not x.is_cuda:
        return None
    if x.dtype not in (torch.bfloat16, torch.float32) or x.stride(-1) != 1 or x.shape[1] % 32:
        return None
    if residual is not None and (residual.dtype not in (torch.bfloat16, torch.float32)
                                 or residual.shape != x.shape or residual.stride(-1) != 1):
        return None
    lib = library()
    m, k = x.shape
    y = torch.empty((m, k), dtype=torch.bfloat16, device=x.device)
    r_out = None if residual is None else torch.empty((m, k), dtype=torch.float32, device=x.device)
    activation = _new_activation(lib, m, k, 0, x.device)
    _check(lib, lib.kai_fused_norm_prepare(
        x.data_ptr(), _DTYPE_CODES[x.dtype], x.stride(0),
        None if residual is None else residual.data_ptr(), 0 if residual is None else _DTYPE_CODES[residual.dtype],
        0 if residual is None else residual.stride(0), None if r_out is None else r_out.data_ptr(),
        weight32.data_ptr(), float(eps), y.data_ptr(), m, k, activation.data_ptr(), _stream(x.device)))
    STASH[producer] = (_key(y), activation, y)
    return y, r_out


def _run(x, weights, types, rows_out, two_pass, out_f32):
    lib = library()
    m, k = x.shape
    if two_pass == 0 and CONSUMER_OF:
        producer = CONSUMER_OF.get(weights[0].data_ptr())
        entry = STASH.get(producer) if producer is not None else None
        if entry is not None and entry[0] == _key(x):
            return _mmvq_into(lib, entry[1], weights, types, rows_out, m, k, 0, out_f32, x.device)
    activation = _new_activation(lib, m, k, two_pass, x.device)
    _check(lib, lib.kai_fused_prepare(x.data_ptr(), _DTYPE_CODES[x.dtype], m, k, x.stride(0),
                                      activation.data_ptr(), two_pass, _stream(x.device)))
    return _mmvq_into(lib, activation, weights, types, rows_out, m, k, two_pass, out_f32, x.device)


@torch.library.custom_op("kaillm::fused_mmvq_view", mutates_args=())
def fused_mmvq_view(x: torch.Tensor, weights: list[torch.Tensor], types: list[int], rows_out: list[int],
                    a: int, b: int, s: int, out_f32: bool) -> torch.Tensor:
    """GEMV on x[..., view]: x's columns as [a][b][s] read as [b][a][s], with no copy."""
    lib = library()
    m, k = x.shape
    activation = _new_activation(lib, m, k, 0, x.device)
    _check(lib, lib.kai_fused_prepare_view(x.data_ptr(), _DTYPE_CODES[x.dtype], m, k, x.stride(0),
                                           activation.data_ptr(), a, b, s, _stream(x.device)))
    return _mmvq_into(lib, activation, weights, types, rows_out, m, k, 0, out_f32, x.device)


@fused_mmvq_view.register_fake
def _fake_view(x, weights, types, rows_out, a, b, s, out_f32):
    return x.new_empty((x.shape[0], sum(rows_out)), dtype=torch.float32 if out_f32 else torch.bfloat16)


@torch.library.custom_op("kaillm::fused_mmvq_swiglu", mutates_args=())
def fused_mmvq_swiglu(gate_up: torch.Tensor, weights: list[torch.Tensor], types: list[int], rows_out: list[int],
                      out_f32: bool) -> torch.Tensor:
    """GEMV on silu(gate) * up read straight from a merged [m, 2k] gate_up output."""
    lib = library()
    m, k = gate_up.shape[0], gate_up.shape[1] // 2
    activation = _new_activation(lib, m, k, 0, gate_up.device)
    _check(lib, lib.kai_fused_prepare_swiglu(gate_up.data_ptr(), _DTYPE_CODES[gate_up.dtype], m, k,
                                             gate_up.stride(0), activation.data_ptr(), _stream(gate_up.device)))
    return _mmvq_into(lib, activation, weights, types, rows_out, m, k, 0, out_f32, gate_up.device)


@fused_mmvq_swiglu.register_fake
def _fake_swiglu(gate_up, weights, types, rows_out, out_f32):
    return gate_up.new_empty((gate_up.shape[0], sum(rows_out)), dtype=torch.float32 if out_f32 else torch.bfloat16)


_MMQ_GROUPS = {}


def _mmq_group(weights, types, rows_out):
    key = (tuple(w.data_ptr() for w in weights), tuple(types), tuple(rows_out))
    group = _MMQ_GROUPS.get(key)
    if group is None:
        count = len(weights)
        group = ((ctypes.c_void_p * count)(*[w.data_ptr() for w in weights]),
                 (ctypes.c_int * count)(*types), (ctypes.c_int64 * count)(*rows_out))
        _MMQ_GROUPS[key] = group
    return group


def _mmq_run(x, weights, types, rows_out, out_f32):
    lib = library()
    m, k = x.shape
    ptrs, ctypes_types, ctypes_rows = _mmq_group(weights, types, rows_out)
    device = x.device.index if x.device.index is not None else torch.cuda.current_device()
    size = lib.kai_fused_mmq_workspace(device, ctypes_types, ctypes_rows, len(weights), k, m, int(out_f32))
    if not size:
        raise RuntimeError(lib.current_direct_error().decode())
    total = sum(rows_out)
    out = _out(m, total, out_f32, x.device)
    scratch = torch.empty(size, dtype=torch.uint8, device=x.device)
    _check(lib, lib.kai_fused_mmq_run(ptrs, ctypes_types, ctypes_rows, len(weights), x.data_ptr(),
                                      _DTYPE_CODES[x.dtype], x.stride(0), k, m, out.data_ptr(),
                                      0 if out_f32 else 1, 0 if out_f32 else total, scratch.data_ptr(), size,
                                      device, _stream(x.device)))
    return out


@torch.library.custom_op("kaillm::fused_mmq", mutates_args=())
def fused_mmq(x: torch.Tensor, weights: list[torch.Tensor], types: list[int], rows_out: list[int],
              out_f32: bool) -> torch.Tensor:
    return _mmq_run(x, weights, types, rows_out, out_f32)


@fused_mmq.register_fake
def _fake_mmq(x, weights, types, rows_out, out_f32):
    return x.new_empty((x.shape[0], sum(rows_out)), dtype=torch.float32 if out_f32 else torch.bfloat16)


@torch.library.custom_op("kaillm::fused_mmvq", mutates_args=())
def fused_mmvq(x: torch.Tensor, weights: list[torch.Tensor], types: list[int], rows_out: list[int],
               two_pass: int, out_f32: bool) -> torch.Tensor:
    return _run(x, weights, types, rows_out, two_pass, out_f32)


@fused_mmvq.register_fake
def _fake(x, weights, types, rows_out, two_pass, out_f32):
    return x.new_empty((x.shape[0], sum(rows_out)), dtype=torch.float32 if out_f32 else torch.bfloat16)


class FusedProjection:
    """A merged projection (one or more original GGUF matrices sharing an input)."""

    def __init__(self, parts):
        self.weights = [p.weight for p in parts]
        self.types = [int(p.weight_type) for p in parts]
        self.rows_out = [int(p.shape[0]) for p in parts]
        self.k = int(parts[0].shape[1])
        self.dtype = parts[0].dtype
        self.total = sum(self.rows_out)
        lib = library()
        self._supported = tuple(
            rows for rows in range(1, MAX_ROWS + 1)
            if all(lib.kai_fused_supported(t, n, self.k, rows) for t, n in zip(self.types, self.rows_out))
        )
        self._mmq = (
            mmq_mode()
            and all(t in MMQ_TYPES for t in self.types)
            and self.total % 4 == 0
            and self.k % 4 == 0
        )
        if self._mmq:
            device = parts[0].weight.device.index or 0
            count = len(parts)
            types = (ctypes.c_int * count)(*self.types)
            rows = (ctypes.c_int64 * count)(*self.rows_out)
            self._mmq = all(
                lib.kai_fused_mmq_workspace(device, types, rows, count, self.k, m, 0) > 0 for m in (16, 512)
            )

    def supports(self, x):
        rows = x.numel() // x.shape[-1] if x.shape[-1] else 0
        if not (x.dtype in _DTYPE_CODES and x.is_cuda):
            return False
        return rows in self._supported or (self._mmq and rows > MAX_ROWS)

    def _finish(self, out, lead, output_dtype):
        if output_dtype not in (torch.float32, torch.bfloat16):
            out = out.to(output_dtype)
        return out.reshape(*lead, self.total)

    def call_view(self, x, view, output_dtype=None):
        """The projection of x[..., view] for <= 8 rows (yaqa_linear.py:350-354 of the
        reference): view = (a, b, s) moves S-wide column segments from [a][b][s] to [b][a][s]."""
        output_dtype = self.dtype if output_dtype is None else output_dtype
        x2 = x.reshape(-1, self.k).contiguous()
        out = fused_mmvq_view(x2, self.weights, self.types, self.rows_out, int(view[0]), int(view[1]),
                              int(view[2]), output_dtype == torch.float32)
        return self._finish(out, x.shape[:-1], output_dtype)

    def call_swiglu(self, gate_up, output_dtype=None):
        """The projection of silu(gate) * up for <= 8 rows, gate_up = [gate | up] of width 2k."""
        output_dtype = self.dtype if output_dtype is None else output_dtype
        g2 = gate_up.reshape(-1, 2 * self.k).contiguous()
        out = fused_mmvq_swiglu(g2, self.weights, self.types, self.rows_out, output_dtype == torch.float32)
        return self._finish(out, gate_up.shape[:-1], output_dtype)

    def __call__(self, x, output_dtype=None):
        output_dtype = self.dtype if output_dtype is None else output_dtype
        x2 = x.reshape(-1, self.k).contiguous()
        if x2.shape[0] > MAX_ROWS:
            out = fused_mmq(x2, self.weights, self.types, self.rows_out, output_dtype == torch.float32)
        else:
            out = fused_mmvq(x2, self.weights, self.types, self.rows_out, mode() - 1,
                             output_dtype == torch.float32)
        return self._finish(out, x.shape[:-1], output_dtype)


def prepare(parts):
    """FusedProjection for compact GGUF parts, or None when any part is ineligible."""
    if mode() == 0 or not parts:
        return None
    k = parts[0].shape[1]
    for part in parts:
        if (
            not part.is_quantized
            or int(part.weight_type) not in TYPES
            or part.shape[1] != k
            or not part.weight.is_cuda
            or part.weight.dtype != torch.uint8
            or not part.weight.is_contiguous()
            or part.dtype not in (torch.bfloat16, torch.float16, torch.float32)
        ):
            return None
    fused = FusedProjection(parts)
    return fused if (fused._supported or fused._mmq) else None
