"""Merged GGUF projections as torch custom ops over libkai_hip.so.

The interface is the one the reference's plugin binds
(``vllm_gguf_plugin/quantization/native_fused.py``): module names ``ENV``, ``MAX_ROWS``,
``TYPES``, ``MMQ_TYPES``, ``mode()``, ``mmq_mode()``, ``library()``, ``ext_available()``,
``prepare(parts)`` returning a ``FusedProjection`` or ``None``, the producer protocol
``norm_prepare`` / ``CONSUMER_OF`` / ``STASH``, and the op schemas ``kaillm::fused_mmvq``,
``kaillm::fused_mmq``, ``kaillm::fused_mmvq_view``, ``kaillm::fused_mmvq_swiglu``.

How it is organised here: a ``_Group`` holds one projection's matrices with their C-ABI
argument arrays, built once; every op resolves its group from the weights it is given
(``_group_for``) and runs one of two plans:

* decode, 1..``MAX_ROWS`` rows: one activation buffer (prepared from x, from a column view
  of x, from a merged gate|up row, or taken from a producer's stash), then one GEMV launch
  per matrix into its column slice of the merged output;
* batched, more rows: one ``kai_fused_mmq_run`` call for the whole group with a scratch
  sized by ``kai_fused_mmq_workspace``.

``library()`` returns ``None`` when libkai_hip.so is not built, and ``prepare()`` then
returns ``None``, as the reference's bridge does when its native library is absent; the
ops themselves raise (``_require``). There is no CPU path.

KAILLM_FUSED_MMVQ: "0" disabled, "1" single pass (default), "2" two passes.
KAILLM_FUSED_MMQ: "0" disables the batched path, "1" (default) enables it.
"""
import ctypes
import os
from collections import OrderedDict

import torch

from . import native
from .formats import WEIGHT_TYPES

ENV = "KAILLM_FUSED_MMVQ"
MMQ_ENV = "KAILLM_FUSED_MMQ"
MAX_ROWS = 8
TYPES = WEIGHT_TYPES
MMQ_TYPES = WEIGHT_TYPES

# Activation element types the C ABI takes, by code.
_ACT_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def _env_choice(name, default, allowed):
    value = os.environ.get(name, default)
    if value not in allowed:
        raise ValueError(f"{name} must be one of {', '.join(allowed)}")
    return value


def mode():
    """0 (fused decode off), 1 (single-pass activation) or 2 (two passes)."""
    return int(_env_choice(ENV, "1", ("0", "1", "2")))


def mmq_mode():
    """Whether projections of more than MAX_ROWS rows take the batched entry."""
    return _env_choice(MMQ_ENV, "1", ("0", "1")) == "1"


def library():
    """libkai_hip.so, or None when it has not been built."""
    return native.library() if native.library_path().is_file() else None


def _require():
    lib = library()
    if lib is None:
        raise RuntimeError(f"{native.library_path()} is missing: build it with __graft_entry__.build()")
    return lib


def ext_available():
    """The fused activation producers can feed the decode GEMV (single-pass mode)."""
    lib = library()
    return lib is not None and hasattr(lib, "kai_fused_norm_prepare") and mode() == 1


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _out_dtype(out_f32):
    return torch.float32 if out_f32 else torch.bfloat16


class _Group:
    """The matrices of one merged projection (device pointers, types, rows) and their C-ABI
    argument arrays. It holds no tensor: the caller keeps the weights alive."""

    def __init__(self, key):
        ptrs, types, rows = key
        self.ptrs, self.types, self.rows = list(ptrs), list(types), list(rows)
        self.count = len(ptrs)
        self.total = sum(self.rows)
        self.offsets = [sum(self.rows[:i]) for i in range(self.count)]
        self.c_ptrs = (ctypes.c_void_p * self.count)(*self.ptrs)
        self.c_types = (ctypes.c_int * self.count)(*self.types)
        self.c_rows = (ctypes.c_int64 * self.count)(*self.rows)

    def new_output(self, m, out_f32, device):
        return torch.empty((m, self.total), dtype=_out_dtype(out_f32), device=device)

    def gemv(self, lib, activation, m, k, two_pass, out_f32, device):
        """One GEMV per matrix from a prepared activation into [m, total]."""
        out = self.new_output(m, out_f32, device)
        stream = torch.cuda.current_stream(device).cuda_stream
        base, elem = out.data_ptr(), out.element_size()
        for w, t, n, off in zip(self.ptrs, self.types, self.rows, self.offsets):
            native.check(lib, lib.kai_fused_mmvq(w, t, n, k, m, activation.data_ptr(), two_pass,
                                                 base + off * elem, 0 if out_f32 else 1, self.total, stream))
        return out

    def batched(self, lib, x, out_f32):
        """The whole group in one kai_fused_mmq_run call."""
        m, k = x.shape
        device = x.device.index if x.device.index is not None else torch.cuda.current_device()
        size = lib.kai_fused_mmq_workspace(device, self.c_types, self.c_rows, self.count, k, m, int(out_f32))
        if size == 0:
            raise RuntimeError(lib.current_direct_error().decode())
        scratch = torch.empty(size, dtype=torch.uint8, device=x.device)
        out = self.new_output(m, out_f32, x.device)
        native.check(lib, lib.kai_fused_mmq_run(self.c_ptrs, self.c_types, self.c_rows, self.count, x.data_ptr(),
                                                _ACT_CODE[x.dtype], x.stride(0), k, m, out.data_ptr(),
                                                0 if out_f32 else 1, 0, scratch.data_ptr(), size, device,
                                                _stream(x)))
        return out


_GROUPS = OrderedDict()
_MAX_GROUPS = 4096  # a model's projections; older entries are rebuilt on their next call


def _group_for(weights, types, rows):
    """The _Group of these weights, built once per distinct (pointers, types, rows)."""
    key = (tuple(w.data_ptr() for w in weights), tuple(int(t) for t in types), tuple(int(n) for n in rows))
    group = _GROUPS.get(key)
    if group is None:
        group = _GROUPS[key] = _Group(key)
        if len(_GROUPS) > _MAX_GROUPS:
            _GROUPS.popitem(last=False)
    return group


def _activation_buffer(lib, m, k, two_pass, device):
    return torch.empty(lib.kai_fused_activation_bytes(m, k, two_pass), dtype=torch.uint8, device=device)


# ---------------------------------------------------------------------------- producers
# A norm whose output feeds registered consumer projections stores that output's
# activation under its producer id (STASH[producer] = (key, activation, y)); a consumer
# projection, found by its first weight pointer in CONSUMER_OF, whose input is exactly that
# output (same storage, shape, stride, dtype and device) uses the stashed activation.
CONSUMER_OF = {}
STASH = {}


def _key(t):
    return (t.data_ptr(), t.shape[0], t.shape[1], t.stride(0), t.dtype, t.device)


def _stashed_activation(weights, x):
    producer = CONSUMER_OF.get(weights[0].data_ptr()) if CONSUMER_OF else None
    if producer is None:
        return None
    entry = STASH.get(producer)
    return entry[1] if entry is not None and entry[0] == _key(x) else None


def norm_prepare(producer, x, residual, weight32, eps):
    """Gemma RMSNorm of 1..MAX_ROWS rows that also prepares its output's activation.

    Returns (y bf16, fp32 residual stream or None), or None when the inputs are not ones the
    fused producer takes (the caller then runs its own norm). The stash keeps y alive, so its
    storage cannot be reused by a different tensor matching the key."""
    if not ext_available() or not x.is_cuda or x.dim() != 2 or not 1 <= x.shape[0] <= MAX_ROWS:
        return None
    m, k = x.shape
    if k % 32 or x.dtype not in (torch.bfloat16, torch.float32) or x.stride(1) != 1:
        return None
    if residual is not None and (residual.shape != x.shape or residual.stride(1) != 1
                                 or residual.dtype not in (torch.bfloat16, torch.float32)):
        return None
    lib = library()
    y = torch.empty((m, k), dtype=torch.bfloat16, device=x.device)
    r_out = None if residual is None else torch.empty((m, k), dtype=torch.float32, device=x.device)
    activation = _activation_buffer(lib, m, k, 0, x.device)
    r_args = (None, 0, 0, None) if residual is None else (
        residual.data_ptr(), _ACT_CODE[residual.dtype], residual.stride(0), r_out.data_ptr())
    native.check(lib, lib.kai_fused_norm_prepare(x.data_ptr(), _ACT_CODE[x.dtype], x.stride(0), r_args[0], r_args[1],
                                                 r_args[2], r_args[3], weight32.data_ptr(), float(eps), y.data_ptr(),
                                                 m, k, activation.data_ptr(), _stream(x)))
    STASH[producer] = (_key(y), activation, y)
    return y, r_out


# ---------------------------------------------------------------------------- torch ops

def _fake(x, rows_out, out_f32):
    return x.new_empty((x.shape[0], sum(rows_out)), dtype=_out_dtype(out_f32))


@torch.library.custom_op("kaillm::fused_mmvq", mutates_args=())
def fused_mmvq(x: torch.Tensor, weights: list[torch.Tensor], types: list[int], rows_out: list[int],
               two_pass: int, out_f32: bool) -> torch.Tensor:
    """x [m <= 8, k] through every matrix of the group: [m, sum(rows_out)], F32 or BF16."""
    lib = _require()
    m, k = x.shape
    group = _group_for(weights, types, rows_out)
    activation = _stashed_activation(weights, x) if two_pass == 0 else None
    if activation is None:
        activation = _activation_buffer(lib, m, k, two_pass, x.device)
        native.check(lib, lib.kai_fused_prepare(x.data_ptr(), _ACT_CODE[x.dtype], m, k, x.stride(0),
                                                activation.data_ptr(), two_pass, _stream(x)))
    return group.gemv(lib, activation, m, k, two_pass, out_f32, x.device)


@fused_mmvq.register_fake
def _(x, weights, types, rows_out, two_pass, out_f32):
    return _fake(x, rows_out, out_f32)


@torch.library.custom_op("kaillm::fused_mmq", mutates_args=())
def fused_mmq(x: torch.Tensor, weights: list[torch.Tensor], types: list[int], rows_out: list[int],
              out_f32: bool) -> torch.Tensor:
    """x [m > 8, k] through every matrix of the group in one batched call."""
    return _group_for(weights, types, rows_out).batched(_require(), x, out_f32)


@fused_mmq.register_fake
def _(x, weights, types, rows_out, out_f32):
    return _fake(x, rows_out, out_f32)


@torch.library.custom_op("kaillm::fused_mmvq_view", mutates_args=())
def fused_mmvq_view(x: torch.Tensor, weights: list[torch.Tensor], types: list[int], rows_out: list[int],
                    a: int, b: int, s: int, out_f32: bool) -> torch.Tensor:
    """The group on x[..., view] with no copy: x's columns read as [a][b][s] -> [b][a][s]."""
    lib = _require()
    m, k = x.shape
    activation = _activation_buffer(lib, m, k, 0, x.device)
    native.check(lib, lib.kai_fused_prepare_view(x.data_ptr(), _ACT_CODE[x.dtype], m, k, x.stride(0),
                                                 activation.data_ptr(), a, b, s, _stream(x)))
    return _group_for(weights, types, rows_out).gemv(lib, activation, m, k, 0, out_f32, x.device)


@fused_mmvq_view.register_fake
def _(x, weights, types, rows_out, a, b, s, out_f32):
    return _fake(x, rows_out, out_f32)


@torch.library.custom_op("kaillm::fused_mmvq_swiglu", mutates_args=())
def fused_mmvq_swiglu(gate_up: torch.Tensor, weights: list[torch.Tensor], types: list[int], rows_out: list[int],
                      out_f32: bool) -> torch.Tensor:
    """The group on silu(gate) * up, read straight from a merged [m, 2k] gate_up output."""
    lib = _require()
    m, k = gate_up.shape[0], gate_up.shape[1] // 2
    activation = _activation_buffer(lib, m, k, 0, gate_up.device)
    native.check(lib, lib.kai_fused_prepare_swiglu(gate_up.data_ptr(), _ACT_CODE[gate_up.dtype], m, k,
                                                   gate_up.stride(0), activation.data_ptr(), _stream(gate_up)))
    return _group_for(weights, types, rows_out).gemv(lib, activation, m, k, 0, out_f32, gate_up.device)


@fused_mmvq_swiglu.register_fake
def _(gate_up, weights, types, rows_out, out_f32):
    return _fake(gate_up, rows_out, out_f32)


# ---------------------------------------------------------------------------- projection

def _rows_of(x):
    return x.numel() // x.shape[-1] if x.shape[-1] else 0


class FusedProjection:
    """One or more original GGUF matrices that share an input, run as one projection.

    ``weights``, ``types``, ``rows_out``, ``k``, ``dtype`` and ``total`` describe the group;
    ``_supported`` lists the decode row counts every matrix takes and ``_mmq`` whether the
    batched entry takes the group."""

    def __init__(self, parts):
        lib = _require()
        self.weights = [p.weight for p in parts]
        self.types = [int(p.weight_type) for p in parts]
        self.rows_out = [int(p.shape[0]) for p in parts]
        self.k = int(parts[0].shape[1])
        self.dtype = parts[0].dtype
        self.total = sum(self.rows_out)
        self._group = _group_for(self.weights, self.types, self.rows_out)
        self._supported = tuple(m for m in range(1, MAX_ROWS + 1) if all(
            lib.kai_fused_supported(t, n, self.k, m) for t, n in zip(self.types, self.rows_out)))
        self._mmq = False
        if mmq_mode() and all(t in MMQ_TYPES for t in self.types) and self.total % 4 == 0 and self.k % 4 == 0:
            device = self.weights[0].device.index or 0
            g = self._group
            self._mmq = lib.kai_fused_mmq_workspace(device, g.c_types, g.c_rows, g.count, self.k, MAX_ROWS + 1, 0) > 0

    def supports(self, x):
        """Whether x (any leading shape, last dimension k) runs on the fused path."""
        if x.dtype not in _ACT_CODE or not x.is_cuda:
            return False
        m = _rows_of(x)
        return m in self._supported or (self._mmq and m > MAX_ROWS)

    def _shaped(self, out, lead, output_dtype):
        return (out if out.dtype == output_dtype else out.to(output_dtype)).reshape(*lead, self.total)

    def __call__(self, x, output_dtype=None):
        output_dtype = output_dtype or self.dtype
        flat = x.reshape(-1, self.k).contiguous()
        f32 = output_dtype == torch.float32
        if flat.shape[0] > MAX_ROWS:
            out = fused_mmq(flat, self.weights, self.types, self.rows_out, f32)
        else:
            out = fused_mmvq(flat, self.weights, self.types, self.rows_out, mode() - 1, f32)
        return self._shaped(out, x.shape[:-1], output_dtype)

    def call_view(self, x, view, output_dtype=None):
        """The projection of x[..., view] for up to MAX_ROWS rows; view = (a, b, s) reads
        x's columns as [a][b][s] in the order [b][a][s]."""
        output_dtype = output_dtype or self.dtype
        a, b, s = (int(v) for v in view)
        out = fused_mmvq_view(x.reshape(-1, self.k).contiguous(), self.weights, self.types, self.rows_out, a, b,
                              s, output_dtype == torch.float32)
        return self._shaped(out, x.shape[:-1], output_dtype)

    def call_swiglu(self, gate_up, output_dtype=None):
        """The projection of silu(gate) * up for up to MAX_ROWS rows of [gate | up] (2k)."""
        output_dtype = output_dtype or self.dtype
        out = fused_mmvq_swiglu(gate_up.reshape(-1, 2 * self.k).contiguous(), self.weights, self.types,
                                self.rows_out, output_dtype == torch.float32)
        return self._shaped(out, gate_up.shape[:-1], output_dtype)


def _eligible(part, k):
    w = part.weight
    return (part.is_quantized and int(part.weight_type) in TYPES and part.shape[1] == k and w.is_cuda
            and w.dtype == torch.uint8 and w.is_contiguous()
            and part.dtype in (torch.bfloat16, torch.float16, torch.float32))


def prepare(parts):
    """A FusedProjection over compact GGUF parts, or None when the fused path is off, the
    library is not built, a part is not eligible, or no row count is supported."""
    if not parts or mode() == 0 or library() is None:
        return None
    k = parts[0].shape[1]
    if not all(_eligible(p, k) for p in parts):
        return None
    fused = FusedProjection(parts)
    return fused if fused._supported or fused._mmq else None
