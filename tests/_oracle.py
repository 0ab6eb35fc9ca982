"""numpy wrappers around the CPU oracle (oracle/liboracle.so) — the checker.

Test infrastructure only; the product (kaillm_amd) never imports this.
"""
import ctypes
import subprocess
from functools import lru_cache
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_SO = ROOT / "oracle" / "liboracle.so"

Q4_0, Q8_0, Q8_1, Q2_K, Q4_K, Q6_K, IQ3_S = 2, 8, 9, 10, 12, 14, 21
WEIGHT_TYPES = (Q8_0, Q4_0, Q4_K, Q6_K, Q2_K, IQ3_S)
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q8_1: (32, 36), Q2_K: (256, 84), Q4_K: (256, 144),
         Q6_K: (256, 210), IQ3_S: (256, 110)}
NAMES = {Q4_0: "Q4_0", Q8_0: "Q8_0", Q2_K: "Q2_K", Q4_K: "Q4_K", Q6_K: "Q6_K", IQ3_S: "IQ3_S"}


@lru_cache(maxsize=1)
def lib():
    if not ORACLE_SO.is_file():
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
    o = ctypes.CDLL(str(ORACLE_SO))
    i64, ptr, c_int = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int
    o.oracle_half_to_float.argtypes = [ctypes.c_uint16]
    o.oracle_half_to_float.restype = ctypes.c_float
    o.oracle_float_to_half.argtypes = [ctypes.c_float]
    o.oracle_float_to_half.restype = ctypes.c_uint16
    o.oracle_activation_bytes.argtypes = [i64, i64, c_int]
    o.oracle_activation_bytes.restype = ctypes.c_size_t
    o.oracle_prepare.argtypes = [ptr, c_int, i64, i64, i64, ptr, c_int]
    o.oracle_prepare.restype = c_int
    o.oracle_dequantize_row.argtypes = [c_int, ptr, i64, ptr]
    o.oracle_dequantize_row.restype = c_int
    o.oracle_mul_mat.argtypes = [c_int, ptr, i64, i64, i64, ptr, c_int, ptr, c_int]
    o.oracle_mul_mat.restype = c_int
    o.oracle_mul_mat_f32.argtypes = [c_int, ptr, i64, i64, i64, ptr, c_int, ptr, i64, c_int]
    o.oracle_mul_mat_f32.restype = c_int
    o.oracle_float_to_bf16.argtypes = [ctypes.c_float]
    o.oracle_float_to_bf16.restype = ctypes.c_uint16
    o.oracle_expf.argtypes = [ctypes.c_float]
    o.oracle_expf.restype = ctypes.c_float
    o.oracle_prepare_view.argtypes = [ptr, c_int, i64, i64, i64, ptr, i64, i64, i64]
    o.oracle_prepare_view.restype = c_int
    o.oracle_prepare_swiglu.argtypes = [ptr, c_int, i64, i64, i64, ptr]
    o.oracle_prepare_swiglu.restype = c_int
    o.oracle_norm_prepare.argtypes = [ptr, c_int, i64, ptr, c_int, i64, ptr, ptr, ctypes.c_float, ptr, i64, i64,
                                      ptr]
    o.oracle_norm_prepare.restype = c_int
    o.oracle_mmq_layout.argtypes = [c_int]
    o.oracle_mmq_layout.restype = c_int
    o.oracle_mmq_blocks128.argtypes = [i64]
    o.oracle_mmq_blocks128.restype = i64
    o.oracle_mmq_plane_bytes.argtypes = [i64, i64]
    o.oracle_mmq_plane_bytes.restype = ctypes.c_size_t
    o.oracle_prepare_mmq.argtypes = [ptr, c_int, i64, i64, i64, c_int, ptr, ptr]
    o.oracle_prepare_mmq.restype = c_int
    o.oracle_mul_mat_mmq.argtypes = [c_int, ptr, i64, i64, i64, ptr, ptr, ptr, c_int]
    o.oracle_mul_mat_mmq.restype = c_int
    o.oracle_prepare_legacy.argtypes = [ptr, c_int, i64, i64, i64, ptr]
    o.oracle_prepare_legacy.restype = c_int
    o.oracle_mul_mat_legacy.argtypes = [c_int, ptr, i64, i64, i64, ptr, c_int, ptr, c_int]
    o.oracle_mul_mat_legacy.restype = c_int
    o.oracle_build_info.restype = ctypes.c_char_p
    return o


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


DTYPE_CODE = {np.float32: 0, "bf16": 1, np.float16: 2}


def activation_bytes(m, k, two_pass=0):
    return lib().oracle_activation_bytes(m, k, two_pass)


def prepare(x, two_pass=0, dtype_code=None, stride=None):
    """x: float32 [m,k] (code 0), float16 (code 2) or uint16 bf16 bits (code 1)."""
    x = np.ascontiguousarray(x)
    if dtype_code is None:
        dtype_code = 0 if x.dtype == np.float32 else 2 if x.dtype == np.float16 else 1
    m, cols = x.shape
    k = cols if stride is None else stride[1]
    stride_x = cols
    out = np.zeros(activation_bytes(m, k, two_pass), dtype=np.uint8)
    assert lib().oracle_prepare(_p(x), dtype_code, m, k, stride_x, _p(out), two_pass) == 0
    return out


def _code(x):
    return 0 if x.dtype == np.float32 else 2 if x.dtype == np.float16 else 1


def prepare_view(x, a, b, s):
    """Activation of x's columns permuted as [a][b][s] -> [b][a][s] (bf16 as uint16 bits)."""
    x = np.ascontiguousarray(x)
    m, k = x.shape
    out = np.zeros(activation_bytes(m, k), dtype=np.uint8)
    assert lib().oracle_prepare_view(_p(x), _code(x), m, k, k, _p(out), a, b, s) == 0
    return out


def prepare_swiglu(gate_up):
    """Activation of rd(rd(silu(gate)) * up) from a merged [m, 2k] row."""
    gate_up = np.ascontiguousarray(gate_up)
    m, k2 = gate_up.shape
    k = k2 // 2
    out = np.zeros(activation_bytes(m, k), dtype=np.uint8)
    assert lib().oracle_prepare_swiglu(_p(gate_up), _code(gate_up), m, k, k2, _p(out)) == 0
    return out


def norm_prepare(x, w32, eps, residual=None):
    """-> (activation, y bf16 bits [m, k], residual_out f32 [m, k] or None)."""
    x = np.ascontiguousarray(x)
    m, k = x.shape
    w32 = np.ascontiguousarray(w32, dtype=np.float32)
    out = np.zeros(activation_bytes(m, k), dtype=np.uint8)
    y = np.zeros((m, k), dtype=np.uint16)
    r_out = None
    rp, rcode = None, 0
    if residual is not None:
        residual = np.ascontiguousarray(residual)
        r_out = np.zeros((m, k), dtype=np.float32)
        rp, rcode = _p(residual), _code(residual)
    assert lib().oracle_norm_prepare(_p(x), _code(x), k, rp, rcode, k, None if r_out is None else _p(r_out),
                                     _p(w32), eps, _p(y), m, k, _p(out)) == 0
    return out, y, r_out


def split_activation(buf, m, k, two_pass=0):
    """-> (d [m, k/32] f32, s [m, k/32] f32, q [m, k] int8, inverse [m] f32, pass-2 tuple or None)."""
    nb = k // 32
    pass_bytes = (m * nb * 36 + 255) // 256 * 256

    def one(off):
        blocks = buf[off:off + m * nb * 36].reshape(m, nb, 36)
        d = blocks[:, :, 0:2].copy().view(np.float16).reshape(m, nb).astype(np.float32)
        s = blocks[:, :, 2:4].copy().view(np.float16).reshape(m, nb).astype(np.float32)
        q = blocks[:, :, 4:].copy().view(np.int8).reshape(m, k)
        return d, s, q

    d, s, q = one(0)
    p2 = one(pass_bytes) if two_pass else None
    inv_off = pass_bytes * (2 if two_pass else 1)
    inverse = buf[inv_off:inv_off + 4 * m].copy().view(np.float32)
    return d, s, q, inverse, p2


def dequantize(qtype, w, k):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    n = w.shape[0]
    out = np.empty((n, k), dtype=np.float32)
    for r in range(n):
        assert lib().oracle_dequantize_row(qtype, _p(w[r]), k, _p(out[r])) == 0
    return out


def mul_mat(qtype, w, k, activation, m, two_pass=0, threads=8):
    """Reference GEMV/GEMM in FP64: out [m, n]."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    n = w.shape[0]
    out = np.empty((m, n), dtype=np.float64)
    assert lib().oracle_mul_mat(qtype, _p(w), n, k, m, _p(activation), two_pass, _p(out), threads) == 0
    return out


def normwise_rel(y, ref):
    """max |y - ref| / max |ref| per output row (activation row), worst row."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    num = np.abs(y - ref).max(axis=-1)
    den = np.abs(ref).max(axis=-1)
    return float(np.max(num / np.maximum(den, 1e-300)))


def random_blocks(qtype, n, k, rng):
    """Random but valid wire bytes: every bit pattern, with fp16 scales set to sane values."""
    qk, bb = BLOCK[qtype]
    nb = k // qk
    w = rng.integers(0, 256, size=(n, nb, bb), dtype=np.uint8)

    def put_half(off, lo, hi):
        vals = rng.uniform(lo, hi, size=(n, nb)).astype(np.float16)
        w[:, :, off:off + 2] = vals.view(np.uint8).reshape(n, nb, 2)

    if qtype in (Q8_0, Q4_0):
        put_half(0, -0.01, 0.01)
    elif qtype == Q4_K:
        put_half(0, 0.0, 0.002)
        put_half(2, 0.0, 0.002)
    elif qtype == Q6_K:
        put_half(208, -0.002, 0.002)
    elif qtype == Q2_K:
        put_half(80, 0.0, 0.004)
        put_half(82, 0.0, 0.004)
    elif qtype == IQ3_S:
        put_half(0, 0.0, 0.002)
    return w.reshape(n, nb * bb)


# ----------------------------------------------------------------- batched path (m > 8)

D4, DS4, D2S6 = 0, 1, 2
LAYOUT_NAMES = {D4: "D4", DS4: "DS4", D2S6: "D2S6"}


def mmq_layout(qtype):
    return lib().oracle_mmq_layout(qtype)


def mmq_blocks128(k):
    return lib().oracle_mmq_blocks128(k)


def prepare_mmq(x, layout, dtype_code=None):
    """-> (plane uint8 [K/128 padded, m, 144], inverse f32 [m]) of the batched path."""
    x = np.ascontiguousarray(x)
    if dtype_code is None:
        dtype_code = _code(x)
    m, k = x.shape
    plane = np.zeros(lib().oracle_mmq_plane_bytes(m, k), dtype=np.uint8)
    inverse = np.zeros(m, dtype=np.float32)
    assert lib().oracle_prepare_mmq(_p(x), dtype_code, m, k, k, layout, _p(plane), _p(inverse)) == 0
    return plane.reshape(mmq_blocks128(k), m, 144), inverse


def split_plane(plane, layout):
    """-> (q int8 [m, Kpad], d [m, Kpad/G] f32, sums [m, Kpad/16 or Kpad/32] f32 or None).

    sums: DS4 per 32 values; D2S6 per 16 values with NaN where no sum is stored."""
    nb, m, _ = plane.shape
    q = plane[:, :, 16:].copy().view(np.int8).transpose(1, 0, 2).reshape(m, nb * 128)
    hdr = plane[:, :, :16].copy()
    if layout == D4:
        d = hdr.view(np.float32).reshape(nb, m, 4).transpose(1, 0, 2).reshape(m, nb * 4)
        return q, d, None
    h = hdr.view(np.float16).astype(np.float32).reshape(nb, m, 8).transpose(1, 0, 2)
    if layout == DS4:
        return q, h[:, :, 0::2].reshape(m, nb * 4), h[:, :, 1::2].reshape(m, nb * 4)
    sums = np.full((m, nb, 8), np.nan, dtype=np.float32)
    sums[:, :, :6] = h[:, :, 2:8]
    return q, h[:, :, :2].reshape(m, nb * 2), sums.reshape(m, nb * 8)


def mul_mat_mmq(qtype, w, k, plane, inverse, threads=8):
    """Reference batched GEMM (GGML MMQ arithmetic) in FP64: out [m, n]."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    plane = np.ascontiguousarray(plane)
    n = w.shape[0]
    m = plane.shape[1]
    out = np.empty((m, n), dtype=np.float64)
    assert lib().oracle_mul_mat_mmq(qtype, _p(w), n, k, m, _p(plane), _p(inverse), _p(out), threads) == 0
    return out


def prepare_legacy(x, dtype_code=None):
    """The legacy _C_gguf activation of x [m, k] (float32 / float16 / bf16 bits as uint16)."""
    x = np.ascontiguousarray(x)
    if dtype_code is None:
        dtype_code = _code(x)
    m, k = x.shape
    out = np.zeros(activation_bytes(m, k), dtype=np.uint8)
    assert lib().oracle_prepare_legacy(_p(x), dtype_code, m, k, k, _p(out)) == 0
    return out


def mul_mat_legacy(qtype, w, k, activation, m, batched, threads=8):
    """ggml_mul_mat_vec_a8 (batched=0) / ggml_mul_mat_a8 (batched=1) in FP64: out [m, n]."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    n = w.shape[0]
    out = np.empty((m, n), dtype=np.float64)
    assert lib().oracle_mul_mat_legacy(qtype, _p(w), n, k, m, _p(activation), batched, _p(out), threads) == 0
    return out


def legacy_reference(qtype, w, x, batched, dtype_code=None, threads=8):
    """The legacy op's result for x [m, k]."""
    return mul_mat_legacy(qtype, w, x.shape[1], prepare_legacy(x, dtype_code), x.shape[0], batched, threads)


def mmq_reference(qtype, w, x, dtype_code=None, threads=8):
    """The batched path's result for x [m, k] (float32 / float16 / bf16 bits as uint16)."""
    k = x.shape[1]
    plane, inverse = prepare_mmq(x, mmq_layout(qtype), dtype_code)
    return mul_mat_mmq(qtype, w, k, plane, inverse, threads)
