"""Pin the oracle's fused activation producers (view, SwiGLU, Gemma RMSNorm) on the CPU.

The reference's producers are kai_prepare_ext.cuh:121-251 (entries
current_ggml_direct.cu:883-944). Two of their steps have no specified bits there: CUDA's
expf and the order of the norm's sum of squares. The oracle fixes them as the HIP kernels
do, so the checks below are against what the mathematics fixes instead: libm's double exp
(2 ulp), an FP64 RMSNorm (bf16 rounding), torch's own bf16 conversion, the view as a plain
transposed copy through the already-pinned oracle_prepare, and SwiGLU values that are
exact in the input dtype.
"""
import numpy as np
import pytest
import torch

import _oracle as O

BF16 = "bf16"


def bf16_bits(x32):
    """torch's float32 -> bfloat16 rounding, as uint16 bits (independent of the oracle)."""
    return torch.from_numpy(np.ascontiguousarray(x32, dtype=np.float32)).to(torch.bfloat16).view(
        torch.int16).numpy().view(np.uint16)


def bits_to_f32(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def as_dtype(x32, dtype):
    if dtype == BF16:
        return bf16_bits(x32)
    return x32.astype(dtype)


def to_f64(x):
    return bits_to_f32(x).astype(np.float64) if x.dtype == np.uint16 else x.astype(np.float64)


# ----------------------------------------------------------------- scalar helpers

def test_float_to_bf16_matches_torch():
    rng = np.random.default_rng(10)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(3.0),
        (rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32)).view(np.float32),
        # exact ties at the bf16 boundary, both parities, and specials
        (np.arange(0x3F800000, 0x3F800000 + 0x40000, 0x8000, dtype=np.uint32)).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45, 3.4028235e38, 1.1754944e-38], dtype=np.float32),
    ])
    ours = np.array([O.lib().oracle_float_to_bf16(float(v)) for v in vals], dtype=np.uint16)
    want = bf16_bits(vals)
    nan = np.isnan(vals)
    assert np.array_equal(ours[~nan], want[~nan])
    assert np.all(np.isnan(bits_to_f32(ours[nan])))


def _ulp32(x64):
    """Spacing of float32 at |x| (subnormal spacing 2^-149 below 2^-126)."""
    e = np.floor(np.log2(np.maximum(np.abs(x64), 2.0 ** -126)))
    return 2.0 ** (e - 23)


def test_expf_within_two_ulp_of_double_exp():
    rng = np.random.default_rng(11)
    x = np.concatenate([
        rng.uniform(-103.9, 88.72, 40000), rng.uniform(-1.0, 1.0, 20000), rng.uniform(-20.0, 20.0, 20000),
        np.arange(-149, 128, dtype=np.float64) * np.log(2.0),  # n ln2: reduction boundaries
    ]).astype(np.float32)
    got = np.array([O.lib().oracle_expf(float(v)) for v in x], dtype=np.float64)
    want = np.exp(x.astype(np.float64))
    err = np.abs(got - want) / _ulp32(want)
    assert err.max() <= 2.0, (x[err.argmax()], err.max())


def test_expf_special_values():
    e = O.lib().oracle_expf
    assert e(0.0) == 1.0 and e(-0.0) == 1.0
    assert np.isnan(e(float("nan")))
    assert e(88.7229) == np.inf and e(float("inf")) == np.inf
    assert e(-104.0) == 0.0 and e(float("-inf")) == 0.0
    assert 0.0 < e(-100.0) < 2.0 ** -126  # subnormal range is kept
    assert e(88.72) < np.inf


# ----------------------------------------------------------------- view

@pytest.mark.parametrize("dtype", [np.float32, BF16, np.float16])
@pytest.mark.parametrize("m,a,b,s", [(1, 2, 3, 32), (3, 16, 4, 64), (8, 4, 40, 32), (2, 1, 5, 128), (2, 7, 1, 96)])
def test_view_is_the_transposed_copy(dtype, m, a, b, s):
    """Stored column c reads x column ((c/s)%a)*b*s + (c/(a*s))*s + c%s: x viewed as
    [a][b][s] and stored as [b][a][s]."""
    rng = np.random.default_rng(a * 1000 + b * 10 + s)
    k = a * b * s
    x = as_dtype(rng.standard_normal((m, k)).astype(np.float32) * 4, dtype)
    xt = np.ascontiguousarray(x.reshape(m, a, b, s).transpose(0, 2, 1, 3).reshape(m, k))
    want = O.prepare(xt, dtype_code=1 if dtype == BF16 else None)
    assert np.array_equal(O.prepare_view(x, a, b, s), want)


def test_view_rejects_inconsistent_shapes():
    x = np.zeros((1, 96), dtype=np.float32)
    out = np.zeros(O.activation_bytes(1, 96), dtype=np.uint8)
    f = O.lib().oracle_prepare_view
    assert f(O._p(x), 0, 1, 96, 96, O._p(out), 2, 2, 32) == -1   # a*b*s != k
    assert f(O._p(x), 0, 1, 96, 96, O._p(out), 3, 2, 16) == -1   # s % 32


# ----------------------------------------------------------------- SwiGLU

@pytest.mark.parametrize("dtype", [np.float32, BF16, np.float16])
def test_swiglu_exact_cases(dtype):
    """Where exp(-g) is exactly 1 (g = 0), 0 (g >= 104) or inf (g <= -89), silu(g) is
    g / 2, g or -0, and the activation is the preparation of rd(rd(silu(g)) * u)
    computed here in FP64 with the dtype's own rounding; swapping gate and up, or
    reading the wrong half, changes the codes."""
    rng = np.random.default_rng(12)
    m, k = 3, 256
    g = rng.choice(np.array([0.0, 104.0, 160.0, 1024.0, -89.0, -300.0, 250.0], dtype=np.float32), size=(m, k))
    if dtype == np.float16:  # f16 tops out at 65504: keep g * u in range
        g = np.where(np.abs(g) > 300, np.sign(g) * 300, g).astype(np.float32)
    u = rng.standard_normal((m, k)).astype(np.float32)
    gd, ud = as_dtype(g, dtype), as_dtype(u, dtype)
    g64, u64 = to_f64(gd), to_f64(ud)
    silu = np.where(g64 == 0, 0.0, np.where(g64 > 0, g64, -0.0))
    prod32 = (silu * u64).astype(np.float32)  # silu is exact in the dtype; one rounding of g*u
    v = as_dtype(prod32, dtype)
    want = O.prepare(v, dtype_code=1 if dtype == BF16 else None)
    got = O.prepare_swiglu(np.concatenate([gd, ud], axis=1))
    assert np.array_equal(got, want)
    swapped = O.prepare_swiglu(np.concatenate([ud, gd], axis=1))
    assert not np.array_equal(swapped, want)


@pytest.mark.parametrize("dtype", [np.float32, BF16, np.float16])
def test_swiglu_random_against_fp64(dtype):
    rng = np.random.default_rng(13)
    m, k = 4, 1024
    g = as_dtype((rng.standard_normal((m, k)) * 3).astype(np.float32), dtype)
    u = as_dtype(rng.standard_normal((m, k)).astype(np.float32), dtype)
    g64, u64 = to_f64(g), to_f64(u)
    ref = g64 / (1.0 + np.exp(-g64)) * u64
    d, _, q, inv, _ = O.split_activation(O.prepare_swiglu(np.concatenate([g, u], axis=1)), m, k)
    deq = np.repeat(d.astype(np.float64), 32, axis=1) * q * inv[:, None].astype(np.float64)
    step = np.repeat(d.astype(np.float64), 32, axis=1) * inv[:, None]
    rel = {np.float32: 1e-6, BF16: 2.0 ** -7, np.float16: 2.0 ** -10}[dtype]
    assert np.all(np.abs(deq - ref) <= 0.6 * step + rel * np.abs(ref) + 1e-30)


# ----------------------------------------------------------------- Gemma RMSNorm

@pytest.mark.parametrize("xdtype", [np.float32, BF16])
@pytest.mark.parametrize("rdtype", [None, np.float32, BF16])
@pytest.mark.parametrize("m,k", [(1, 96), (3, 5120), (2, 32768)])
def test_norm_against_fp64(xdtype, rdtype, m, k):
    rng = np.random.default_rng(k + m)
    x = as_dtype((rng.standard_normal((m, k)) * 2).astype(np.float32), xdtype)
    r = None if rdtype is None else as_dtype(rng.standard_normal((m, k)).astype(np.float32), rdtype)
    w = (1.0 + rng.standard_normal(k) * 0.1).astype(np.float32)
    eps = 1e-6
    act, y, r_out = O.norm_prepare(x, w, eps, r)
    v32 = to_f64(x).astype(np.float32)
    if r is not None:
        v32 = v32 + to_f64(r).astype(np.float32)  # one float32 addition
        assert np.array_equal(r_out.view(np.uint32), v32.view(np.uint32))
    v = v32.astype(np.float64)
    ref = v / np.sqrt((v * v).mean(axis=1, keepdims=True) + eps) * w
    yf = bits_to_f32(y).astype(np.float64)
    assert np.all(np.abs(yf - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-30)
    near = bf16_bits(ref.astype(np.float32))
    assert np.mean(near != y) < 0.01  # off torch's rounding of the FP64 value only at boundaries
    assert np.array_equal(act, O.prepare(y, dtype_code=1))  # the activation quantises stored y


def test_norm_eps_and_zero_row():
    k = 64
    x = np.zeros((1, k), dtype=np.float32)
    w = np.ones(k, dtype=np.float32)
    act, y, _ = O.norm_prepare(x, w, 1e-6)
    assert np.all(y == 0)
    _, _, q, inv, _ = O.split_activation(act, 1, k)
    assert np.all(q == 0) and inv[0] == 1.0
    x = np.full((1, k), 3.0, dtype=np.float32)  # rms 3, eps 7: rstd = 1/4
    _, y, _ = O.norm_prepare(x, w, 7.0)
    assert np.all(bits_to_f32(y) == 0.75)
