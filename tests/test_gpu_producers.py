"""Fused activation producers on the GPU against the CPU oracle, through the C ABI.

kai_fused_prepare_view / kai_fused_prepare_swiglu / kai_fused_norm_prepare replace the
reference's entries of the same names (current_ggml_direct.cu:883-944). Bar: bit-exact
activation bytes, bf16 y and fp32 residual stream; the oracle repeats the kernels' fixed
exp and reduction order, and is pinned on the CPU (test_oracle_producers.py).
"""
import numpy as np
import pytest
import torch

import _oracle as O
from test_gpu_parity import DEV, _stream, to_dev, used_bytes

pytestmark = pytest.mark.gpu

CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def host(t):
    """Tensor -> numpy in the oracle's encoding (bf16 as uint16 bits)."""
    t = t.contiguous().cpu()
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()


def act_buffer(kai, m, k):
    return torch.full((kai.kai_fused_activation_bytes(m, k, 0),), 0xA5, dtype=torch.uint8, device=DEV)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,a,b,s,pad", [(1, 2, 3, 32, 0), (3, 16, 8, 32, 64), (8, 4, 40, 32, 0),
                                         (2, 32, 4, 128, 32), (5, 1, 160, 32, 0)])
def test_view_bit_exact(kai, dtype, m, a, b, s, pad):
    k = a * b * s
    print(f"view dtype={dtype} m={m} a={a} b={b} s={s} pad={pad}", flush=True)
    rng = np.random.default_rng(k + m)
    full = to_dev((rng.standard_normal((m, k + pad)) * rng.uniform(0.01, 50, (m, 1))).astype(np.float32)).to(dtype)
    x = full[:, :k]
    act = act_buffer(kai, m, k)
    st = kai.kai_fused_prepare_view(x.data_ptr(), CODE[dtype], m, k, x.stride(0), act.data_ptr(), a, b, s,
                                    _stream())
    assert st == 0, kai.current_direct_error()
    torch.cuda.synchronize()
    ref = O.prepare_view(host(x), a, b, s)
    assert np.array_equal(used_bytes(act.cpu().numpy(), m, k, 0), used_bytes(ref, m, k, 0))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,k,pad", [(1, 256, 0), (3, 5120, 64), (8, 17408, 0), (2, 32768, 0), (4, 96, 32)])
def test_swiglu_bit_exact(kai, dtype, m, k, pad):
    print(f"swiglu dtype={dtype} m={m} k={k} pad={pad}", flush=True)
    rng = np.random.default_rng(k * 3 + m)
    g = rng.standard_normal((m, k)) * 4
    g[:, ::17] = rng.uniform(-120, 120, g[:, ::17].shape)  # exp overflow, underflow, subnormal
    g[:, 5::31] = 0.0
    u = rng.standard_normal((m, k))
    full = to_dev(np.concatenate([g, u, np.zeros((m, pad))], axis=1).astype(np.float32)).to(dtype)
    act = act_buffer(kai, m, k)
    st = kai.kai_fused_prepare_swiglu(full.data_ptr(), CODE[dtype], m, k, full.stride(0), act.data_ptr(),
                                      _stream())
    assert st == 0, kai.current_direct_error()
    torch.cuda.synchronize()
    ref = O.prepare_swiglu(host(full[:, :2 * k]))
    assert np.array_equal(used_bytes(act.cpu().numpy(), m, k, 0), used_bytes(ref, m, k, 0))


@pytest.mark.parametrize("xdtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rdtype", [None, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("m,k,pad", [(1, 96, 0), (3, 2560, 32), (8, 5120, 0), (2, 32768, 0)])
def test_norm_bit_exact(kai, xdtype, rdtype, m, k, pad):
    print(f"norm x={xdtype} r={rdtype} m={m} k={k} pad={pad}", flush=True)
    rng = np.random.default_rng(k * 5 + m)
    xs = rng.standard_normal((m, k + pad)) * rng.uniform(0.1, 30, (m, 1))
    x = to_dev(xs.astype(np.float32)).to(xdtype)[:, :k]
    r = None
    if rdtype is not None:
        r = to_dev(rng.standard_normal((m, k + pad)).astype(np.float32)).to(rdtype)[:, :k]
    w = to_dev((1.0 + rng.standard_normal(k) * 0.2).astype(np.float32))
    eps = 1e-6
    y = torch.empty((m, k), dtype=torch.bfloat16, device=DEV)
    r_out = torch.full((m, k), float("nan"), dtype=torch.float32, device=DEV) if r is not None else None
    act = act_buffer(kai, m, k)
    st = kai.kai_fused_norm_prepare(
        x.data_ptr(), CODE[xdtype], x.stride(0), None if r is None else r.data_ptr(),
        0 if r is None else CODE[rdtype], 0 if r is None else r.stride(0),
        None if r_out is None else r_out.data_ptr(), w.data_ptr(), eps, y.data_ptr(), m, k, act.data_ptr(),
        _stream())
    assert st == 0, kai.current_direct_error()
    torch.cuda.synchronize()
    ref_act, ref_y, ref_r = O.norm_prepare(host(x), w.cpu().numpy(), eps, None if r is None else host(r))
    assert np.array_equal(host(y), ref_y)
    if r is not None:
        assert np.array_equal(r_out.cpu().numpy().view(np.uint32), ref_r.view(np.uint32))
    assert np.array_equal(used_bytes(act.cpu().numpy(), m, k, 0), used_bytes(ref_act, m, k, 0))


def test_producer_feeds_the_gemv(kai):
    """The SwiGLU producer's activation drives kai_fused_mmvq like kai_fused_prepare's:
    the Q4_K down projection on it matches the oracle's GEMV on the oracle's activation."""
    from test_gpu_parity import TOL_F32

    print("swiglu -> mmvq", flush=True)
    rng = np.random.default_rng(77)
    m, k, n = 2, 2048, 640
    gu = to_dev(rng.standard_normal((m, 2 * k)).astype(np.float32)).to(torch.bfloat16)
    w = O.random_blocks(O.Q4_K, n, k, rng)
    act = act_buffer(kai, m, k)
    assert kai.kai_fused_prepare_swiglu(gu.data_ptr(), 1, m, k, 2 * k, act.data_ptr(), _stream()) == 0
    w_dev = to_dev(w.reshape(n, -1))
    out = torch.empty((m, n), dtype=torch.float32, device=DEV)
    st = kai.kai_fused_mmvq(w_dev.data_ptr(), O.Q4_K, n, k, m, act.data_ptr(), 0, out.data_ptr(), 0, n,
                            _stream())
    assert st == 0, kai.current_direct_error()
    torch.cuda.synchronize()
    ref = O.mul_mat(O.Q4_K, w.reshape(n, -1), k, O.prepare_swiglu(host(gu)), m)
    assert O.normwise_rel(out.cpu().numpy(), ref) <= TOL_F32


# ----------------------------------------------------------------- torch ops / apply()

def _layer(parts_np, k, dtype=torch.bfloat16):
    from kaillm_amd.linear import PackedGGUFLinear

    layer = torch.nn.Module()
    layer.gguf_compact = torch.nn.ModuleList([PackedGGUFLinear(to_dev(w), t, dtype) for t, w in parts_np])
    return layer


class _CountingLibrary:
    """The product library with a count of kai_fused_prepare calls."""

    def __init__(self, lib):
        self._lib, self.prepares = lib, 0

    def kai_fused_prepare(self, *args):
        self.prepares += 1
        return self._lib.kai_fused_prepare(*args)

    def __getattr__(self, name):
        return getattr(self._lib, name)


def test_apply_swiglu_small_and_large_batches(kai):
    from test_gpu_parity import TOL_BF16
    from kaillm_amd.linear import GGUFLinearMethod

    rng = np.random.default_rng(81)
    k = 1024
    parts_np = [(O.Q4_K, O.random_blocks(O.Q4_K, 256, k, rng))]
    layer, method = _layer(parts_np, k), GGUFLinearMethod()

    def act_fn(gu):
        return torch.nn.functional.silu(gu[..., :k]) * gu[..., k:]

    for m in (1, 5, 8, 12):
        print(f"apply_swiglu m={m}", flush=True)
        gu = to_dev(rng.standard_normal((1, m, 2 * k)).astype(np.float32)).to(torch.bfloat16)
        y = method.apply_swiglu(layer, gu, act_fn)
        assert y.shape == (1, m, 256) and y.dtype == torch.bfloat16
        if m <= 8:  # the producer path
            ref = O.mul_mat(O.Q4_K, parts_np[0][1], k, O.prepare_swiglu(host(gu.reshape(m, 2 * k))), m)
        else:       # act_fn, then the batched path
            ref = O.mmq_reference(O.Q4_K, parts_np[0][1], host(act_fn(gu).reshape(m, k)), 1)
        assert O.normwise_rel(y.float().reshape(m, -1).cpu().numpy(), ref) <= 2 * TOL_BF16


def test_apply_through_input_view_equals_the_copy(kai):
    from kaillm_amd.linear import GGUFLinearMethod

    rng = np.random.default_rng(82)
    a, b, s = 4, 8, 64
    k = a * b * s
    parts_np = [(O.Q6_K, O.random_blocks(O.Q6_K, 192, k, rng)), (O.Q4_K, O.random_blocks(O.Q4_K, 64, k, rng))]
    layer, method = _layer(parts_np, k), GGUFLinearMethod()
    layer._kai_input_gather = torch.arange(k, device=DEV).reshape(a, b, s).transpose(0, 1).reshape(k)
    layer._kai_input_view = (a, b, s)
    plain = _layer(parts_np, k)
    for m in (1, 3, 8, 16):
        print(f"apply view m={m}", flush=True)
        x = to_dev(rng.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16)
        got = method.apply(layer, x)
        want = GGUFLinearMethod().apply(plain, x[:, layer._kai_input_gather].contiguous())
        assert torch.equal(got, want)


def test_norm_prepare_stash_feeds_its_consumer(kai, monkeypatch):
    from test_gpu_parity import TOL_F32
    from kaillm_amd import native_fused
    from kaillm_amd.linear import GGUFLinearMethod

    rng = np.random.default_rng(83)
    m, k, eps = 3, 2048, 1e-6
    parts_np = [(O.Q4_K, O.random_blocks(O.Q4_K, 320, k, rng))]
    layer, method = _layer(parts_np, k, torch.float32), GGUFLinearMethod()
    producer = 12345
    layer._kai_act_producer = producer
    counting = _CountingLibrary(native_fused.library())
    monkeypatch.setattr(native_fused, "library", lambda: counting)
    monkeypatch.setattr(native_fused, "CONSUMER_OF", {})
    monkeypatch.setattr(native_fused, "STASH", {})
    method._fused(layer)
    assert native_fused.CONSUMER_OF == {layer._kai_fused.weights[0].data_ptr(): producer}

    x = to_dev(rng.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16)
    r = to_dev(rng.standard_normal((m, k)).astype(np.float32))
    w32 = to_dev((1 + 0.1 * rng.standard_normal(k)).astype(np.float32))
    y, r_out = native_fused.norm_prepare(producer, x, r, w32, eps)
    ref_act, ref_y, ref_r = O.norm_prepare(host(x), w32.cpu().numpy(), eps, r.cpu().numpy())
    assert np.array_equal(host(y), ref_y) and np.array_equal(r_out.cpu().numpy(), ref_r)
    out = method.apply(layer, y)
    assert counting.prepares == 0                      # the stashed activation was used
    ref = O.mul_mat(O.Q4_K, parts_np[0][1], k, ref_act, m)
    assert O.normwise_rel(out.cpu().numpy(), ref) <= TOL_F32
    method.apply(layer, y.clone())                     # another tensor: prepares its own
    assert counting.prepares == 1
    assert native_fused.norm_prepare(producer, x.float().to(torch.float16), None, w32, eps) is None  # F16 x
