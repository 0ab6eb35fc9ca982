"""The legacy GGUF op surface (kaillm_amd.ops) on the GPU.

ggml_dequantize replaces csrc/gguf/gguf_kernel.cu:87-102: bit-exact against the oracle's
dequantisation (gguf-py's formulas in fp32) rounded to the output type by numpy / torch.
The legacy activation (kai_ggml_quantize_q8_1, quantize_q8_1 of gguf_kernel.cu:32-69) is
bit-exact against oracle_prepare_legacy, special blocks included. ggml_mul_mat_vec_a8 /
ggml_mul_mat_a8 (gguf_kernel.cu:104-290) are within the path's normwise bound (1e-3, plus
the output type's rounding) of oracle_mul_mat_legacy's FP64 result; the legacy forms differ
from the fused path's by 7e-3 (Q4_K on ggml_mul_mat_a8) and 1.6e-2 (Q4_0) on these inputs,
so the bound tells them apart. The fused_mul_mat_gguf dispatch (quantization/linear.py:40-63)
is checked against the legacy op it picks.
"""
import numpy as np
import pytest
import torch

import _oracle as O
from test_gpu_parity import DEV, TOL_F32, to_dev

pytestmark = pytest.mark.gpu

OUT_TOL = {torch.float32: TOL_F32, torch.bfloat16: 2.0 ** -8 + TOL_F32, torch.float16: 2.0 ** -11 + TOL_F32}


def _weights(qtype, n, k, rng, kind):
    if kind == "random":
        return O.random_blocks(qtype, n, k, rng)
    from kaillm_amd.formats import quantize
    return quantize(rng.normal(0, 0.02, (n, k)).astype(np.float32), qtype)


def _round(ref32, dtype):
    t = torch.from_numpy(ref32)
    return t if dtype == torch.float32 else t.to(dtype)


@pytest.mark.parametrize("qtype", O.WEIGHT_TYPES, ids=lambda t: O.NAMES[t])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("kind", ["random", "quantized"])
def test_dequantize_bit_exact(kai, qtype, dtype, kind):
    from kaillm_amd.ops import ggml_dequantize

    print(f"dequantize {O.NAMES[qtype]} {dtype} {kind}", flush=True)
    rng = np.random.default_rng(qtype * 31 + len(kind))
    n, k = 37, 1024
    w = _weights(qtype, n, k, rng, kind)
    got = ggml_dequantize(to_dev(w), qtype, n, k, dtype).cpu()
    want = _round(O.dequantize(qtype, w, k), dtype)
    assert got.dtype == dtype and got.shape == (n, k)
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    assert torch.equal(got.view(bits), want.view(bits))


def test_dequantize_defaults_and_empty(kai):
    from kaillm_amd.ops import ggml_dequantize

    rng = np.random.default_rng(5)
    w = O.random_blocks(O.Q8_0, 4, 64, rng)
    got = ggml_dequantize(to_dev(w), O.Q8_0, 4, 64, None)
    assert got.dtype == torch.float16
    assert ggml_dequantize(to_dev(w), O.Q8_0, 0, 64, torch.float32).shape == (0, 64)


def _host(x):
    """Device activation -> (numpy array the oracle reads, dtype code or None)."""
    xh = x.cpu()
    if x.dtype == torch.bfloat16:
        return xh.view(torch.int16).numpy().view(np.uint16), 1
    return xh.numpy(), None


def _special_rows(m, k, dtype, rng):
    """Random rows with the quantiser's corner cases planted in the first blocks."""
    x = rng.standard_normal((m, k)).astype(np.float32) * rng.choice([1e-3, 1.0, 30.0], size=(m, 1))
    if m >= 4 and k >= 64:
        x[0, :32] = -0.0                                   # sum -0, d 0
        x[1, :32] = 4000.0                                 # sum overflows fp16 to inf
        x[2, :32] = 0.0
        x[2, 0], x[2, 1] = 1e-6, -2e-7                     # d underflows fp16 to 0
        x[3, :32] = 0.0
        x[3, 0], x[3, 16], x[3, 1] = 4096.0, -4096.0, 2.0 ** -12   # butterfly grouping: sum 2^-12
        x[3, 32:64] = 0.0
        x[3, 32], x[3, 33], x[3, 48] = 4096.0, -4096.0, 2.0 ** -12  # ... and here 0
    return to_dev(x).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,k", [(1, 32), (5, 96), (33, 5120), (4, 40960)])
def test_legacy_quantize_bit_exact(kai, dtype, m, k):
    print(f"legacy quantize {dtype} m={m} k={k}", flush=True)
    rng = np.random.default_rng(m * 7 + k)
    wide = _special_rows(m, k + 64, dtype, rng)
    x = wide[:, :k]                                        # row stride k + 64
    code = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[dtype]
    act = torch.empty(kai.kai_fused_activation_bytes(m, k, 0), dtype=torch.uint8, device=DEV)
    st = kai.kai_ggml_quantize_q8_1(x.data_ptr(), code, m, k, wide.stride(0), act.data_ptr(),
                                    torch.cuda.current_stream().cuda_stream)
    assert st == 0, kai.current_direct_error()
    torch.cuda.synchronize()
    xh, hcode = _host(x.contiguous())
    want = O.prepare_legacy(xh, hcode)
    got = act.cpu().numpy()
    nb = m * (k // 32) * 36
    off = (nb + 255) // 256 * 256
    assert np.array_equal(got[:nb], want[:nb])
    assert np.array_equal(got[off:off + 4 * m], want[off:off + 4 * m])


@pytest.mark.parametrize("qtype", O.WEIGHT_TYPES, ids=lambda t: O.NAMES[t])
@pytest.mark.parametrize("m", [1, 5, 9, 17, 40])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("batched", [0, 1], ids=["vec_a8", "a8"])
def test_legacy_ops_against_oracle(kai, qtype, m, dtype, batched):
    from kaillm_amd.ops import ggml_mul_mat_a8, ggml_mul_mat_vec_a8

    if batched and qtype == O.IQ3_S:
        pytest.skip("no _C_gguf IQ3_S GEMM: test_legacy_iq3s_gemm_is_the_dequantising_route")
    print(f"legacy {'ggml_mul_mat_a8' if batched else 'ggml_mul_mat_vec_a8'} {O.NAMES[qtype]} m={m} {dtype}",
          flush=True)
    rng = np.random.default_rng(qtype * 100 + m + 7 * batched)
    n, k = 200, 1024
    w = _weights(qtype, n, k, rng, "quantized")
    x = to_dev(rng.standard_normal((m, k)).astype(np.float32)).to(dtype)
    xh, code = _host(x)
    ref = O.legacy_reference(qtype, w, xh, batched, code)
    op = ggml_mul_mat_a8 if batched else ggml_mul_mat_vec_a8
    y = op(to_dev(w), x, qtype, n)
    assert y.dtype == dtype and y.shape == (m, n)
    err = O.normwise_rel(y.float().cpu().numpy(), ref)
    print(f"  normwise rel err {err:.3e}")
    assert err <= OUT_TOL[dtype]


def test_legacy_gemm_shapes(kai):
    """Row counts that are not a multiple of four on the decode route (Q4_0) and the planes
    route (Q4_K); K above 32768 dequantises."""
    from kaillm_amd.ops import ggml_mul_mat_a8, ggml_mul_mat_vec_a8

    rng = np.random.default_rng(3)
    x = to_dev(rng.standard_normal((12, 256)).astype(np.float32))
    w = _weights(O.Q4_0, 66, 256, rng, "quantized")
    y = ggml_mul_mat_a8(to_dev(w), x, O.Q4_0, 66)
    assert O.normwise_rel(y.cpu().numpy(), O.legacy_reference(O.Q4_0, w, x.cpu().numpy(), 1)) <= TOL_F32
    w = _weights(O.Q4_K, 66, 256, rng, "quantized")
    y = ggml_mul_mat_a8(to_dev(w), x, O.Q4_K, 66)
    assert O.normwise_rel(y.cpu().numpy(), O.legacy_reference(O.Q4_K, w, x.cpu().numpy(), 1)) <= TOL_F32
    assert O.normwise_rel(ggml_mul_mat_vec_a8(to_dev(w), x, O.Q4_K, 66).cpu().numpy(),
                          O.legacy_reference(O.Q4_K, w, x.cpu().numpy(), 0)) <= TOL_F32
    kk = 33024
    w = _weights(O.Q8_0, 16, kk, rng, "quantized")
    xb = rng.standard_normal((2, kk)).astype(np.float32)
    y = ggml_mul_mat_vec_a8(to_dev(w), to_dev(xb), O.Q8_0, 16).cpu().numpy()
    assert O.normwise_rel(y, xb.astype(np.float64) @ O.dequantize(O.Q8_0, w, kk).astype(np.float64).T) <= 1e-5


@pytest.mark.parametrize("qtype", [O.Q4_K, O.Q6_K], ids=lambda t: O.NAMES[t])
def test_legacy_gemm_many_rows(kai, qtype):
    """ggml_mul_mat_a8 at 300 and 1030 activation rows: the legacy quantisation into the planes by
    a workgroup per whole row (from 256 rows), a row of zeros and rows of very different
    scales."""
    from kaillm_amd.ops import ggml_mul_mat_a8

    for m in (300, 1030):
        print(f"legacy a8 many rows {O.NAMES[qtype]} m={m}", flush=True)
        rng = np.random.default_rng(qtype + m)
        n, k = 68, 1024
        x = (rng.standard_normal((m, k)) * rng.uniform(1e-2, 1e2, (m, 1))).astype(np.float32)
        x[7] = 0.0
        w = _weights(qtype, n, k, rng, "random")
        y = ggml_mul_mat_a8(to_dev(w), to_dev(x), qtype, n).cpu().numpy()
        assert O.normwise_rel(y, O.legacy_reference(qtype, w, x, 1)) <= TOL_F32
        assert np.all(y[7] == 0.0)


# ggml_mul_mat_a8 on the planes route (Q4_K, Q8_0, Q6_K) with row counts that are not a
# multiple of four (an odd vocabulary, say), through every batched kernel: the small-M and
# persistent GEMMs (9 and 16 rows) and the tiled one (17 and 40).
@pytest.mark.parametrize("qtype", [O.Q4_K, O.Q8_0, O.Q6_K], ids=lambda t: O.NAMES[t])
@pytest.mark.parametrize("n", [1, 67, 4099])
@pytest.mark.parametrize("m", [9, 16, 17, 40])
def test_legacy_gemm_ragged_rows(kai, qtype, n, m):
    from kaillm_amd.ops import ggml_mul_mat_a8

    print(f"legacy a8 ragged rows {O.NAMES[qtype]} n={n} m={m}", flush=True)
    rng = np.random.default_rng(n + m + qtype)
    k = 512
    w = _weights(qtype, n, k, rng, "quantized")
    x = to_dev(rng.standard_normal((m, k)).astype(np.float32))
    y = ggml_mul_mat_a8(to_dev(w), x, qtype, n)
    assert y.shape == (m, n)
    err = O.normwise_rel(y.cpu().numpy(), O.legacy_reference(qtype, w, x.cpu().numpy(), 1))
    print(f"  normwise rel err {err:.3e}")
    assert err <= TOL_F32


def test_legacy_iq3s_gemm_is_the_dequantising_route(kai):
    """ops.py:200-208: no _C_gguf IQ3_S GEMM, so the op is x @ dequant(W).T (the reference runs
    its Triton GEMM of the same product)."""
    from kaillm_amd.ops import ggml_dequantize, ggml_mul_mat_a8

    rng = np.random.default_rng(9)
    n, k = 96, 512
    w = _weights(O.IQ3_S, n, k, rng, "quantized")
    for dtype, tol in ((torch.float32, 1e-5), (torch.bfloat16, 2.0 ** -7)):
        x = to_dev(rng.standard_normal((20, k)).astype(np.float32)).to(dtype)
        y = ggml_mul_mat_a8(to_dev(w), x, O.IQ3_S, n)
        assert torch.equal(y, x @ ggml_dequantize(to_dev(w), O.IQ3_S, n, k, dtype).T)
        dense = x.float().cpu().numpy().astype(np.float64) @ O.dequantize(O.IQ3_S, w, k).astype(np.float64).T
        assert O.normwise_rel(y.float().cpu().numpy(), dense) <= tol


def test_fused_mul_mat_gguf_dispatch(kai):
    from kaillm_amd.ops import fused_mul_mat_gguf

    rng = np.random.default_rng(11)
    # unquantized weight: a plain matmul
    wf = torch.randn(64, 96, device=DEV, dtype=torch.float16)
    x = torch.randn(3, 96, device=DEV, dtype=torch.float16)
    assert torch.equal(fused_mul_mat_gguf(x, wf, 1), x @ wf.T)
    assert fused_mul_mat_gguf(x[:0], wf, 1).shape == (0, 64)
    # quantized: the legacy ops at the reference's thresholds (160 rows: up to 6 on the GEMV)
    n, k = 160, 2048
    w = _weights(O.Q4_K, n, k, rng, "quantized")
    for m in (1, 6, 7, 33):
        print(f"fused_mul_mat_gguf Q4_K m={m}", flush=True)
        xm = to_dev(rng.standard_normal((m, k)).astype(np.float16))
        ref = O.legacy_reference(O.Q4_K, w, xm.cpu().numpy(), int(m > 6))
        y = fused_mul_mat_gguf(xm, to_dev(w), O.Q4_K)
        assert y.dtype == torch.float16
        assert O.normwise_rel(y.float().cpu().numpy(), ref) <= OUT_TOL[torch.float16]
    # IQ3_S above its threshold (16 rows here) is not an MMQ type: dequantise, then a matmul
    w = _weights(O.IQ3_S, 64, 512, rng, "quantized")
    xm = to_dev(rng.standard_normal((17, 512)).astype(np.float32))
    y = fused_mul_mat_gguf(xm, to_dev(w), O.IQ3_S).cpu().numpy()
    ref = xm.cpu().numpy().astype(np.float64) @ O.dequantize(O.IQ3_S, w, 512).astype(np.float64).T
    assert O.normwise_rel(y, ref) <= 1e-5
    # K beyond the fused path's 32768: dequantise, then a matmul (F32 here, so no rounding of x)
    kk = 33024
    w = _weights(O.Q6_K, 24, kk, rng, "quantized")
    xb = rng.standard_normal((3, kk)).astype(np.float32)
    print("fused_mul_mat_gguf Q6_K K=33024 (dequantize path)", flush=True)
    y = fused_mul_mat_gguf(to_dev(xb), to_dev(w), O.Q6_K).cpu().numpy()
    ref = xb.astype(np.float64) @ O.dequantize(O.Q6_K, w, kk).astype(np.float64).T
    assert O.normwise_rel(y, ref) <= 1e-5
    with pytest.raises(NotImplementedError):
        fused_mul_mat_gguf(x, torch.zeros(4, 18, dtype=torch.uint8, device=DEV), 3)
