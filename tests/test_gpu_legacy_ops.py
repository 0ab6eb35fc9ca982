"""The legacy GGUF op surface (kaillm_amd.ops) on the GPU.

ggml_dequantize replaces csrc/gguf/gguf_kernel.cu:87-102: bit-exact against the oracle's
dequantisation (gguf-py's formulas in fp32) rounded to the output type by numpy / torch.
ggml_mul_mat_vec_a8 / ggml_mul_mat_a8 (gguf_kernel.cu:104-290) and the fused_mul_mat_gguf
dispatch (quantization/linear.py:40-63) run on the fused kernels: within the path's
normwise bound of the oracle's FP64 result, plus the output type's rounding.
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


@pytest.mark.parametrize("qtype", O.WEIGHT_TYPES, ids=lambda t: O.NAMES[t])
@pytest.mark.parametrize("m", [1, 5, 8, 9, 40])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_mul_mat_a8_against_oracle(kai, qtype, m, dtype):
    from kaillm_amd.ops import ggml_mul_mat_a8, ggml_mul_mat_vec_a8

    print(f"mul_mat_a8 {O.NAMES[qtype]} m={m} {dtype}", flush=True)
    rng = np.random.default_rng(qtype * 100 + m)
    n, k = 200, 1024
    w = _weights(qtype, n, k, rng, "quantized")
    x = to_dev(rng.standard_normal((m, k)).astype(np.float32)).to(dtype)
    xh = x.cpu()
    xb, code = (xh.view(torch.int16).numpy().view(np.uint16), 1) if dtype == torch.bfloat16 else (xh.numpy(), None)
    ref = O.mul_mat(qtype, w, k, O.prepare(xb, dtype_code=code), m) if m <= 8 else O.mmq_reference(qtype, w, xb, code)
    op = ggml_mul_mat_vec_a8 if m <= 8 else ggml_mul_mat_a8
    y = op(to_dev(w), x, qtype, n)
    assert y.dtype == dtype and y.shape == (m, n)
    assert O.normwise_rel(y.float().cpu().numpy(), ref) <= OUT_TOL[dtype]


def test_fused_mul_mat_gguf_dispatch(kai):
    from kaillm_amd.ops import fused_mul_mat_gguf

    rng = np.random.default_rng(11)
    # unquantized weight: a plain matmul
    wf = torch.randn(64, 96, device=DEV, dtype=torch.float16)
    x = torch.randn(3, 96, device=DEV, dtype=torch.float16)
    assert torch.equal(fused_mul_mat_gguf(x, wf, 1), x @ wf.T)
    assert fused_mul_mat_gguf(x[:0], wf, 1).shape == (0, 64)
    # quantized, small and large batches through the fused kernels
    n, k = 160, 2048
    w = _weights(O.Q4_K, n, k, rng, "quantized")
    for m in (1, 2, 7, 33):
        print(f"fused_mul_mat_gguf Q4_K m={m}", flush=True)
        xm = to_dev(rng.standard_normal((m, k)).astype(np.float16))
        xn = xm.cpu().numpy()
        ref = O.mul_mat(O.Q4_K, w, k, O.prepare(xn), m) if m <= 8 else O.mmq_reference(O.Q4_K, w, xn)
        y = fused_mul_mat_gguf(xm, to_dev(w), O.Q4_K)
        assert y.dtype == torch.float16
        assert O.normwise_rel(y.float().cpu().numpy(), ref) <= OUT_TOL[torch.float16]
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
