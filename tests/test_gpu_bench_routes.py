"""Every route that bench.py times, at its full shape, against the CPU oracle.

The cases are generated from bench.py's own tables (C3 at C3_BATCHES, and every leg of
LEGS), so a leg added to the bench brings its parity test with it. Each case runs the call
the bench times, on the bench's data: weights quantized from seeded N(0, 0.02) (drawn on
the GPU, as bench.Runner does), activations fp16 N(0, 1); up to 8 rows kai_fused_prepare +
kai_fused_mmvq (decode arithmetic, O.mul_mat), above 8 rows kai_fused_mmq_run (batched
arithmetic, O.mmq_reference). The oracle checks a seeded sample of output columns that
includes the first and last four rows of the matrix.

Extra cases cover the one-row GEMV routes of the long-row matrices in their other modes:
the two-pass activation, and BF16 output into a merged projection's column slice.
"""
import numpy as np
import pytest
import torch

import _oracle as O
import bench
from test_gpu_fullsize import sample_cols
from test_gpu_parity import DEV, TOL_BF16, TOL_F32, gpu_mmq, gpu_mmvq, gpu_prepare, to_dev

pytestmark = pytest.mark.gpu

CASES = [(f"C3 {name} {O.NAMES[q]} {n}x{k} m{m}", q, n, k, m)
         for name, q, n, k in bench.C3 for m in bench.C3_BATCHES]
CASES += [(f"{cfg} {mname} {O.NAMES[q]} {n}x{k} m{m}", q, n, k, m)
          for cfg, mname, q, n, k, ms in bench.LEGS for m in ms]


def bench_weights(qtype, n, k, seed):
    """The bench's weights: N(0, 0.02) drawn on the GPU, quantized on the host."""
    from kaillm_amd.formats import quantize
    g = torch.Generator(device=DEV).manual_seed(seed)
    w32 = torch.randn((n, k), generator=g, device=DEV, dtype=torch.float32).mul_(0.02).cpu().numpy()
    return quantize(w32, qtype)


@pytest.mark.parametrize("name,qtype,n,k,m", CASES, ids=[c[0] for c in CASES])
def test_bench_route(kai, name, qtype, n, k, m):
    print(f"bench route {name}: {bench.kernel_name(qtype, m, n, k)}", flush=True)
    rng = np.random.default_rng(n + 3 * k + 7 * m + qtype)
    w = bench_weights(qtype, n, k, seed=n + k + qtype)
    x = rng.standard_normal((m, k), dtype=np.float32).astype(np.float16)
    w_dev, x_dev = to_dev(w), to_dev(x)
    cols = sample_cols(n, rng)
    if m <= 8:
        out = gpu_mmvq(kai, qtype, w_dev, n, k, gpu_prepare(kai, x_dev), m)
        ref = O.mul_mat(qtype, w[cols], k, O.prepare(x), m, threads=16)
    else:
        out = gpu_mmq(kai, [(qtype, w, w_dev)], x_dev)
        ref = O.mmq_reference(qtype, w[cols], x, threads=16)
    got = out[:, torch.from_numpy(cols).to(out.device)].cpu().numpy()
    del out
    assert not np.isnan(got).any()
    err = O.normwise_rel(got, ref)
    print(f"  normwise rel err {err:.3e}")
    assert err <= TOL_F32


# One-row GEMV of the long rows (K = 17408): the coalesced LDS-transpose stream for Q6_K
# (mmvq_kernel<Q6_K, 1, ..., G = 32>) and the IQ3_S stream, in two-pass mode and with BF16
# output into columns [37, 37 + n) of a merged [1, n + 50] output.
LONG_ROWS = [(O.Q6_K, 5120, 17408), (O.IQ3_S, 5120, 17408), (O.Q2_K, 5120, 17408)]


@pytest.mark.parametrize("qtype,n,k", LONG_ROWS, ids=[f"{O.NAMES[q]}-{n}x{k}" for q, n, k in LONG_ROWS])
def test_one_row_long_rows_two_pass_bf16_merged(kai, qtype, n, k):
    print(f"one-row long rows {O.NAMES[qtype]} {n}x{k}: two-pass, bf16 merged stride", flush=True)
    rng = np.random.default_rng(qtype + 17)
    w = bench_weights(qtype, n, k, seed=qtype + 5)
    x = rng.standard_normal((1, k), dtype=np.float32)
    w_dev, x_dev = to_dev(w), to_dev(x)
    cols = sample_cols(n, rng)
    for two_pass in (0, 1):
        act = gpu_prepare(kai, x_dev, two_pass)
        ref = O.mul_mat(qtype, w[cols], k, O.prepare(x, two_pass), 1, two_pass, threads=16)
        out = gpu_mmvq(kai, qtype, w_dev, n, k, act, 1, two_pass, bf16=True, stride=n + 50, offset=37)
        got = out.float().cpu().numpy()
        assert np.isnan(got[:, :37]).all() and np.isnan(got[:, 37 + n:]).all()  # neighbours untouched
        err16 = O.normwise_rel(got[:, 37:37 + n][:, cols], ref)
        out32 = gpu_mmvq(kai, qtype, w_dev, n, k, act, 1, two_pass).cpu().numpy()
        err32 = O.normwise_rel(out32[:, cols], ref)
        print(f"  two_pass={two_pass}: bf16 {err16:.3e}, f32 {err32:.3e}")
        assert err16 <= TOL_BF16 and err32 <= TOL_F32
