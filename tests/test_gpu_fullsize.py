"""Parity at BASELINE.json's full shapes, through the C ABI.

The GPU runs every product at its real size; the CPU oracle checks a seeded sample of
output columns (weight rows), chosen to include the first and last rows of the matrix,
so its cost stays bounded. Also covers the GEMV variants that only large matrices reach
(two row sets per wave, from 8192 row sets on).
"""
import numpy as np
import pytest
import torch

import _oracle as O
from test_gpu_parity import TOL_F32, gpu_mmq, gpu_mmvq, gpu_prepare, to_dev

pytestmark = pytest.mark.gpu


def sample_cols(n, rng, count=64):
    edge = list(range(4)) + list(range(n - 4, n))
    return np.unique(np.concatenate([edge, rng.choice(n, size=min(count, n), replace=False)]))


def quantized(qtype, n, k, rng):
    from kaillm_amd.formats import quantize
    return quantize((rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)), qtype)


# kai_fused_mmvq at 34816 x 5120: the GEMV's two row sets per wave for Q4_K at 1-3 rows and
# the other formats at 3-4 rows; above the GEMV's rows on this matrix (Q4_K at 4, Q2_K at 3)
# the persistent paired GEMM.
TWO_SETS = [(O.Q4_K, 2), (O.Q4_K, 3), (O.Q4_K, 4), (O.Q2_K, 3), (O.IQ3_S, 3), (O.IQ3_S, 4),
            (O.Q4_0, 3), (O.Q4_0, 4), (O.Q8_0, 3), (O.Q8_0, 4), (O.Q6_K, 3), (O.Q6_K, 4)]


@pytest.mark.parametrize("qtype,m", TWO_SETS, ids=[f"{O.NAMES[t]}-m{m}" for t, m in TWO_SETS])
def test_gemv_two_row_sets(kai, qtype, m):
    n, k = 34816, 5120
    print(f"gemv two row sets {O.NAMES[qtype]} {n}x{k} m={m}", flush=True)
    rng = np.random.default_rng(qtype * 10 + m)
    w = O.random_blocks(qtype, n, k, rng)
    x = rng.standard_normal((m, k), dtype=np.float32).astype(np.float16)
    out = gpu_mmvq(kai, qtype, to_dev(w), n, k, gpu_prepare(kai, to_dev(x)), m)
    cols = sample_cols(n, rng)
    ref = O.mul_mat(qtype, w[cols], k, O.prepare(x), m, threads=16)
    err = O.normwise_rel(out[:, cols].cpu().numpy(), ref)
    print(f"  normwise rel err {err:.3e}")
    assert err <= TOL_F32


# GEMV with K split (waves sharing each row) on matrices of few rows (kai_mmvq.cuh
# gemv_k_split: 2 or 4 parts): Q2_K at one and two rows; Q4_K, Q4_0 and Q8_0 at one row, and
# Q4_0 and Q8_0 at two rows on rows of at most 2048 values; the other formats at three and four;
# Q4_0 at five to eight rows on matrices of fewer 16-row sets than CUs.
K_SPLIT = [(O.Q2_K, 5120, 17408, 1), (O.Q2_K, 5120, 17408, 2), (O.Q6_K, 5120, 6144, 3), (O.Q6_K, 5120, 6144, 4),
           (O.IQ3_S, 5120, 17408, 3), (O.Q4_0, 2048, 8192, 4), (O.Q8_0, 2048, 2048, 3), (O.Q4_K, 7168, 5120, 4),
           (O.Q4_K, 7168, 5120, 1), (O.Q4_0, 2048, 8192, 1), (O.Q4_0, 3072, 2048, 2), (O.Q8_0, 2048, 2048, 1),
           (O.Q8_0, 2048, 2048, 2), (O.Q4_0, 2048, 8192, 8), (O.Q4_0, 3072, 2048, 5), (O.Q4_0, 3072, 2048, 7)]


@pytest.mark.parametrize("qtype,n,k,m", K_SPLIT, ids=[f"{O.NAMES[t]}-{n}x{k}-m{m}" for t, n, k, m in K_SPLIT])
def test_gemv_k_split(kai, qtype, n, k, m):
    print(f"gemv k split {O.NAMES[qtype]} {n}x{k} m={m}", flush=True)
    rng = np.random.default_rng(qtype * 100 + m)
    w = O.random_blocks(qtype, n, k, rng)
    x = rng.standard_normal((m, k), dtype=np.float32).astype(np.float16)
    out = gpu_mmvq(kai, qtype, to_dev(w), n, k, gpu_prepare(kai, to_dev(x)), m)
    cols = sample_cols(n, rng)
    ref = O.mul_mat(qtype, w[cols], k, O.prepare(x), m, threads=16)
    err = O.normwise_rel(out[:, cols].cpu().numpy(), ref)
    print(f"  normwise rel err {err:.3e}")
    assert err <= TOL_F32


# C2 (LFM-like Q4_0 decode) qkv at every batch, checked in full.
@pytest.mark.parametrize("m", [1, 2, 4, 8])
def test_c2_qkv_decode(kai, m):
    n, k = 3072, 2048
    print(f"C2 Q4_0 qkv m={m}", flush=True)
    rng = np.random.default_rng(300 + m)
    w = quantized(O.Q4_0, n, k, rng)
    x = rng.standard_normal((m, k), dtype=np.float32).astype(np.float16)
    out = gpu_mmvq(kai, O.Q4_0, to_dev(w), n, k, gpu_prepare(kai, to_dev(x)), m)
    ref = O.mul_mat(O.Q4_0, w, k, O.prepare(x), m, threads=16)
    assert O.normwise_rel(out.cpu().numpy(), ref) <= TOL_F32


# The batched path (kai_fused_mmq_run) at every BASELINE shape above 8 rows, like every
# other leg the bench times, is in test_gpu_bench_routes.py (cases generated from bench.py).
