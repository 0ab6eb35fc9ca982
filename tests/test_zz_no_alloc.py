"""kai_fused_mmq_run_noalloc: the batched entry without a scratch argument (its scratch is a
device array the library holds per GPU). Through the C ABI, its output equals
kai_fused_mmq_run's bit for bit on two calls in a row, the second smaller than the first,
and a call beyond its capacity fails with a message and writes nothing."""
import ctypes

import numpy as np
import pytest
import torch

import _oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _group(kai, mats):
    count = len(mats)
    types = (ctypes.c_int * count)(*[t for t, _ in mats])
    rows = (ctypes.c_int64 * count)(*[w.shape[0] for _, w in mats])
    ptrs = (ctypes.c_void_p * count)(*[w.data_ptr() for _, w in mats])
    return types, rows, ptrs, count


def _run(kai, mats, x, noalloc, bf16=False):
    m, k = x.shape
    types, rows, ptrs, count = _group(kai, mats)
    total = sum(w.shape[0] for _, w in mats)
    out = torch.full((m, total), float("nan"), dtype=torch.bfloat16 if bf16 else torch.float32, device=DEV)
    code = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[x.dtype]
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        st = kai.kai_fused_mmq_run_noalloc(ptrs, types, rows, count, x.data_ptr(), code, x.stride(0), k, m,
                                           out.data_ptr(), int(bf16), 0, 0, stream)
    else:
        size = kai.kai_fused_mmq_workspace(0, types, rows, count, k, m, int(not bf16))
        scratch = torch.empty(size, dtype=torch.uint8, device=DEV)
        st = kai.kai_fused_mmq_run(ptrs, types, rows, count, x.data_ptr(), code, x.stride(0), k, m,
                                   out.data_ptr(), int(bf16), 0, scratch.data_ptr(), size, 0, stream)
    assert st == 0, kai.current_direct_error()
    torch.cuda.synchronize()
    return out


def test_noalloc_equals_scratch_entry_on_two_calls(kai):
    rng = np.random.default_rng(2024)
    k = 5120
    mats = []
    for qtype, n in ((O.Q4_K, 1024), (O.Q6_K, 512), (O.Q2_K, 256)):
        w = O.random_blocks(qtype, n, k, rng)
        mats.append((qtype, torch.from_numpy(w).to(DEV)))
    for m, dtype, bf16 in ((80, torch.float16, False), (17, torch.bfloat16, True)):
        print(f"noalloc m={m} {dtype} bf16_out={bf16}", flush=True)
        x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(DEV).to(dtype)
        got = _run(kai, mats, x, noalloc=True, bf16=bf16)
        want = _run(kai, mats, x, noalloc=False, bf16=bf16)
        assert torch.equal(got, want)
        xs = x.view(torch.int16).cpu().numpy().view(np.uint16) if dtype == torch.bfloat16 else x.cpu().numpy()
        ref = np.concatenate([O.mmq_reference(t, w.cpu().numpy(), xs, 1 if dtype == torch.bfloat16 else None)
                              for t, w in mats], axis=1)
        assert O.normwise_rel(got.float().cpu().numpy(), ref) <= (2.0 ** -8 if bf16 else 1e-3)


def test_noalloc_small_m_routes_after_a_larger_call(kai):
    """Up to 16 rows the scratch holds the small-M image and, for matrices on the small-M GEMM,
    its partial sums: a group with one matrix on each 9..16-row kernel (Q6_K 5120 x 5120: 320
    row sets, the small-M GEMM and its reduction; Q4_K 7168 x 5120: 448 row sets, the
    persistent GEMM over the image), at 16 and then 9 rows, right after an 80-row call that
    filled the array with other bytes; bit for bit against kai_fused_mmq_run."""
    rng = np.random.default_rng(99)
    mats = []
    k = 5120
    for qtype, n in ((O.Q6_K, 5120), (O.Q4_K, 7168)):
        w = O.random_blocks(qtype, n, k, rng)
        mats.append((qtype, torch.from_numpy(w).to(DEV)))
    big = torch.from_numpy(rng.standard_normal((80, k)).astype(np.float16)).to(DEV)
    _run(kai, mats, big, noalloc=True)
    for m in (16, 9):
        print(f"noalloc small-M m={m}", flush=True)
        x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float16)).to(DEV)
        got = _run(kai, mats, x, noalloc=True)
        want = _run(kai, mats, x, noalloc=False)
        assert torch.equal(got, want)
        ref = np.concatenate([O.mmq_reference(t, w.cpu().numpy(), x.cpu().numpy(), threads=16)
                              for t, w in mats], axis=1)
        assert O.normwise_rel(got.cpu().numpy(), ref) <= 1e-3


def test_noalloc_refuses_beyond_capacity(kai):
    rng = np.random.default_rng(7)
    k, m = 17408, 2048   # 40 MiB of planes
    w = torch.from_numpy(O.random_blocks(O.Q6_K, 16, k, rng)).to(DEV)
    types, rows, ptrs, count = _group(kai, [(O.Q6_K, w)])
    x = torch.zeros((m, k), dtype=torch.float16, device=DEV)
    out = torch.full((m, 16), 7.0, device=DEV)
    st = kai.kai_fused_mmq_run_noalloc(ptrs, types, rows, count, x.data_ptr(), 2, k, k, m, out.data_ptr(), 0, 0,
                                       0, torch.cuda.current_stream().cuda_stream)
    assert st == -1 and b"16 MiB" in kai.current_direct_error()
    torch.cuda.synchronize()
    assert torch.all(out == 7.0)
