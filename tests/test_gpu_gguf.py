"""GGUF ingestion on the GPU: kai_upload_rows moves a file's tensor bytes into HBM unchanged,
with row and block permutations applied while staging, and a model file's matrices loaded
this way drive the fused path (the reference reads through gguf_reader.py:116-390 and
permutes on the host, quantization/yaqa_linear.py:102-148)."""
import numpy as np
import pytest
import torch

import _oracle as O
from test_gpu_parity import DEV, TOL_BF16, to_dev

pytestmark = pytest.mark.gpu


def test_upload_unchanged_and_permuted(kai, tmp_path):
    from kaillm_amd import gguf

    rng = np.random.default_rng(21)
    big = rng.integers(0, 256, (4096, 320 * 34), dtype=np.uint8)   # 44.6 MB Q8_0: several staging rounds
    small = rng.integers(0, 256, (7, 3 * 144), dtype=np.uint8)
    path = tmp_path / "m.gguf"
    gguf.write_gguf(path, [("small", 12, (768, 7), small), ("big", 8, (10240, 4096), big)], alignment=64)
    r = gguf.GGUFReader(path)
    print("upload big unchanged", flush=True)
    got = gguf.upload(r, r.tensor("big"), DEV)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), torch.from_numpy(big))
    rows = torch.randperm(4096, generator=torch.Generator().manual_seed(1))[:3000]
    blocks = torch.randperm(320, generator=torch.Generator().manual_seed(2))
    print("upload big permuted", flush=True)
    got = gguf.upload(r, r.tensor("big"), DEV, rows, blocks)
    want = big[rows.numpy()].reshape(3000, 320, 34)[:, blocks.numpy()].reshape(3000, -1)
    assert torch.equal(got.cpu(), torch.from_numpy(np.ascontiguousarray(want)))
    got = gguf.upload(r, r.tensor("small"), DEV, torch.tensor([6, 6, 0]))
    assert torch.equal(got.cpu(), torch.from_numpy(small[[6, 6, 0]]))


def test_upload_rejects_bad_arguments(kai, tmp_path):
    from kaillm_amd import native

    lib = native.library()
    path = str(tmp_path / "none.gguf").encode()
    buf = torch.empty(64, dtype=torch.uint8, device=DEV)
    assert lib.kai_upload_rows(path, 0, 1, 64, None, 1, 0, None, buf.data_ptr(), 0) == -1
    assert b"Cannot open" in lib.current_direct_error()
    order = np.array([3], dtype=np.int64)
    assert lib.kai_upload_rows(path, 0, 2, 64, order.ctypes.data, 1, 0, None, buf.data_ptr(), 0) == -1
    assert b"out of range" in lib.current_direct_error()
    assert lib.kai_upload_rows(path, 0, 2, 64, None, 1, 48, order.ctypes.data, buf.data_ptr(), 0) == -1
    assert b"Invalid upload" in lib.current_direct_error()


def test_model_file_drives_the_fused_path(kai, tmp_path):
    """A Q4_K + Q6_K projection read from a GGUF file, with a row permutation, a
    block-moving column permutation on one matrix and a segment-transpose column
    permutation on another, gives the oracle's result on the permuted host weights."""
    from kaillm_amd import gguf
    from kaillm_amd.formats import quantize
    from kaillm_amd.linear import GGUFLinearMethod

    rng = np.random.default_rng(22)
    k = 2048
    wa = quantize(rng.normal(0, 0.02, (384, k)).astype(np.float32), O.Q4_K)
    wb = quantize(rng.normal(0, 0.02, (256, k)).astype(np.float32), O.Q6_K)
    path = tmp_path / "model.gguf"
    gguf.write_gguf(path, [("blk.0.attn_qkv.weight", O.Q4_K, (k, 384), wa), ("blk.0.attn_output.weight", O.Q6_K,
                                                                            (k, 256), wb)],
                    {"general.architecture": (gguf.STRING, "qwen35")})
    r = gguf.GGUFReader(path)
    method = GGUFLinearMethod()

    rows = torch.randperm(384, generator=torch.Generator().manual_seed(3))
    blocks = torch.randperm(k // 256, generator=torch.Generator().manual_seed(4))
    columns = torch.cat([torch.arange(256) + 256 * int(b) for b in blocks])
    part, gather, view = gguf.load_packed(r, "blk.0.attn_qkv.weight", torch.bfloat16, DEV, rows, columns)
    assert gather is None and view is None
    layer = torch.nn.Module()
    layer.gguf_compact = torch.nn.ModuleList([part])
    w_host = wa[rows.numpy()].reshape(384, k // 256, 144)[:, blocks.numpy()].reshape(384, -1)
    for m in (1, 4, 24):
        print(f"gguf-loaded Q4_K m={m}", flush=True)
        x = to_dev(rng.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16)
        y = method.apply(layer, x)
        xb = x.view(torch.int16).cpu().numpy().view(np.uint16)
        ref = O.mul_mat(O.Q4_K, np.ascontiguousarray(w_host), k, O.prepare(xb, dtype_code=1), m) if m <= 8 \
            else O.mmq_reference(O.Q4_K, np.ascontiguousarray(w_host), xb, 1)
        assert O.normwise_rel(y.float().cpu().numpy(), ref) <= 2 * TOL_BF16

    a, b, s = 4, 8, 64
    columns = torch.arange(k).view(b, a, s).transpose(0, 1).reshape(-1)  # inverse of the (a, b, s) transpose
    part, gather, view = gguf.load_packed(r, "blk.0.attn_output.weight", torch.bfloat16, DEV, None, columns)
    assert view == (a, b, s)
    layer = torch.nn.Module()
    layer.gguf_compact = torch.nn.ModuleList([part])
    layer._kai_input_gather, layer._kai_input_view = gather, view
    for m in (2, 12):
        print(f"gguf-loaded Q6_K through the input view m={m}", flush=True)
        x = to_dev(rng.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16)
        y = method.apply(layer, x)
        xs = x[:, gather].contiguous()   # the stored-column order of the activation
        xb = xs.view(torch.int16).cpu().numpy().view(np.uint16)
        ref = O.mul_mat(O.Q6_K, wb, k, O.prepare(xb, dtype_code=1), m) if m <= 8 \
            else O.mmq_reference(O.Q6_K, wb, xb, 1)
        assert O.normwise_rel(y.float().cpu().numpy(), ref) <= 2 * TOL_BF16
