"""GGUF ingestion on the CPU: the reader against hand-assembled known-answer files, the
writer byte for byte against the same bytes, error handling, and the stored-tensor
permutation logic (quantization/yaqa_linear.py:102-148 of the reference).

The known-answer bytes are assembled here field by field from the GGUF v3 layout (magic,
version, counts, key-value records, tensor-info records, aligned data), independently of
kaillm_amd.gguf; no GGUF file or gguf package exists in this environment to compare with.
"""
import struct

import numpy as np
import pytest
import torch

from kaillm_amd import gguf


def _s(text):
    b = text.encode()
    return struct.pack("<Q", len(b)) + b


def known_answer_file(alignment=64):
    rng = np.random.default_rng(1)
    q4k = rng.integers(0, 256, (3, 2 * 144), dtype=np.uint8)        # 3 rows of 512 Q4_K values
    norm = np.arange(5, dtype=np.float32) - 2.5
    bf = np.array([0x3F80, 0xC000, 0x0000, 0x7F80], dtype=np.uint16)  # BF16 [2, 2]
    kv = b"".join([
        _s("general.architecture") + struct.pack("<I", 8) + _s("qwen35"),
        _s("general.alignment") + struct.pack("<I", 4) + struct.pack("<I", alignment),
        _s("tokenizer.ggml.tokens") + struct.pack("<IIQ", 9, 8, 2) + _s("a") + _s("bc"),
        _s("qwen35.rope.dims") + struct.pack("<IIQ", 9, 5, 3) + struct.pack("<3i", 16, -24, 24),
        _s("general.use_bias") + struct.pack("<I", 7) + b"\x01",
        _s("qwen35.eps") + struct.pack("<I", 6) + struct.pack("<f", 1e-6),
    ])
    q4k_bytes = q4k.nbytes                                     # 864 -> next tensor at 896
    norm_off = -(-q4k_bytes // alignment) * alignment
    bf_off = norm_off + -(-norm.nbytes // alignment) * alignment
    infos = b"".join([
        _s("blk.0.ffn_down.weight") + struct.pack("<I2QIQ", 2, 512, 3, 12, 0),
        _s("output_norm.weight") + struct.pack("<IQIQ", 1, 5, 0, norm_off),
        _s("rope_freqs") + struct.pack("<I2QIQ", 2, 2, 2, 30, bf_off),
    ])
    head = struct.pack("<IIQQ", 0x46554747, 3, 3, 6) + kv + infos
    data_start = -(-len(head) // alignment) * alignment
    body = bytearray(head + b"\0" * (data_start - len(head)))
    body += q4k.tobytes() + b"\0" * (norm_off - q4k_bytes)
    body += norm.tobytes() + b"\0" * (bf_off - norm_off - norm.nbytes)
    body += bf.tobytes() + b"\0" * (-bf.nbytes % alignment)
    return bytes(body), data_start, (q4k, norm, bf), (norm_off, bf_off)


def test_reader_known_answer(tmp_path):
    raw, data_start, (q4k, norm, bf), (norm_off, bf_off) = known_answer_file()
    path = tmp_path / "ka.gguf"
    path.write_bytes(raw)
    r = gguf.GGUFReader(path)
    assert r.version == 3 and r.alignment == 64 and r.data_offset == data_start
    assert list(r.fields) == ["general.architecture", "general.alignment", "tokenizer.ggml.tokens",
                              "qwen35.rope.dims", "general.use_bias", "qwen35.eps"]
    assert r.fields["general.architecture"].contents() == "qwen35"
    assert r.fields["general.alignment"].contents() == 64
    assert r.fields["tokenizer.ggml.tokens"].contents() == ["a", "bc"]
    assert r.fields["tokenizer.ggml.tokens"].contents(1) == "bc"
    assert r.fields["qwen35.rope.dims"].contents() == [16, -24, 24]
    assert r.fields["qwen35.rope.dims"].types == [gguf.ARRAY, gguf.INT32]
    assert r.fields["general.use_bias"].contents() is True
    assert r.fields["qwen35.eps"].contents() == pytest.approx(1e-6)
    t0, t1, t2 = r.tensors
    assert (t0.name, t0.tensor_type, t0.shape.tolist(), t0.n_elements, t0.n_bytes) == \
        ("blk.0.ffn_down.weight", 12, [512, 3], 1536, 864)
    assert t0.data_offset == data_start and t0.data.shape == (3, 288) and t0.data.dtype == np.uint8
    assert np.array_equal(t0.data, q4k)
    assert t1.data_offset == data_start + norm_off and np.array_equal(t1.data, norm)
    assert t2.data_offset == data_start + bf_off and t2.data.dtype == np.uint16
    assert np.array_equal(t2.data, bf.reshape(2, 2))
    assert r.tensor("output_norm.weight").name == "output_norm.weight"
    with pytest.raises(KeyError):
        r.tensor("missing")


def test_writer_reproduces_the_known_answer(tmp_path):
    raw, _, (q4k, norm, bf), _ = known_answer_file()
    path = tmp_path / "w.gguf"
    meta = {
        "general.architecture": (gguf.STRING, "qwen35"),
        "general.alignment": (gguf.UINT32, 64),
        "tokenizer.ggml.tokens": (gguf.ARRAY, (gguf.STRING, ["a", "bc"])),
        "qwen35.rope.dims": (gguf.ARRAY, (gguf.INT32, [16, -24, 24])),
        "general.use_bias": (gguf.BOOL, 1),
        "qwen35.eps": (gguf.FLOAT32, 1e-6),
    }
    gguf.write_gguf(path, [("blk.0.ffn_down.weight", 12, (512, 3), q4k), ("output_norm.weight", 0, (5,), norm),
                           ("rope_freqs", 30, (2, 2), bf)], meta, alignment=64)
    assert path.read_bytes() == raw


def test_default_alignment_and_version_2(tmp_path):
    rng = np.random.default_rng(2)
    w = rng.integers(0, 256, (4, 34), dtype=np.uint8)          # 4 rows of 32 Q8_0 values
    path = tmp_path / "v2.gguf"
    gguf.write_gguf(path, [("a", 8, (32, 4), w), ("b", 8, (32, 4), w[::-1].copy())], version=2)
    r = gguf.GGUFReader(path)
    assert r.version == 2 and r.alignment == 32 and r.data_offset % 32 == 0
    assert r.tensors[1].data_offset - r.tensors[0].data_offset == 160  # 136 bytes padded to 32
    assert np.array_equal(r.tensors[1].data, w[::-1])


@pytest.mark.parametrize("mutate,message", [
    (lambda b: b"GGUX" + b[4:], "magic"),
    (lambda b: b[:4] + struct.pack("<I", 4) + b[8:], "version"),
    (lambda b: b[:4] + struct.pack(">I", 3) + b[8:], "Big-endian"),
    (lambda b: b[:200], "truncated"),
])
def test_reader_rejects_bad_files(tmp_path, mutate, message):
    raw, *_ = known_answer_file()
    path = tmp_path / "bad.gguf"
    path.write_bytes(mutate(raw))
    with pytest.raises(ValueError, match=message):
        gguf.GGUFReader(path)


def test_reader_rejects_duplicates_and_overruns(tmp_path):
    w = np.zeros((2, 34), dtype=np.uint8)
    path = tmp_path / "dup.gguf"
    gguf.write_gguf(path, [("x", 8, (32, 2), w), ("x", 8, (32, 2), w)])
    with pytest.raises(ValueError, match="duplicated"):
        gguf.GGUFReader(path)
    gguf.write_gguf(path, [("x", 8, (32, 2), w)])
    raw = path.read_bytes()
    path.write_bytes(raw[:-40])
    with pytest.raises(ValueError, match="past the end"):
        gguf.GGUFReader(path)


# ----------------------------------------------------------------- stored-tensor permutations

def test_permute_stored_rows_and_block_columns():
    rng = np.random.default_rng(3)
    n, k, bb = 5, 1024, 144
    data = torch.from_numpy(rng.integers(0, 256, (n, k // 256 * bb), dtype=np.uint8))
    rows = torch.tensor([4, 0, 3, 1, 2])
    blocks = [2, 0, 3, 1]
    columns = torch.cat([torch.arange(256) + 256 * b for b in blocks])
    out, gather = gguf.permute_stored(data, 12, rows, columns)
    want = data.numpy()[rows.numpy()].reshape(n, 4, bb)[:, blocks].reshape(n, -1)
    assert gather is None and np.array_equal(out.numpy(), want)
    assert gguf.block_order(columns, 256).tolist() == blocks


def test_permute_stored_other_columns_give_the_inverse_gather():
    k = 512
    columns = torch.randperm(k, generator=torch.Generator().manual_seed(4))
    data = torch.zeros((2, k // 256 * 144), dtype=torch.uint8)
    out, gather = gguf.permute_stored(data, 12, None, columns)
    assert out is data
    x = torch.randn(3, k, dtype=torch.float64)
    w = torch.randn(2, k, dtype=torch.float64)
    # the permuted layer W[:, columns] on x equals the stored W on x gathered
    assert torch.allclose(x @ w[:, columns].T, x.index_select(-1, gather) @ w.T)
    dense = torch.randn(2, k)
    out, gather = gguf.permute_stored(dense, 0, None, columns)
    assert gather is None and torch.equal(out, dense[:, columns])


@pytest.mark.parametrize("a,b,s", [(4, 8, 64), (2, 3, 32), (16, 2, 128)])
def test_transpose_view_detects_segment_transposes(a, b, s):
    n = a * b * s
    gather = torch.arange(n).view(a, b, s).transpose(0, 1).reshape(-1)
    assert gguf.transpose_view(gather) == (a, b, s)
    assert gguf.transpose_view(torch.arange(n)) is None
    broken = gather.clone()
    broken[[5, 6]] = broken[[6, 5]]
    assert gguf.transpose_view(broken) is None
