"""The apply() surface on the GPU: YAQAMixedLinearMethod building layer.yaqa_parts from a
GGUF file (yaqa_linear.py:150-405 of the reference), its per-part path, and the
non-compact GGUFLinearMethod.apply over a merged qweight with shards
(quantization/linear.py:365-407), each checked against the oracle: the fused path's
arithmetic for the compact parts, the legacy ops' for the non-compact layers."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import _oracle as O
from test_gpu_parity import DEV, TOL_BF16, to_dev

pytestmark = pytest.mark.gpu


def _ref(qtype, w, x_dev):
    """Oracle result of the fused path for x on device (decode up to 8 rows, batched above)."""
    m, k = x_dev.shape
    if x_dev.dtype == torch.bfloat16:
        xs, code = x_dev.view(torch.int16).cpu().numpy().view(np.uint16), 1
    else:
        xs, code = x_dev.cpu().numpy(), None
    if m <= 8:
        return O.mul_mat(qtype, w, k, O.prepare(xs, dtype_code=code), m)
    return O.mmq_reference(qtype, w, xs, code)


def _legacy_ref(qtype, w, x_dev, rows):
    """Oracle result of the non-compact dispatch (quantization/linear.py:40-63) for a matrix of
    `rows` rows: the legacy ggml_mul_mat_vec_a8 up to mmvq_safe rows, ggml_mul_mat_a8 above."""
    m = x_dev.shape[0]
    safe = (8 if rows > 5120 else 16) if qtype == O.IQ3_S else (2 if rows > 5120 else 6)
    if x_dev.dtype == torch.bfloat16:
        xs, code = x_dev.view(torch.int16).cpu().numpy().view(np.uint16), 1
    else:
        xs, code = x_dev.cpu().numpy(), None
    return O.legacy_reference(qtype, w, xs, int(m > safe), code)


def test_yaqa_mixed_method_from_a_gguf_file(kai, tmp_path):
    """gate and up from a GGUF file into one merged projection: create_weights with a row
    permutation on gate and a block-moving column permutation on both, then apply() at
    decode and batched sizes, plus bias."""
    from kaillm_amd import gguf
    from kaillm_amd.formats import quantize
    from kaillm_amd.linear import PackedGGUFLinear, YAQAMixedLinearMethod

    rng = np.random.default_rng(41)
    k, n_gate, n_up = 1024, 256, 128
    wg = quantize(rng.normal(0, 0.02, (n_gate, k)).astype(np.float32), O.Q4_K)
    wu = quantize(rng.normal(0, 0.02, (n_up, k)).astype(np.float32), O.Q6_K)
    path = tmp_path / "mlp.gguf"
    gguf.write_gguf(path, [("blk.0.ffn_gate.weight", O.Q4_K, (k, n_gate), wg),
                           ("blk.0.ffn_up.weight", O.Q6_K, (k, n_up), wu)])
    rows = torch.randperm(n_gate, generator=torch.Generator().manual_seed(1))
    blocks = torch.randperm(k // 256, generator=torch.Generator().manual_seed(2))
    columns = torch.cat([torch.arange(256) + 256 * int(b) for b in blocks])
    cfg = SimpleNamespace(yaqa_readers={str(path): gguf.GGUFReader(path)},
                          gguf_row_permutations={"blk.0.ffn_gate.weight": rows},
                          gguf_column_permutations={"blk.0.ffn_gate.weight": columns, "blk.0.ffn_up.weight": columns},
                          canonical_gguf_rounding=True, yaqa_consumed_names=set(), yaqa_consumed_tensors=set())
    parts = [("model.layers.0.mlp.gate_proj.weight", (str(path), "blk.0.ffn_gate.weight", None)),
             ("model.layers.0.mlp.up_proj.weight", (str(path), "blk.0.ffn_up.weight", None))]
    method = YAQAMixedLinearMethod(cfg, parts)
    layer = torch.nn.Module()
    method.create_weights(layer, k, [n_gate, n_up], k, n_gate + n_up, torch.bfloat16)
    method.process_weights_after_loading(layer)
    assert [type(p) for p in layer.yaqa_parts] == [PackedGGUFLinear, PackedGGUFLinear]
    assert all(p.role == "body" and p.canonical_rounding for p in layer.yaqa_parts)
    assert cfg.yaqa_consumed_tensors == {"blk.0.ffn_gate.weight", "blk.0.ffn_up.weight"}
    assert getattr(layer, "_kai_input_gather", None) is None   # block-moving: applied to the bytes
    wg_host = wg[rows.numpy()].reshape(n_gate, k // 256, 144)[:, blocks.numpy()].reshape(n_gate, -1)
    wu_host = wu.reshape(n_up, k // 256, 210)[:, blocks.numpy()].reshape(n_up, -1)
    bias = torch.randn(n_gate + n_up, device=DEV, dtype=torch.bfloat16)
    for m in (1, 5, 24):
        print(f"yaqa mixed apply m={m}", flush=True)
        x = to_dev(rng.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16)
        y = method.apply(layer, x)
        assert y.shape == (m, n_gate + n_up) and y.dtype == torch.bfloat16
        ref = np.concatenate([_ref(O.Q4_K, np.ascontiguousarray(wg_host), x),
                              _ref(O.Q6_K, np.ascontiguousarray(wu_host), x)], axis=1)
        assert O.normwise_rel(y.float().cpu().numpy(), ref) <= TOL_BF16
        assert torch.equal(method.apply(layer, x, bias), y + bias)


def test_yaqa_mixed_per_part_path(kai):
    """_apply_original runs each part on its own and concatenates when the parts do not form
    one fused projection (here one part is a dense module)."""
    from kaillm_amd.linear import PackedGGUFLinear, YAQAMixedLinearMethod

    rng = np.random.default_rng(42)
    k = 512
    w = O.random_blocks(O.Q4_K, 64, k, rng)
    dense = torch.nn.Linear(k, 32, bias=False).to(DEV)
    layer = torch.nn.Module()
    layer.yaqa_parts = torch.nn.ModuleList([PackedGGUFLinear(to_dev(w), O.Q4_K, torch.float32), dense])
    method = YAQAMixedLinearMethod(None, [])
    x = to_dev(rng.standard_normal((3, k)).astype(np.float32))
    with torch.no_grad():
        y = method.apply(layer, x)
    assert layer._kai_fused is False
    assert O.normwise_rel(y[:, :64].cpu().numpy(), _ref(O.Q4_K, w, x)) <= 1e-3
    with torch.no_grad():
        assert torch.allclose(y[:, 64:], dense(x), rtol=1e-5, atol=1e-5)


def _merged_qweight(shards):
    """A merged qweight as the reference's loader pads it (linear.py:291-333): shard rows
    stacked, each row padded to the widest shard's bytes."""
    width = max(w.shape[1] for _, _, w in shards)
    total = sum(w.shape[0] for _, _, w in shards)
    data = np.zeros((total, width), dtype=np.uint8)
    offsets, start = {}, 0
    for sid, _, w in shards:
        data[start:start + w.shape[0], :w.shape[1]] = w
        offsets[sid] = (start, start + w.shape[0], w.shape[1])
        start += w.shape[0]
    return data, offsets


@pytest.mark.parametrize("mixed", [False, True], ids=["one-type", "mixed-types"])
@pytest.mark.parametrize("m", [1, 6, 20])
def test_gguf_linear_method_non_compact_shards(kai, mixed, m):
    """layer.qweight holding q|k|v shards: one GGUF type runs as one product over the merged
    tensor, mixed types run per shard on their slices (linear.py:365-407), bias added in place."""
    from kaillm_amd.formats import quantize
    from kaillm_amd.linear import GGUFLinearMethod

    print(f"non-compact shards mixed={mixed} m={m}", flush=True)
    rng = np.random.default_rng(43 + m)
    k = 512
    kinds = {"q": O.Q4_K, "k": O.Q6_K if mixed else O.Q4_K, "v": O.Q8_0 if mixed else O.Q4_K}
    sizes = {"q": 128, "k": 64, "v": 64}
    shards = [(s, kinds[s], quantize(rng.normal(0, 0.02, (sizes[s], k)).astype(np.float32), kinds[s]))
              for s in ("q", "k", "v")]
    data, offsets = _merged_qweight(shards)
    qweight = to_dev(data)
    qweight.shard_id = ["v", "q", "k"]            # any order naming q: run as q, k, v
    qweight.shard_offset_map = offsets
    layer = SimpleNamespace(qweight=qweight, qweight_type=SimpleNamespace(
        weight_type=O.Q4_K, shard_weight_type={s: kinds[s] for s in ("k", "v")}))
    x = to_dev(rng.standard_normal((m, k)).astype(np.float32)).to(torch.float16)
    bias = torch.randn(256, device=DEV, dtype=torch.float16)
    y = GGUFLinearMethod().apply(layer, x)
    assert y.shape == (m, 256) and y.dtype == torch.float16
    ref = np.concatenate([_legacy_ref(t, w, x, 256 if not mixed else w.shape[0]) for _, t, w in shards], axis=1)
    assert O.normwise_rel(y.float().cpu().numpy(), ref) <= 2.0 ** -11 + 1e-3   # fp16 output rounding
    assert torch.equal(GGUFLinearMethod().apply(layer, x, bias), y + bias)


def test_gguf_linear_method_unsharded_qweight(kai):
    from kaillm_amd.linear import GGUFLinearMethod

    rng = np.random.default_rng(44)
    w = O.random_blocks(O.Q2_K, 96, 768, rng)
    qweight = to_dev(w)
    layer = SimpleNamespace(qweight=qweight, qweight_type=SimpleNamespace(weight_type=O.Q2_K, shard_weight_type={}))
    x = to_dev(rng.standard_normal((4, 768)).astype(np.float32))
    y = GGUFLinearMethod().apply(layer, x)
    assert y.dtype == torch.float32
    assert O.normwise_rel(y.cpu().numpy(), _legacy_ref(O.Q2_K, w, x, 96)) <= 1e-3


@pytest.mark.parametrize("m", [1, 5, 12, 40])
def test_packed_linear_forward_bias_and_fp32_output(kai, m):
    """PackedGGUFLinear(x, bias, output_dtype=torch.float32), the vocabulary role's FP32
    logits (compact.py:364-407): the fused result in FP32 plus the bias, and in the layer
    dtype by default."""
    from kaillm_amd.linear import PackedGGUFLinear

    print(f"PackedGGUFLinear.forward bias / fp32 m={m}", flush=True)
    rng = np.random.default_rng(900 + m)
    n, k = 136, 768
    w = O.random_blocks(O.Q6_K, n, k, rng)
    p = PackedGGUFLinear(to_dev(w), O.Q6_K, torch.bfloat16, role="vocabulary")
    x_dev = to_dev(rng.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16)
    ref = _ref(O.Q6_K, w, x_dev)
    bias = torch.randn(n, device=DEV, dtype=torch.float32)
    y32 = p(x_dev.reshape(1, m, k), bias, output_dtype=torch.float32)
    assert y32.shape == (1, m, n) and y32.dtype == torch.float32
    assert O.normwise_rel((y32 - bias).reshape(m, n).cpu().numpy(), ref) <= 1e-3
    y16 = p(x_dev)
    assert y16.dtype == torch.bfloat16 and y16.shape == (m, n)
    assert O.normwise_rel(y16.float().cpu().numpy(), ref) <= TOL_BF16
