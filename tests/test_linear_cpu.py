"""The Python boundary without a GPU: PackedGGUFLinear's constructor rules and keyword
arguments (compact.py:201-250 of the reference), prepare() returning None when the
library is absent (native_fused.py:350-352), the environment switches, and the op schemas."""
from types import SimpleNamespace

import pytest
import torch

import _oracle as O


def _bytes(qtype, n, k):
    qk, bb = O.BLOCK[qtype]
    return torch.zeros((n, k // qk * bb), dtype=torch.uint8)


def test_packed_linear_keywords_and_shape():
    from kaillm_amd.linear import PackedGGUFLinear

    p = PackedGGUFLinear(_bytes(O.Q4_K, 8, 512), O.Q4_K, torch.bfloat16, canonical_rounding=True, role="body")
    assert p.shape == (8, 512) and p.is_quantized and p.role == "body" and p.canonical_rounding
    assert p.weight.dtype == torch.uint8 and p.weight.is_contiguous()
    q = PackedGGUFLinear(_bytes(O.Q8_0, 3, 64), O.Q8_0, torch.float16)
    assert q.role is None and not q.canonical_rounding and q.shape == (3, 64)


@pytest.mark.parametrize("kwargs,message", [
    (dict(role="head"), "Unknown GGUF matrix role"),
    (dict(dtype=torch.int8), "FP16, BF16, or FP32"),
    (dict(weight_type=3), "Unsupported compact GGUF type"),
    (dict(data=torch.zeros((2, 145), dtype=torch.uint8)), "whole number of wire blocks"),
    (dict(data=torch.zeros((2, 144), dtype=torch.int16)), "uint8 wire bytes"),
    (dict(data=torch.zeros(144, dtype=torch.uint8)), "two-dimensional"),
])
def test_packed_linear_rejects(kwargs, message):
    from kaillm_amd.linear import PackedGGUFLinear

    args = dict(data=_bytes(O.Q4_K, 2, 256), weight_type=O.Q4_K, dtype=torch.bfloat16)
    role = kwargs.pop("role", None)
    args.update(kwargs)
    with pytest.raises(ValueError, match=message):
        PackedGGUFLinear(args["data"], args["weight_type"], args["dtype"], role=role)


def test_prepare_returns_none_without_the_library(monkeypatch, tmp_path):
    from kaillm_amd import native, native_fused

    part = SimpleNamespace(weight=torch.zeros((4, 144), dtype=torch.uint8), weight_type=O.Q4_K, shape=(4, 256),
                           dtype=torch.bfloat16, is_quantized=True)
    monkeypatch.setenv(native.LIBRARY_ENV, str(tmp_path / "absent.so"))
    assert native_fused.library() is None
    assert native_fused.prepare([part]) is None
    assert not native_fused.ext_available()
    with pytest.raises(RuntimeError, match="missing"):
        native_fused.fused_mmvq(torch.zeros((1, 256)), [part.weight], [O.Q4_K], [4], 0, True)


def test_prepare_declines_ineligible_parts_and_disabled_mode(monkeypatch):
    from kaillm_amd import native_fused

    cpu_part = SimpleNamespace(weight=torch.zeros((4, 144), dtype=torch.uint8), weight_type=O.Q4_K, shape=(4, 256),
                               dtype=torch.bfloat16, is_quantized=True)
    assert native_fused.prepare([cpu_part]) is None      # not a device tensor
    assert native_fused.prepare([]) is None
    monkeypatch.setenv(native_fused.ENV, "0")
    assert native_fused.mode() == 0 and native_fused.prepare([cpu_part]) is None
    monkeypatch.setenv(native_fused.ENV, "3")
    with pytest.raises(ValueError):
        native_fused.mode()
    monkeypatch.setenv(native_fused.MMQ_ENV, "0")
    assert native_fused.mmq_mode() is False


def test_op_schemas_are_registered():
    from kaillm_amd import native_fused, ops  # noqa: F401

    for name in ("fused_mmvq", "fused_mmq", "fused_mmvq_view", "fused_mmvq_swiglu", "ggml_dequantize",
                 "ggml_mul_mat_vec_a8", "ggml_mul_mat_a8", "fused_mul_mat_gguf"):
        assert hasattr(torch.ops.kaillm, name), name
    schema = str(torch.ops.kaillm.fused_mmvq.default._schema)
    # torch.library.custom_op types `int` arguments as SymInt, as for the reference's ops
    assert "(Tensor x, Tensor[] weights, SymInt[] types, SymInt[] rows_out, SymInt two_pass, bool out_f32)" in schema
    assert "SymInt a, SymInt b, SymInt s, bool out_f32" in str(torch.ops.kaillm.fused_mmvq_view.default._schema)


def test_packed_linear_forward_checks_arguments():
    """forward(x, bias=None, *, output_dtype=None) checks width, dtype/device and the output
    dtype before running (compact.py:364-394); on the CPU the fused path then refuses."""
    import inspect

    from kaillm_amd.linear import PackedGGUFLinear

    p = PackedGGUFLinear(_bytes(O.Q4_K, 8, 512), O.Q4_K, torch.bfloat16)
    sig = inspect.signature(p.forward)
    assert list(sig.parameters) == ["x", "bias", "output_dtype"]
    assert sig.parameters["output_dtype"].kind is inspect.Parameter.KEYWORD_ONLY
    with pytest.raises(ValueError, match="width does not match"):
        p(torch.zeros((2, 256), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="share dtype and device"):
        p(torch.zeros((2, 512), dtype=torch.float16))
    with pytest.raises(ValueError, match="output dtype must match activations or FP32"):
        p(torch.zeros((2, 512), dtype=torch.bfloat16), output_dtype=torch.float16)
    with pytest.raises(RuntimeError, match="fused GGUF path cannot run"):
        p(torch.zeros((2, 512), dtype=torch.bfloat16), torch.zeros(8, dtype=torch.bfloat16),
          output_dtype=torch.float32)
