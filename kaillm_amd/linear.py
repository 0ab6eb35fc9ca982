"""The quantized-linear ``apply()`` surface over packed GGUF wire bytes.

Interface of the reference's plugin, built on the fused projection of this package:

* ``PackedGGUFLinear(data, weight_type, dtype, *, canonical_rounding=False, role=None)``
  (``quantization/compact.py:189-315``): one original GGUF matrix as its unchanged wire
  bytes ``uint8 [N, K/qk*bytes]`` on the GPU, with ``weight``, ``weight_type``, ``dtype``,
  ``shape``, ``is_quantized``, ``role`` and ``canonical_rounding``. Unlike the reference
  (``compact.py:235-238``) it takes ROCm tensors. ``canonical_rounding`` selects the
  reference's dense-reconstruction backends, which are not on the fused path; it is kept
  for the callers that pass it.
* ``GGUFLinearMethod.apply(layer, x, bias)`` (``quantization/linear.py:341-407``): a layer
  with ``gguf_compact`` parts runs them as one fused projection; a layer with a merged
  ``qweight`` (shards of one or several GGUF types, ``shard_id`` / ``shard_offset_map`` /
  ``qweight_type.shard_weight_type``) runs ``fused_mul_mat_gguf`` per type.
* ``YAQAMixedLinearMethod`` (``quantization/yaqa_linear.py:150-405``): ``create_weights``
  loads a projection's GGUF sources into ``layer.yaqa_parts`` (permutations applied while
  uploading, the input gather / view recorded); ``apply`` applies the input gather, then
  ``_apply_original``: the fused projection when it takes the input, else each part on its
  own and the outputs concatenated.
* ``apply_swiglu(layer, gate_up, act_fn)`` on both methods: up to 8 rows prepare the down
  projection's activation straight from ``gate_up``.

When the fused path cannot run an input, a part raises: this package has no other kernels.
"""
import os

import torch

from . import native_fused
from .formats import FORMATS, WEIGHT_TYPES
from .ops import fused_mul_mat_gguf

_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
_ROLES = (None, "body", "vocabulary")


class PackedGGUFLinear(torch.nn.Module):
    """One GGUF matrix as contiguous row-major wire bytes on the GPU."""

    def __init__(self, data: torch.Tensor, weight_type: int, dtype: torch.dtype, *,
                 canonical_rounding: bool = False, role: str | None = None):
        super().__init__()
        if role not in _ROLES:
            raise ValueError("Unknown GGUF matrix role")
        if dtype not in _DTYPES:
            raise ValueError("Compact GGUF requires FP16, BF16, or FP32 activations")
        if data.ndim != 2:
            raise ValueError("Compact GGUF weights must be a two-dimensional tensor")
        weight_type = int(weight_type)
        if weight_type not in WEIGHT_TYPES:
            raise ValueError(f"Unsupported compact GGUF type: {weight_type}")
        if data.dtype != torch.uint8:
            raise ValueError("Quantized GGUF data must contain uint8 wire bytes")
        _, _, qk, block_bytes = FORMATS[weight_type]
        if data.shape[1] == 0 or data.shape[1] % block_bytes:
            raise ValueError("GGUF row width must be a whole number of wire blocks")
        self.weight_type, self.dtype, self.role = weight_type, dtype, role
        self.canonical_rounding = bool(canonical_rounding)
        self.is_quantized = True
        self.shape = (int(data.shape[0]), int(data.shape[1]) // block_bytes * qk)
        self.register_buffer("weight", data.detach().contiguous())

    def forward(self, x: torch.Tensor, bias: torch.Tensor | None = None, *,
                output_dtype: torch.dtype | None = None) -> torch.Tensor:
        """x @ W.T (+ bias) in output_dtype (the layer dtype, or FP32 for e.g. vocabulary
        logits), with the reference's argument checks (``compact.py:364-394``)."""
        if x.shape[-1] != self.shape[1]:
            raise ValueError("GGUF activation width does not match the weight matrix")
        if x.dtype != self.dtype or x.device != self.weight.device:
            raise ValueError("GGUF activations and weights must share dtype and device")
        output_dtype = self.dtype if output_dtype is None else output_dtype
        if output_dtype not in (self.dtype, torch.float32):
            raise ValueError("Compact GGUF output dtype must match activations or FP32")
        projection = getattr(self, "_kai_fused", None)
        if projection is None:
            projection = native_fused.prepare([self]) or False
            self._kai_fused = projection
        if not projection or not projection.supports(x):
            raise RuntimeError(f"the fused GGUF path cannot run x{tuple(x.shape)} {x.dtype} on {self.shape}")
        return _with_bias(projection(x, output_dtype), bias)


def _with_bias(out, bias):
    return out if bias is None else out + bias


def _rows(x):
    return x.numel() // x.shape[-1] if x.shape[-1] else 0


class _FusedLinear:
    """What both linear methods share: the layer's parts run as one FusedProjection, built on
    first use and kept on the layer (``_kai_fused``, False when ineligible), its consumer
    registration for a norm producer (``_kai_act_producer``), and the producer paths of up to
    8 rows (SwiGLU from gate_up, the column view of the input)."""

    def _parts(self, layer):
        raise NotImplementedError

    def _fused(self, layer):
        projection = getattr(layer, "_kai_fused", None)
        if projection is None:
            parts = list(self._parts(layer))
            projection = (native_fused.prepare(parts) if all(isinstance(p, PackedGGUFLinear) for p in parts)
                          else None) or False
            layer._kai_fused = projection
            producer = layer.__dict__.get("_kai_act_producer")
            if projection and producer is not None:
                native_fused.CONSUMER_OF[projection.weights[0].data_ptr()] = producer
        return projection

    def _producer_path(self, layer, x, width):
        """The fused projection when x (width columns) has 1..8 rows the producers take."""
        projection = self._fused(layer)
        if not projection or not x.is_cuda or x.dtype not in _DTYPES or x.shape[-1] != width(projection):
            return None
        if _rows(x) not in projection._supported or not native_fused.ext_available():
            return None
        return projection

    def apply_swiglu(self, layer, gate_up, act_fn):
        """down_proj(act_fn(gate_up)) with act_fn = silu(gate) * up: up to 8 rows prepare the
        activation straight from gate_up; other inputs apply act_fn first."""
        if getattr(layer, "_kai_input_gather", None) is None and os.environ.get("KAILLM_FUSED_SWIGLU", "1") == "1":
            projection = self._producer_path(layer, gate_up, lambda p: 2 * p.k)
            if projection is not None:
                return projection.call_swiglu(gate_up)
        return self.apply(layer, act_fn(gate_up))

    def _gathered(self, layer, x, bias):
        """(result, x): the view producer's result for up to 8 rows when the layer has an
        input view and no bias, else (None, the input in the stored column order)."""
        gather = getattr(layer, "_kai_input_gather", None)
        if gather is None:
            return None, x
        view = getattr(layer, "_kai_input_view", None)
        if view is not None:
            if bias is None:
                projection = self._producer_path(layer, x, lambda p: p.k)
                if projection is not None:
                    return projection.call_view(x, view), x
            a, b, s = view  # one strided copy: columns [a][b][s] -> [b][a][s]
            return None, x.unflatten(-1, (a, b, s)).transpose(-3, -2).flatten(-3)
        return None, x.index_select(-1, gather)

    def _run_parts(self, layer, x, bias):
        projection = self._fused(layer)
        if projection and projection.supports(x):
            return _with_bias(projection(x), bias)
        outputs = [part(x) for part in self._parts(layer)]
        return _with_bias(outputs[0] if len(outputs) == 1 else torch.cat(outputs, dim=-1), bias)


class GGUFLinearMethod(_FusedLinear):
    """``apply(layer, x, bias)`` of the plugin's GGUF linear (quantization/linear.py:341-407).

    Compact layers list their matrices in ``layer.gguf_compact``; their optional attributes,
    as the reference's loader sets them (yaqa_linear.py:259-266, weights_adapter/qwen35.py:181):
    ``_kai_input_gather`` (column index applied to x first), ``_kai_input_view`` ((a, b, s) when
    that index is the segment transpose [a][b][s] -> [b][a][s]) and ``_kai_act_producer`` (the
    id of the norm whose output this layer consumes, see native_fused.norm_prepare).
    Other layers hold a merged ``qweight`` (see ``_apply_sharded``)."""

    def _parts(self, layer):
        return layer.gguf_compact

    def apply(self, layer, x, bias=None):
        if hasattr(layer, "gguf_compact"):
            done, x = self._gathered(layer, x, bias)
            return done if done is not None else self._run_parts(layer, x, bias)
        return self._apply_sharded(layer, x, bias)

    @staticmethod
    def _apply_sharded(layer, x, bias):
        """A merged ``qweight`` (linear.py:365-407): its shards in ``qweight.shard_id`` order
        (q, k, v first when present) carry GGUF types ``qweight_type.shard_weight_type[id]``
        (default ``qweight_type.weight_type``). One type: one product over the whole merged
        tensor; several: one product per shard on ``qweight[start:end, :width]`` from
        ``qweight.shard_offset_map[id] = (start, end, width)``, concatenated."""
        qweight, qtype = layer.qweight, layer.qweight_type
        shards = list(getattr(qweight, "shard_id", None) or ())
        if not shards:
            out = fused_mul_mat_gguf(x, qweight, int(qtype.weight_type))
        else:
            if "q" in shards:
                shards = ["q", "k", "v"]
            per_shard = getattr(qtype, "shard_weight_type", {})
            kinds = [int(per_shard.get(s, qtype.weight_type)) for s in shards]
            if len(set(kinds)) == 1:
                out = fused_mul_mat_gguf(x, qweight, kinds[0])
            else:
                pieces = []
                for shard, kind in zip(shards, kinds):
                    start, end, width = qweight.shard_offset_map[shard]
                    pieces.append(fused_mul_mat_gguf(x, qweight[start:end, :width].contiguous(), kind))
                out = torch.cat(pieces, dim=1)
        return out if bias is None else out.add_(bias)


class YAQAMixedLinearMethod(_FusedLinear):
    """The plugin's default compact-mode linear method (quantization/yaqa_linear.py:150-405)
    for projections whose sources are ordinary GGUF matrices.

    ``parts`` lists ``(name, (path, tensor_name, descriptor))`` per source matrix, in shard
    order; ``quant_config`` provides ``yaqa_readers`` (path -> kaillm_amd.gguf.GGUFReader) and
    optionally ``gguf_row_permutations`` / ``gguf_column_permutations`` (tensor name -> index
    tensor), ``yaqa_consumed_names`` / ``yaqa_consumed_tensors`` (sets, filled here). YAQA-
    format sources (a descriptor) are not GGUF wire blocks and are refused."""

    def __init__(self, quant_config, parts):
        self.quant_config = quant_config
        self.parts = list(parts)

    def _parts(self, layer):
        return layer.yaqa_parts

    def _expected_rows(self, output_partition_sizes):
        """Rows per source: one source takes the whole output; otherwise one source per
        partition, or consecutive partitions grouped per source tensor (one GGUF tensor
        holding e.g. q|k|v of a merged projection), as yaqa_linear.py:183-199 groups them."""
        sizes = [int(s) for s in output_partition_sizes]
        if len(self.parts) == 1:
            return [sum(sizes)]
        if len(sizes) == len(self.parts):
            return sizes
        grouped, it = [], iter(sizes)
        for _, (path, tensor_name, _) in self.parts:
            need = self._source_shape(path, tensor_name)[0]
            got = 0
            for size in it:
                got += size
                if got >= need:
                    break
            grouped.append(got)
        return grouped if sum(grouped) == sum(sizes) else sizes

    def _source_shape(self, path, tensor_name):
        t = self.quant_config.yaqa_readers[path].tensor(tensor_name)
        return int(t.shape[1]), int(t.shape[0])  # (rows, columns): GGUF dims are innermost first

    def create_weights(self, layer, input_size_per_partition, output_partition_sizes, input_size, output_size,
                       params_dtype, **extra_weight_attrs):
        from . import gguf

        if getattr(layer, "tp_size", 1) != 1:
            raise ValueError("Packed YAQA currently requires tensor_parallel_size=1")
        cfg = self.quant_config
        rows_perm = getattr(cfg, "gguf_row_permutations", {}) or {}
        cols_perm = getattr(cfg, "gguf_column_permutations", {}) or {}
        device = torch.empty(0).device if torch.empty(0).is_cuda else torch.device("cuda", torch.cuda.current_device())
        expected = self._expected_rows(output_partition_sizes)
        if len(expected) != len(self.parts):
            raise ValueError("Mixed YAQA shards differ from vLLM output partitions")
        modules, gathers = [], []
        for (name, (path, tensor_name, descriptor)), want_rows in zip(self.parts, expected):
            if descriptor is not None:
                raise ValueError(f"YAQA-format matrices are not GGUF wire blocks: {tensor_name}")
            part, gather, view = gguf.load_packed(cfg.yaqa_readers[path], tensor_name, params_dtype, device,
                                                  rows_perm.get(tensor_name), cols_perm.get(tensor_name))
            part.role = "body"
            part.canonical_rounding = bool(getattr(cfg, "canonical_gguf_rounding", False))
            if part.shape[1] != input_size_per_partition:
                raise ValueError(f"Mixed YAQA input shape mismatch for {name}")
            if part.shape[0] != want_rows:
                raise ValueError(f"Mixed YAQA output shape mismatch for {name}")
            if gather is not None:
                gathers.append((gather, view))
            modules.append(part)
            for attr, value in (("yaqa_consumed_names", name), ("yaqa_consumed_tensors", tensor_name)):
                consumed = getattr(cfg, attr, None)
                if consumed is not None:
                    consumed.add(value)
        layer.yaqa_parts = torch.nn.ModuleList(modules)
        if gathers:
            first, view = gathers[0]
            if len(gathers) != len(modules) or any(not torch.equal(g, first) for g, _ in gathers):
                raise ValueError("Merged GGUF projections need one shared input permutation")
            layer._kai_input_gather, layer._kai_input_view = first, view

    def process_weights_after_loading(self, layer):
        """Nothing to convert: the parts keep their GGUF wire bytes."""

    def apply(self, layer, x, bias=None):
        done, x = self._gathered(layer, x, bias)
        return done if done is not None else self._apply_original(layer, x, bias)

    def _apply_original(self, layer, x, bias=None):
        """The fused projection when it takes x; else each part on its own, concatenated."""
        return self._run_parts(layer, x, bias)
