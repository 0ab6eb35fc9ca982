"""GGUF wire-format ingestion: read a model file's tensor table and upload packed weights.

Mirrors, for the weights of the fused path:
  * ``GGUFReader`` of the reference's gguf-reader (``gguf-reader/gguf/gguf_reader.py:116-390``):
    ``fields`` (ordered metadata, each ``ReaderField.contents()``), ``tensors`` (``ReaderTensor``
    with ``name``, ``tensor_type``, ``shape`` (GGML order, innermost first), ``n_elements``,
    ``n_bytes``, ``data_offset`` and ``data``, a read-only memory map in numpy order whose
    quantized rows are ``uint8 [..., row_bytes]``), ``alignment`` and ``data_offset``;
  * the loader's stored-tensor permutations (``quantization/yaqa_linear.py:102-148``):
    ``permute_stored`` and ``transpose_view``;
  * ``load_packed``: one GGUF matrix to a ``PackedGGUFLinear`` on the GPU. Rows come straight
    from the file through ``kai_upload_rows``, which applies the row permutation and a
    block-aligned column permutation while staging, so the bytes land in HBM once, in the
    order the kernels read.

The file format is GGUF v2/v3, little-endian: magic, version, tensor and key-value counts,
the key-value section, the tensor-info section, then tensor data at ``alignment``
(``general.alignment``, default 32) from the end of the tensor infos.
"""
from __future__ import annotations

import struct
from collections import OrderedDict
from typing import Any, NamedTuple

import numpy as np
import torch

from . import native

GGUF_MAGIC = 0x46554747  # b"GGUF" read as a little-endian uint32
GGUF_VERSION = 3
GGUF_DEFAULT_ALIGNMENT = 32
READER_SUPPORTED_VERSIONS = (2, 3)
GGML_MAX_DIMS = 4

# Metadata value types.
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALAR = {UINT8: "<u1", INT8: "<i1", UINT16: "<u2", INT16: "<i2", UINT32: "<u4", INT32: "<i4",
           FLOAT32: "<f4", BOOL: "<u1", UINT64: "<u8", INT64: "<i8", FLOAT64: "<f8"}

# GGML tensor types: id -> (name, values per block, bytes per block). The published format table.
GGML_TYPES = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20), 6: ("Q5_0", 32, 22),
    7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 9: ("Q8_1", 32, 36), 10: ("Q2_K", 256, 84), 11: ("Q3_K", 256, 110),
    12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210), 15: ("Q8_K", 256, 292),
    16: ("IQ2_XXS", 256, 66), 17: ("IQ2_XS", 256, 74), 18: ("IQ3_XXS", 256, 98), 19: ("IQ1_S", 256, 50),
    20: ("IQ4_NL", 32, 18), 21: ("IQ3_S", 256, 110), 22: ("IQ2_S", 256, 82), 23: ("IQ4_XS", 256, 136),
    24: ("I8", 1, 1), 25: ("I16", 1, 2), 26: ("I32", 1, 4), 27: ("I64", 1, 8), 28: ("F64", 1, 8),
    29: ("IQ1_M", 256, 56), 30: ("BF16", 1, 2), 34: ("TQ1_0", 256, 54), 35: ("TQ2_0", 256, 66),
    39: ("MXFP4", 32, 17),
}
GGML_QUANT_SIZES = {t: (qk, bb) for t, (_, qk, bb) in GGML_TYPES.items()}
_PLAIN = {0: np.float32, 1: np.float16, 24: np.int8, 25: np.int16, 26: np.int32, 27: np.int64, 28: np.float64}


class ReaderField(NamedTuple):
    """One metadata key-value pair (or one tensor-info record, whose ``types`` is empty)."""

    offset: int
    name: str
    types: list[int]
    value: Any

    def contents(self, index_or_slice: int | slice = slice(None)) -> Any:
        if self.types and self.types[0] == ARRAY:
            return self.value[index_or_slice]
        return self.value


class ReaderTensor(NamedTuple):
    name: str
    tensor_type: int
    shape: np.ndarray
    n_elements: int
    n_bytes: int
    data_offset: int
    data: np.ndarray
    field: ReaderField


class _Cursor:
    def __init__(self, buf: np.ndarray, offset: int):
        self.buf, self.offset = buf, offset

    def take(self, dtype: str, count: int = 1) -> np.ndarray:
        item = np.dtype(dtype)
        end = self.offset + item.itemsize * count
        if end > self.buf.size:
            raise ValueError("GGUF file is truncated")
        out = self.buf[self.offset:end].view(item)
        self.offset = end
        return out

    def scalar(self, dtype: str):
        return self.take(dtype)[0].item()

    def string(self, limit: int = 1 << 30) -> str:
        n = self.scalar("<u8")
        if n > limit:
            raise ValueError(f"String length {n} exceeds the GGUF limit")
        return bytes(self.take("<u1", n)).decode("utf-8")

    def value(self, vtype: int, types: list[int]):
        types.append(vtype)
        if vtype == STRING:
            return self.string()
        if vtype in _SCALAR:
            v = self.scalar(_SCALAR[vtype])
            return bool(v) if vtype == BOOL else v
        if vtype == ARRAY:
            itype = self.scalar("<u4")
            n = self.scalar("<u8")
            if n > 1 << 30:
                raise ValueError(f"Array length {n} exceeds the GGUF limit")
            if itype in _SCALAR:  # one read for a whole numeric array
                types.append(itype)
                values = self.take(_SCALAR[itype], n).tolist()
                return [bool(v) for v in values] if itype == BOOL else values
            sub: list[int] = []
            values = [self.value(itype, sub) for _ in range(n)]
            types.extend(sub[:1] if sub else [itype])
            return values
        raise ValueError(f"Unknown GGUF value type {vtype}")


class GGUFReader:
    """Read-only view of a GGUF file (tensor data memory-mapped, nothing copied)."""

    byte_order = "I"

    def __init__(self, path, mode: str = "r"):
        if mode != "r":
            raise ValueError("Only read-only access is supported")
        self.path = str(path)
        self.data = np.memmap(self.path, mode="r")
        cur = _Cursor(self.data, 0)
        if cur.scalar("<u4") != GGUF_MAGIC:
            raise ValueError("GGUF magic invalid")
        version = cur.scalar("<u4")
        if version & 0xFFFF == 0:
            raise ValueError("Big-endian GGUF files are not supported")
        if version not in READER_SUPPORTED_VERSIONS:
            raise ValueError(f"GGUF version {version} is not supported")
        self.version = version
        n_tensors, n_kv = cur.scalar("<u8"), cur.scalar("<u8")
        self.fields: OrderedDict[str, ReaderField] = OrderedDict()
        for _ in range(n_kv):
            start = cur.offset
            key = cur.string()
            types: list[int] = []
            value = cur.value(cur.scalar("<u4"), types)
            if key in self.fields:
                raise KeyError(f"Duplicate {key} already in list at offset {self.fields[key].offset}")
            self.fields[key] = ReaderField(start, key, types, value)
        infos = []
        for _ in range(n_tensors):
            start = cur.offset
            name = cur.string()
            n_dims = cur.scalar("<u4")
            if n_dims > GGML_MAX_DIMS:
                raise ValueError(f"Tensor dimensions count {n_dims} exceeds GGML_MAX_DIMS")
            dims = cur.take("<u8", n_dims).copy()
            ttype, offset = cur.scalar("<u4"), cur.scalar("<u8")
            infos.append((ReaderField(start, name, [], None), name, dims, ttype, offset))
        align_field = self.fields.get("general.alignment")
        self.alignment = int(align_field.value) if align_field is not None else GGUF_DEFAULT_ALIGNMENT
        if self.alignment <= 0 or self.alignment & (self.alignment - 1):
            raise ValueError(f"Invalid GGUF alignment {self.alignment}")
        self.data_offset = -(-cur.offset // self.alignment) * self.alignment
        self.tensors: list[ReaderTensor] = []
        seen = set()
        for field, name, dims, ttype, offset in infos:
            if name in seen:
                raise ValueError(f"Found duplicated tensor with name {name}")
            seen.add(name)
            if ttype not in GGML_TYPES:
                raise ValueError(f"Unknown GGML tensor type {ttype}")
            qk, bb = GGML_QUANT_SIZES[ttype]
            n_elems = 1
            for d in dims.tolist():
                n_elems *= int(d)
            if dims.size and int(dims[0]) % qk:
                raise ValueError(f"Tensor {name}: row of {int(dims[0])} values is not whole {qk}-value blocks")
            n_bytes = n_elems // qk * bb
            start = self.data_offset + int(offset)
            if start + n_bytes > self.data.size:
                raise ValueError(f"Tensor {name} extends past the end of the file")
            np_dims = tuple(int(d) for d in reversed(dims.tolist())) or (1,)
            if ttype in _PLAIN:
                arr = self.data[start:start + n_bytes].view(_PLAIN[ttype]).reshape(np_dims)
            elif ttype == 30:  # BF16: raw 16-bit words
                arr = self.data[start:start + n_bytes].view(np.uint16).reshape(np_dims)
            else:
                arr = self.data[start:start + n_bytes].reshape(*np_dims[:-1], np_dims[-1] // qk * bb)
            self.tensors.append(ReaderTensor(name, ttype, dims, n_elems, n_bytes, start, arr, field))

    def get_field(self, key: str) -> ReaderField | None:
        return self.fields.get(key)

    def get_tensor(self, idx: int) -> ReaderTensor:
        return self.tensors[idx]

    def tensor(self, name: str) -> ReaderTensor:
        for t in self.tensors:
            if t.name == name:
                return t
        raise KeyError(name)


def inverse_permutation(columns: torch.Tensor) -> torch.Tensor:
    """g with g[columns[i]] = i: the activation gather that matches a weight whose columns
    were permuted by ``columns`` (x_stored = x.index_select(-1, g))."""
    g = torch.empty_like(columns)
    g.scatter_(0, columns, torch.arange(columns.numel(), dtype=columns.dtype, device=columns.device))
    return g


def block_order(columns: torch.Tensor, block: int) -> torch.Tensor | None:
    """When ``columns`` only moves whole ``block``-value blocks (every run of ``block``
    consecutive entries is one source block, in order), the source block of each stored
    block; else None."""
    n = columns.numel()
    if n == 0 or n % block:
        return None
    sources = torch.div(columns[::block], block, rounding_mode="floor")
    rebuilt = (sources[:, None] * block + torch.arange(block, dtype=columns.dtype, device=columns.device)).reshape(-1)
    return sources.to(torch.long) if torch.equal(rebuilt, columns) else None


def permute_stored(data: torch.Tensor, qtype: int, rows: torch.Tensor | None, columns: torch.Tensor | None):
    """A stored matrix under the loader's row and column permutations
    (the reference's _permute_stored, yaqa_linear.py:102-127): returns (data, gather).

    Rows are reordered in place. A column permutation of a dense matrix is applied to it; on
    wire bytes it is applied only when it moves whole GGML blocks (the blocks are reordered);
    otherwise the bytes keep their order and ``gather`` reorders the activation instead."""
    if rows is not None:
        data = data[rows]
    if columns is None:
        return data, None
    if data.dtype != torch.uint8:
        return data[:, columns].contiguous(), None
    qk, bb = GGML_QUANT_SIZES[qtype]
    order = block_order(columns, qk)
    if order is None:
        return data, inverse_permutation(columns)
    blocks = data.reshape(data.shape[0], -1, bb).index_select(1, order.to(data.device))
    return blocks.reshape(data.shape[0], -1).contiguous(), None


def transpose_view(gather: torch.Tensor):
    """(a, b, s) when the gather reads x's columns as [a][b][s] in the order [b][a][s], i.e.
    gather[c] = ((c // s) % a) * b * s + (c // (a * s)) * s + c % s for every column c; else
    None (the reference's _transpose_view, yaqa_linear.py:130-148). Such a gather is the
    fused view producer's input (kai_fused_prepare_view)."""
    g = gather.detach().to("cpu", torch.int64)
    n = g.numel()
    if n < 2 or int(g[0]) != 0:
        return None
    # s: the length of the leading run 0, 1, 2, ... (a segment is copied whole)
    steps = torch.nonzero(g[1:] - g[:-1] != 1)
    if steps.numel() == 0:
        return None
    s = int(steps[0]) + 1
    b = int(g[s]) // s
    if n % s or int(g[s]) % s or b < 2 or n % (b * s):
        return None
    a = n // (b * s)
    c = torch.arange(n)
    expect = ((c // s) % a) * (b * s) + (c // (a * s)) * s + c % s
    return (a, b, s) if torch.equal(g, expect) else None


def upload(reader: GGUFReader, tensor: ReaderTensor, device, rows: torch.Tensor | None = None,
           blocks: torch.Tensor | None = None) -> torch.Tensor:
    """The tensor's stored rows as ``uint8 [rows, row_bytes]`` on ``device``, straight from the
    file: dst row r = source row rows[r], dst block j = source block blocks[j]."""
    qk, bb = GGML_QUANT_SIZES[tensor.tensor_type]
    row_bytes = int(tensor.shape[0]) // qk * bb if tensor.shape.size else bb
    src_rows = tensor.n_bytes // row_bytes
    row_idx = None if rows is None else np.ascontiguousarray(rows.cpu().numpy(), dtype=np.int64)
    blk_idx = None if blocks is None else np.ascontiguousarray(blocks.cpu().numpy(), dtype=np.int64)
    n_rows = src_rows if row_idx is None else row_idx.size
    device = torch.device(device)
    out = torch.empty((n_rows, row_bytes), dtype=torch.uint8, device=device)
    lib = native.library()
    stream = torch.cuda.current_stream(device).cuda_stream

    def ptr(a):
        return None if a is None else a.ctypes.data

    native.check(lib, lib.kai_upload_rows(reader.path.encode(), tensor.data_offset, src_rows, row_bytes,
                                          ptr(row_idx), n_rows, bb, ptr(blk_idx), out.data_ptr(), stream))
    return out


def load_packed(reader: GGUFReader, name: str, dtype: torch.dtype, device,
                row_permutation: torch.Tensor | None = None, column_permutation: torch.Tensor | None = None):
    """(PackedGGUFLinear, gather, view) for one quantized GGUF matrix.

    The row permutation and a block-aligned column permutation are applied during the
    upload; any other column permutation leaves the stored bytes and returns the activation
    gather (with its (a, b, s) form when it is a segment transpose), as the reference's
    loader sets ``_kai_input_gather`` / ``_kai_input_view`` (yaqa_linear.py:259-266).
    """
    from .linear import PackedGGUFLinear

    t = reader.tensor(name)
    if t.tensor_type in _PLAIN or t.tensor_type == 30 or t.shape.size != 2:
        raise ValueError(f"{name} is not a quantized matrix")
    qk = GGML_QUANT_SIZES[t.tensor_type][0]
    blocks, gather = None, None
    if column_permutation is not None:
        blocks = block_order(column_permutation.cpu(), qk)
        if blocks is None:
            gather = inverse_permutation(column_permutation)
    data = upload(reader, t, device, row_permutation, blocks)
    layer = PackedGGUFLinear(data, t.tensor_type, dtype)
    view = transpose_view(gather) if gather is not None else None
    return layer, (None if gather is None else gather.to(device)), view


def write_gguf(path, tensors, metadata=None, alignment: int = GGUF_DEFAULT_ALIGNMENT, version: int = GGUF_VERSION):
    """Write a GGUF file: ``tensors`` is a list of (name, ggml_type, dims (innermost first),
    raw bytes as a numpy array); ``metadata`` maps keys to (value_type, value). Used to build
    test models; it writes only what the reader above reads."""
    metadata = dict(metadata or {})
    if alignment != GGUF_DEFAULT_ALIGNMENT:
        metadata["general.alignment"] = (UINT32, alignment)
    out = bytearray(struct.pack("<IIQQ", GGUF_MAGIC, version, len(tensors), len(metadata)))

    def put_string(s):
        b = s.encode("utf-8")
        out.extend(struct.pack("<Q", len(b)) + b)

    def put_value(vtype, value):
        if vtype == STRING:
            put_string(value)
        elif vtype == ARRAY:
            itype, items = value
            out.extend(struct.pack("<IQ", itype, len(items)))
            for item in items:
                put_value(itype, item)
        else:
            out.extend(np.array([value], dtype=_SCALAR[vtype]).tobytes())

    for key, (vtype, value) in metadata.items():
        put_string(key)
        out.extend(struct.pack("<I", vtype))
        put_value(vtype, value)
    offsets, cursor = [], 0
    for _, _, _, raw in tensors:
        offsets.append(cursor)
        cursor += -(-raw.nbytes // alignment) * alignment
    for (name, ttype, dims, _), offset in zip(tensors, offsets):
        put_string(name)
        out.extend(struct.pack("<I", len(dims)))
        out.extend(struct.pack(f"<{len(dims)}Q", *dims))
        out.extend(struct.pack("<IQ", ttype, offset))
    out.extend(b"\0" * (-len(out) % alignment))
    for (_, _, _, raw), offset in zip(tensors, offsets):
        body = np.ascontiguousarray(raw).view(np.uint8).reshape(-1).tobytes()
        out.extend(body + b"\0" * (-len(body) % alignment))
    with open(path, "wb") as f:
        f.write(out)
