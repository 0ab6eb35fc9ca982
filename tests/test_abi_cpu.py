"""The C ABI without a GPU: the library loads, exports every declared symbol, and
rejects host-detectable bad arguments the way the reference does
(current_ggml_direct.cu:826-863, 946-965, 1196-1218)."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import _oracle as O

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    names = []
    for header in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names += re.findall(r"^[A-Za-z_][\w\s\*]*?\b(\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_every_declared_symbol_is_exported(kai):
    names = declared_functions()
    assert {"kai_fused_supported", "kai_fused_prepare", "kai_fused_mmvq", "kai_fused_mmq_run"} <= set(names)
    for name in names:
        assert hasattr(kai, name), name


@pytest.mark.parametrize("args,want", [
    ((12, 34816, 5120, 1), 1), ((12, 34816, 5120, 8), 1), ((12, 34816, 5120, 9), 0),
    ((12, 34816, 5120, 0), 0), ((12, 100, 5000, 1), 0),  # k % 256
    ((2, 100, 48, 1), 0), ((8, 100, 32768, 1), 1), ((8, 100, 32800, 1), 0),  # k/32 <= 1024
    ((3, 100, 256, 1), 0), ((21, 0, 256, 1), 0), ((21, 2 ** 31, 256, 1), 0), ((14, 5, 256, 4), 1),
])
def test_supported(kai, args, want):
    assert kai.kai_fused_supported(*args) == want


def test_activation_bytes_matches_layout(kai):
    for m, k, tp in ((1, 2048, 0), (3, 5120, 1), (16, 17408, 0), (2048, 5120, 0), (5, 96, 0)):
        assert kai.kai_fused_activation_bytes(m, k, tp) == O.activation_bytes(m, k, tp)


def test_bad_arguments_fail_before_any_launch(kai):
    dummy = ctypes.c_void_p(16)
    assert kai.kai_fused_prepare(None, 0, 1, 64, 64, dummy, 0, 0) == -1
    assert b"Invalid fused activation" in kai.current_direct_error()
    assert kai.kai_fused_prepare(dummy, 0, 1, 60, 64, dummy, 0, 0) == -1   # k % 32
    assert kai.kai_fused_prepare(dummy, 0, 1, 64, 32, dummy, 0, 0) == -1   # stride < k
    assert kai.kai_fused_mmvq(dummy, 12, 16, 256, 9, dummy, 0, dummy, 0, 16, 0) == -1  # m > 8
    assert b"Invalid fused MMVQ" in kai.current_direct_error()
    assert kai.kai_fused_mmvq(dummy, 12, 16, 256, 1, dummy, 0, dummy, 0, 15, 0) == -1  # stride < n
    assert kai.kai_fused_mmvq(dummy, 7, 16, 256, 1, dummy, 0, dummy, 0, 16, 0) == -1   # type
    assert kai.kai_fused_mmvq(None, 12, 16, 256, 1, dummy, 0, dummy, 0, 16, 0) == -1


def test_producers_reject_bad_arguments_before_any_launch(kai):
    """current_ggml_direct.cu:883-944: the reference's argument rules, checked on the host."""
    d = ctypes.c_void_p(256)
    assert kai.kai_fused_prepare_view(d, 1, 1, 96, 96, d, 2, 2, 32, 0) == -1      # a*b*s != k
    assert b"Invalid fused view preparation" in kai.current_direct_error()
    assert kai.kai_fused_prepare_view(d, 1, 9, 96, 96, d, 3, 1, 32, 0) == -1      # m > 8
    assert kai.kai_fused_prepare_view(d, 1, 1, 96, 96, d, 6, 1, 16, 0) == -1      # s % 32
    assert kai.kai_fused_prepare_view(d, 1, 1, 96, 64, d, 3, 1, 32, 0) == -1      # stride < k
    assert kai.kai_fused_prepare_view(d, 3, 1, 96, 96, d, 3, 1, 32, 0) == -1      # dtype
    assert b"F32, BF16 or F16" in kai.current_direct_error()
    assert kai.kai_fused_prepare_view(d, 1, 1, 32800, 32800, d, 1025, 1, 32, 0) == -1
    assert b"32768" in kai.current_direct_error()
    assert kai.kai_fused_prepare_swiglu(d, 1, 1, 64, 127, d, 0) == -1            # stride < 2k
    assert b"Invalid fused SwiGLU preparation" in kai.current_direct_error()
    assert kai.kai_fused_prepare_swiglu(None, 1, 1, 64, 128, d, 0) == -1
    assert kai.kai_fused_prepare_swiglu(d, 1, 0, 64, 128, d, 0) == -1            # m < 1
    assert kai.kai_fused_norm_prepare(d, 1, 64, d, 0, 64, None, d, 1e-6, d, 1, 64, d, 0) == -1  # no r_out
    assert b"Invalid fused norm preparation" in kai.current_direct_error()
    assert kai.kai_fused_norm_prepare(d, 1, 64, None, 0, 0, None, None, 1e-6, d, 1, 64, d, 0) == -1  # no w
    assert kai.kai_fused_norm_prepare(d, 1, 32, None, 0, 0, None, d, 1e-6, d, 1, 64, d, 0) == -1  # stride
    assert kai.kai_fused_norm_prepare(d, 1, 64, None, 0, 0, None, d, 1e-6, ctypes.c_void_p(258), 1, 64, d,
                                      0) == -1
    assert b"16-byte aligned" in kai.current_direct_error()
    assert kai.kai_fused_norm_prepare(d, 2, 64, None, 0, 0, None, d, 1e-6, d, 1, 64, d, 0) == -1  # f16 x
    assert b"BF16 or F32" in kai.current_direct_error()
    assert kai.kai_fused_norm_prepare(d, 1, 64, d, 2, 64, d, d, 1e-6, d, 1, 64, d, 0) == -1  # f16 residual
    assert b"BF16 or F32" in kai.current_direct_error()


def test_dequantize_rejects_bad_arguments_before_any_launch(kai):
    d = ctypes.c_void_p(256)
    assert kai.kai_dequantize(d, 3, 4, 256, d, 1, 0) == -1           # Q4_1 is not implemented
    assert b"Unsupported GGML weight type" in kai.current_direct_error()
    assert kai.kai_dequantize(d, 12, 4, 288, d, 1, 0) == -1          # cols % 256
    assert b"Invalid dequantization" in kai.current_direct_error()
    assert kai.kai_dequantize(None, 12, 4, 256, d, 1, 0) == -1
    assert kai.kai_dequantize(d, 12, -1, 256, d, 1, 0) == -1
    assert kai.kai_dequantize(d, 8, 4, 64, ctypes.c_void_p(258), 2, 0) == -1
    assert b"16-byte aligned" in kai.current_direct_error()
    assert kai.kai_dequantize(d, 8, 4, 64, d, 3, 0) == -1            # output dtype
    assert b"F32, BF16 or F16" in kai.current_direct_error()


def test_mmq_workspace_rules(kai):
    types = (ctypes.c_int * 2)(12, 14)
    rows = (ctypes.c_int64 * 2)(34816, 5120)
    assert kai.kai_fused_mmq_workspace(0, types, rows, 2, 5120, 16, 0) > 0
    assert kai.kai_fused_mmq_workspace(0, types, rows, 2, 5120, 8, 0) == 0          # needs m > 8
    assert b"more than 8" in kai.current_direct_error()
    assert kai.kai_fused_mmq_workspace(0, types, rows, 0, 5120, 16, 0) == 0         # empty group
    odd = (ctypes.c_int64 * 2)(34816, 5119)
    assert kai.kai_fused_mmq_workspace(0, types, odd, 2, 5120, 16, 0) == 0          # sum % 4
    assert kai.kai_fused_mmq_workspace(-1, types, rows, 2, 5120, 16, 0) == 0        # device
    ptrs = (ctypes.c_void_p * 2)(16, 32)
    assert kai.kai_fused_mmq_run(ptrs, types, rows, 2, ctypes.c_void_p(16), 2, 5120, 5120, 16,
                                 ctypes.c_void_p(16), 0, 0, ctypes.c_void_p(16), 10, 0, 0) == -1
    assert b"scratch" in kai.current_direct_error()


def _plane_bytes(m, k):
    return (k + 511) // 512 * 4 * m * 144


def _image_bytes(layout, k):
    return (k + 255) // 256 * (4608 if layout == O.D4 else 5632)


H_TYPES = (O.Q4_K, O.Q4_0, O.Q8_0, O.IQ3_S, O.Q2_K)  # the fp16 GEMM's formats (above 16 rows)


def _uses_h(qtype, m, n):
    """The batched route rule: the fp16 GEMM above 16 rows for its formats."""
    return qtype in H_TYPES and m > 16


def test_mmq_workspace_follows_the_route_rule(kai):
    """Above 16 rows Q4_K reads the fp16 image (34816 or 5120 rows, 80 or 97 rows); Q6_K, on
    the int8 tile kernel, reads its plane (the D2S6 plane has the DS4 plane's size)."""
    a256 = lambda b: (b + 255) // 256 * 256
    for qtype, n, m, image in ((O.Q4_K, 34816, 80, True), (O.Q4_K, 5120, 80, True), (O.Q4_K, 34816, 97, True),
                               (O.Q6_K, 5120, 80, False)):
        types = (ctypes.c_int * 1)(qtype)
        rows = (ctypes.c_int64 * 1)(n)
        got = kai.kai_fused_mmq_workspace(0, types, rows, 1, 5120, m, 1)
        base = a256(4 * m) + (_h_image_bytes(O.DS4, m, 5120) if image else a256(_plane_bytes(m, 5120)))
        assert base <= got, (n, m)
        assert _uses_h(qtype, m, n) == image
        # the remainder is the fp16 GEMM's split-K sums (at most 8 splits of m x n fp32); the int8
        # tile kernel has none
        assert (got - base) % 256 == 0 and got - base <= a256(8 * m * n * 4), (n, m, got - base)
        if not image:
            assert got == base, (n, m, got - base)


def test_mmq_workspace_holds_the_tail_pieces(kai):
    """More fp16 GEMM tiles than CUs with at most half the CUs' worth left for the last round:
    those last tiles (inside the last activation tile) run in K pieces (at most 8, whole
    256-value steps, as many as the idle CUs take), whose sums are pieces x rows x columns
    fp32. Q4_K 18000 x 1024 at 300 rows: 2 x 141 tiles of 256 x 128, the last 26 in 4 pieces
    over rows 256..299 and columns 14720..17999, and Q2_K the same (its 256-row tile fits the
    LDS with 96-byte raw rows); in place of a
    K split, Q4_0 and IQ3_S 33000 x 1024 at 40 and 120 rows: 258 tiles of 128 weight rows, the
    last 2 in 4 pieces over every row and columns 32768..32999; two activation tiles high, Q4_K
    5120 x 17408 at 2048 rows (8 x 40 tiles of 256 x 128, in place of a four-way K split): the
    last 32 weight tiles of the last 2 in 4 pieces, rows 1536..2047 by columns 1024..5119."""
    a256 = lambda b: (b + 255) // 256 * 256
    for qtype, n, k, m, pieces in ((O.Q4_K, 18000, 1024, 300, 4 * 44 * 3280), (O.Q2_K, 18000, 1024, 300, 4 * 44 * 3280),
                                   (O.Q4_0, 33000, 1024, 40, 4 * 40 * 232), (O.IQ3_S, 33000, 1024, 120, 4 * 120 * 232),
                                   (O.Q4_K, 5120, 17408, 2048, 4 * 512 * 4096)):
        types = (ctypes.c_int * 1)(qtype)
        rows = (ctypes.c_int64 * 1)(n)
        got = kai.kai_fused_mmq_workspace(0, types, rows, 1, k, m, 1)
        base = a256(4 * m) + _h_image_bytes(O.mmq_layout(qtype), m, k)
        assert got - base == a256(4 * pieces), (O.NAMES[qtype], got - base)


def _h_image_bytes(layout, m, k):
    """The fp16 GEMM's image of one layout: codes and min-pass sums, each 256-aligned."""
    a256 = lambda b: (b + 255) // 256 * 256
    mpad, kpad = (m + 31) // 32 * 32, (k + 255) // 256 * 256
    codes = kpad * mpad * 2
    mins = 0 if layout == O.D4 else (k + 255) // 256 * mpad * (64 if layout == O.DS4 else 128)
    return a256(codes) + a256(mins)


def test_mmq_workspace_is_inverse_then_one_plane_per_layout(kai):
    """[inverse m f32][D4][DS4][D2S6], each 256-aligned, a region only for a layout that a
    matrix on the int8 kernels reads (Q8_0/Q6_K/IQ3_S: D4; Q4_0/Q4_K: DS4; Q2_K: D2S6): a
    plane, or up to 16 rows the small-M image (per 256-value step 4608 bytes for D4, 5632 with
    the term arrays); above 16 rows the fp16 GEMM's image of each layout its formats read (Q6_K
    keeps the int8 plane); then the partial sums: the small-M GEMM's (16 x 16 fp32 per piece
    of a 16-row set, fewer pieces per set than K steps) or the fp16 GEMM's split-K sums (m x n
    fp32 per split, at most 8 splits)."""
    a256 = lambda b: (b + 255) // 256 * 256
    for tl, m, k in (((12,), 16, 5120), ((12, 14), 80, 17408), ((10, 21, 2), 33, 1024), ((8,), 9, 1056),
                     ((14,), 16, 17408), ((10, 21, 2), 12, 4096), ((14, 21), 40, 5120), ((2,), 600, 1056)):
        types = (ctypes.c_int * len(tl))(*tl)
        rows = (ctypes.c_int64 * len(tl))(*([64] * len(tl)))
        got = kai.kai_fused_mmq_workspace(0, types, rows, len(tl), k, m, 1)
        if m > 16:
            planes = {O.mmq_layout(t) for t in tl if not _uses_h(t, m, 64)}
            images = {O.mmq_layout(t) for t in tl if _uses_h(t, m, 64)}
            want = a256(4 * m) + len(planes) * a256(_plane_bytes(m, k)) + sum(_h_image_bytes(l, m, k) for l in images)
            extra = got - want
            assert extra >= 0 and extra % 256 == 0 and extra <= a256(8 * m * 64 * 4), (tl, m, k, extra)
        else:
            layouts = {O.mmq_layout(t) for t in tl}
            want = a256(4 * m) + sum(a256(_image_bytes(l, k)) for l in layouts)
            assert want <= got <= want + a256((k + 255) // 256 * 4 * 1024)


def test_noalloc_capacity_and_oversized_call(kai):
    assert kai.kai_fused_mmq_noalloc_capacity() == 16 << 20
    types = (ctypes.c_int * 1)(14)
    rows = (ctypes.c_int64 * 1)(5120)
    ptrs = (ctypes.c_void_p * 1)(16)
    # M = 2048 at K = 17408 needs 40 MiB of planes: refused before any device work
    assert kai.kai_fused_mmq_run_noalloc(ptrs, types, rows, 1, ctypes.c_void_p(16), 2, 17408, 17408, 2048,
                                         ctypes.c_void_p(16), 0, 0, 0, 0) == -1
    assert b"16 MiB" in kai.current_direct_error()
    assert kai.kai_fused_mmq_run_noalloc(ptrs, types, rows, 1, ctypes.c_void_p(16), 2, 17408, 17408, 8,
                                         ctypes.c_void_p(16), 0, 0, 0, 0) == -1   # m <= 8
    assert b"more than 8" in kai.current_direct_error()


@pytest.mark.parametrize("qtype", O.WEIGHT_TYPES, ids=lambda t: O.NAMES[t])
def test_quantizer_round_trip(qtype):
    """The host quantizer writes valid blocks whose oracle dequantization tracks the floats."""
    from kaillm_amd.formats import quantize

    rng = np.random.default_rng(qtype)
    w = rng.normal(0, 0.02, (64, 1024)).astype(np.float32)
    packed = quantize(w, qtype)
    deq = O.dequantize(qtype, packed, 1024)
    rel = np.sqrt(((deq - w) ** 2).mean() / (w ** 2).mean())
    bound = {O.Q8_0: 0.01, O.Q4_0: 0.15, O.Q4_K: 0.12, O.Q6_K: 0.04, O.Q2_K: 0.5, O.IQ3_S: 0.35}[qtype]
    assert rel < bound, rel


def test_quantizer_matches_gguf_closed_forms():
    """Q8_0 / Q4_0 follow gguf-py quants.py:382-394 / :223-239 (restated here in numpy)."""
    from kaillm_amd.formats import quantize

    rng = np.random.default_rng(3)
    blocks = rng.normal(0, 0.02, (40, 32)).astype(np.float32)
    d = np.abs(blocks).max(axis=1, keepdims=True) / np.float32(127)
    with np.errstate(divide="ignore"):
        idv = np.where(d == 0, 0, 1 / d).astype(np.float32)
    t = blocks * idv
    a = np.abs(t)
    q = (np.sign(t) * (np.floor(a) + np.floor(2 * (a - np.floor(a))))).astype(np.int8)
    want = np.concatenate([d.astype(np.float16).view(np.uint8), q.view(np.uint8)], axis=1)
    assert np.array_equal(quantize(blocks, O.Q8_0), want)
    imax = np.abs(blocks).argmax(axis=-1)[:, None]
    mx = np.take_along_axis(blocks, imax, axis=-1)
    d4 = mx / np.float32(-8)
    with np.errstate(divide="ignore"):
        id4 = np.where(d4 == 0, 0, 1 / d4).astype(np.float32)
    qs = np.trunc(blocks * id4 + np.float32(8.5)).astype(np.uint8).clip(0, 15)
    qs = qs[:, :16] | (qs[:, 16:] << 4)
    want4 = np.concatenate([d4.astype(np.float16).view(np.uint8), qs], axis=1)
    assert np.array_equal(quantize(blocks, O.Q4_0), want4)


def test_legacy_op_workspace_and_argument_rules(kai):
    """kai_ggml_* (gguf_kernel.cu:32-290): the decode route needs the single-pass activation;
    ggml_mul_mat_a8 on Q4_K / Q8_0 / Q6_K needs the batched path's scratch for one matrix."""
    for m, k in ((1, 256), (8, 4096), (33, 5120)):
        for qtype in O.WEIGHT_TYPES:
            assert kai.kai_ggml_a8_workspace(qtype, 64, k, m, 0) == O.activation_bytes(m, k)
        for qtype in (O.Q4_0, O.Q2_K):
            assert kai.kai_ggml_a8_workspace(qtype, 64, k, m, 1) == O.activation_bytes(m, k)
    a256 = lambda b: (b + 255) // 256 * 256
    for qtype in (O.Q4_K, O.Q8_0, O.Q6_K):
        for m in (9, 16, 17, 80):
            arr = lambda t, v: (t * 1)(v)
            if m <= 16:  # the same small-M images and partial sums as the fused batched entry
                want = kai.kai_fused_mmq_workspace(0, arr(ctypes.c_int, qtype), arr(ctypes.c_int64, 5120), 1, 4096, m, 0)
            else:  # the int8 kernels' plane (the fused entry's fp16 GEMM takes no legacy activation)
                want = a256(4 * m) + a256(_plane_bytes(m, 4096))
            assert kai.kai_ggml_a8_workspace(qtype, 5120, 4096, m, 1) == want > 0
        assert kai.kai_ggml_a8_workspace(qtype, 5120, 4096, 1, 1) > O.activation_bytes(1, 4096)
    assert kai.kai_ggml_a8_workspace(O.IQ3_S, 64, 256, 9, 1) == 0
    assert b"no IQ3_S kernel" in kai.current_direct_error()
    assert kai.kai_ggml_a8_workspace(O.Q4_K, 66, 256, 9, 1) > 0        # planes route: any rows
    assert kai.kai_ggml_a8_workspace(O.Q4_0, 66, 256, 9, 1) > 0        # decode route: any rows
    assert kai.kai_ggml_a8_workspace(O.Q8_0, 64, 32800, 1, 0) == 0     # k <= 32768
    assert kai.kai_ggml_a8_workspace(O.Q8_0, 64, 48, 0, 0) == 0        # no rows
    dummy = ctypes.c_void_p(16)
    need = kai.kai_ggml_a8_workspace(O.Q4_K, 64, 256, 3, 0)
    assert kai.kai_ggml_mul_mat_vec_a8(None, O.Q4_K, 64, dummy, 0, 3, 256, 256, dummy, 0, dummy, need, 0) == -1
    assert kai.kai_ggml_mul_mat_vec_a8(dummy, O.Q4_K, 64, dummy, 0, 3, 256, 128, dummy, 0, dummy, need, 0) == -1
    assert kai.kai_ggml_mul_mat_vec_a8(dummy, O.Q4_K, 64, dummy, 0, 3, 256, 256, dummy, 0, dummy, need - 1, 0) == -1
    assert b"smaller than kai_ggml_a8_workspace" in kai.current_direct_error()
    assert kai.kai_ggml_mul_mat_a8(dummy, O.IQ3_S, 64, dummy, 0, 3, 256, 256, dummy, 0, dummy, 1 << 20, 0) == -1
    assert kai.kai_ggml_quantize_q8_1(dummy, 0, 1, 60, 64, dummy, 0) == -1    # k % 32
    assert kai.kai_ggml_quantize_q8_1(dummy, 0, 1, 64, 32, dummy, 0) == -1    # stride < k
