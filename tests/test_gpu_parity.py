"""Parity of the gfx950 kernels with the CPU oracle, called through the C ABI.

Bars: activation bytes bit-exact (the decode path's Q8_1 blocks, and the batched path's
GGML MMQ planes read back from the scratch); GEMV/GEMM outputs within 1e-3 normwise
max-rel (max|y - ref| / max|ref| per activation row) of the oracle's FP64 result for F32
output, and within 2^-8 for BF16 output (bf16 keeps 8 significant bits, so rounding alone
reaches 2^-9 of max|y|, and up to 2^-8 where max|y| sits just above a power of two). Up to 8 rows the reference is the decode arithmetic
(oracle_prepare + oracle_mul_mat); above 8 rows it is the batched path's
(oracle_prepare_mmq + oracle_mul_mat_mmq, O.mmq_reference).
"""
import ctypes

import numpy as np
import pytest
import torch

import _oracle as O

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-3
TOL_BF16 = 2.0 ** -8
DEV = "cuda:0"


def _stream():
    return torch.cuda.current_stream().cuda_stream


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def gpu_prepare(kai, x_dev, two_pass=0):
    m, k = x_dev.shape
    code = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[x_dev.dtype]
    act = torch.empty(kai.kai_fused_activation_bytes(m, k, two_pass), dtype=torch.uint8, device=DEV)
    st = kai.kai_fused_prepare(x_dev.data_ptr(), code, m, k, x_dev.stride(0), act.data_ptr(), two_pass, _stream())
    assert st == 0, kai.current_direct_error()
    torch.cuda.synchronize()
    return act


def used_bytes(buf, m, k, two_pass):
    """The defined regions of an activation buffer (padding between passes is not written)."""
    nb = k // 32
    pass_bytes = (m * nb * 36 + 255) // 256 * 256
    parts = [buf[:m * nb * 36]]
    if two_pass:
        parts.append(buf[pass_bytes:pass_bytes + m * nb * 36])
    off = pass_bytes * (2 if two_pass else 1)
    parts.append(buf[off:off + 4 * m])
    return np.concatenate(parts)


# ----------------------------------------------------------------- Q8_1 preparation

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,k", [(1, 2048), (3, 5120), (8, 17408), (16, 160), (33, 4096)])
@pytest.mark.parametrize("two_pass", [0, 1])
def test_prepare_bit_exact(kai, dtype, m, k, two_pass):
    print(f"prepare dtype={dtype} m={m} k={k} two_pass={two_pass}", flush=True)
    rng = np.random.default_rng(m * 7 + k)
    x = (rng.standard_normal((m, k)) * rng.uniform(1e-2, 1e2, (m, 1))).astype(np.float32)
    x_dev = to_dev(x).to(dtype)
    act = gpu_prepare(kai, x_dev, two_pass).cpu().numpy()
    if dtype == torch.bfloat16:
        ref = O.prepare(x_dev.view(torch.int16).cpu().numpy().view(np.uint16), two_pass, dtype_code=1)
    else:
        ref = O.prepare(x_dev.cpu().numpy(), two_pass)
    assert np.array_equal(used_bytes(act, m, k, two_pass), used_bytes(ref, m, k, two_pass))


def test_prepare_special_rows_and_stride(kai):
    print("prepare special rows", flush=True)
    k = 256
    x = np.random.default_rng(9).standard_normal((6, k + 64)).astype(np.float32)
    x[0] = 0.0
    x[1, :] = 0.0
    x[1, 7] = 1e-41          # subnormal row maximum
    x[2] *= 1e30             # huge row
    x[3, :32] = 0.0          # a zero block inside a live row
    x[4, 100] = 2.0 ** -126  # tiny but normal values
    x[5] *= 1e-30
    full = to_dev(x)
    view = full[:, :k]       # row stride k + 64
    act = gpu_prepare(kai, view).cpu().numpy()
    ref = O.prepare(np.ascontiguousarray(x[:, :k]))
    assert np.array_equal(used_bytes(act, 6, k, 0), used_bytes(ref, 6, k, 0))


# 32 fp16 values (row maximum 166.4, so the row scale is 1/2) whose block sum term
# d * sum(q) = 0.6550197 * 381 rounds in fp32 to exactly 249.5625, half-way between
# two fp16 values: round-to-even gives 249.5; rounding the exact product once gives
# 249.625. The reference rounds to fp32 first (kai_dual_mmvq.cuh:232).
TIE_BLOCK_F16 = [22511, 51058, 21691, 20463, 18037, 20018, 19290, 22151, 21870, 18441, 48960, 54996,
                 55402, 21306, 22255, 50731, 51473, 18990, 21410, 52474, 16546, 19595, 21490, 21887,
                 20412, 20406, 53101, 19193, 55603, 53311, 18646, 20882]


def test_prepare_fp16_sum_tie_rounds_via_fp32(kai):
    x = np.array(TIE_BLOCK_F16, dtype=np.uint16).view(np.float16).reshape(1, 32)
    act = gpu_prepare(kai, to_dev(x)).cpu().numpy()
    ref = O.prepare(x)
    assert ref[2:4].view(np.float16)[0] == np.float16(249.5)
    assert np.array_equal(used_bytes(act, 1, 32, 0), used_bytes(ref, 1, 32, 0))


# ----------------------------------------------------------------- GEMV (kai_fused_mmvq)

SHAPES = {O.Q8_0: (300, 1024), O.Q4_0: (300, 2048), O.Q4_K: (300, 1280), O.Q6_K: (300, 1536),
          O.Q2_K: (300, 1024), O.IQ3_S: (300, 1280)}


def gpu_mmvq(kai, qtype, w_dev, n, k, act, m, two_pass=0, bf16=False, stride=None, offset=0, out=None):
    stride = stride or n
    if out is None:
        out = torch.full((m, stride), float("nan"), dtype=torch.bfloat16 if bf16 else torch.float32, device=DEV)
    st = kai.kai_fused_mmvq(w_dev.data_ptr(), qtype, n, k, m, act.data_ptr(), two_pass,
                            out.data_ptr() + offset * out.element_size(), 1 if bf16 else 0, stride, _stream())
    assert st == 0, kai.current_direct_error()
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("qtype", O.WEIGHT_TYPES, ids=lambda t: O.NAMES[t])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("weights", ["random", "quantized"])
def test_mmvq_parity_f32(kai, qtype, m, weights):
    print(f"mmvq {O.NAMES[qtype]} m={m} {weights}", flush=True)
    n, k = SHAPES[qtype]
    rng = np.random.default_rng(100 * qtype + m)
    if weights == "random":
        w = O.random_blocks(qtype, n, k, rng)
    else:
        from kaillm_amd.formats import quantize
        w = quantize(rng.normal(0, 0.02, (n, k)).astype(np.float32), qtype)
    x = rng.standard_normal((m, k)).astype(np.float16)
    act = gpu_prepare(kai, to_dev(x))
    out = gpu_mmvq(kai, qtype, to_dev(w), n, k, act, m).cpu().numpy()
    ref = O.mul_mat(qtype, w, k, O.prepare(x), m)
    err = O.normwise_rel(out, ref)
    print(f"  normwise rel err {err:.3e}")
    assert err <= TOL_F32


@pytest.mark.parametrize("qtype", O.WEIGHT_TYPES, ids=lambda t: O.NAMES[t])
@pytest.mark.parametrize("m", [1, 4, 7])
def test_mmvq_bf16_two_pass_and_merged_stride(kai, qtype, m):
    print(f"mmvq bf16/two-pass/stride {O.NAMES[qtype]} m={m}", flush=True)
    n, k = SHAPES[qtype]
    rng = np.random.default_rng(7 * qtype + m)
    w = O.random_blocks(qtype, n, k, rng)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w_dev = to_dev(w)
    for two_pass in (0, 1):
        act = gpu_prepare(kai, to_dev(x), two_pass)
        ref = O.mul_mat(qtype, w, k, O.prepare(x, two_pass), m, two_pass)
        # merged projection: this matrix owns columns [37, 37 + n) of a [m, n + 50] output
        out = gpu_mmvq(kai, qtype, w_dev, n, k, act, m, two_pass, bf16=True, stride=n + 50, offset=37)
        got = out.float().cpu().numpy()
        assert np.isnan(got[:, :37]).all() and np.isnan(got[:, 37 + n:]).all()  # neighbours untouched
        assert O.normwise_rel(got[:, 37:37 + n], ref) <= TOL_BF16
        out32 = gpu_mmvq(kai, qtype, w_dev, n, k, act, m, two_pass).cpu().numpy()
        assert O.normwise_rel(out32, ref) <= TOL_F32


def test_two_pass_is_closer_to_float_activations(kai):
    """Two passes carry ~16-bit activations, so the result moves toward W @ x."""
    rng = np.random.default_rng(5)
    n, k, m = 256, 2048, 2
    w = O.random_blocks(O.Q8_0, n, k, rng)
    x = rng.standard_normal((m, k)).astype(np.float32)
    dense = x.astype(np.float64) @ O.dequantize(O.Q8_0, w, k).astype(np.float64).T
    w_dev = to_dev(w)
    errs = []
    for two_pass in (0, 1):
        out = gpu_mmvq(kai, O.Q8_0, w_dev, n, k, gpu_prepare(kai, to_dev(x), two_pass), m, two_pass)
        errs.append(O.normwise_rel(out.cpu().numpy(), dense))
    assert errs[1] < errs[0] / 10


# ----------------------------------------------------------------- batched group (kai_fused_mmq_run)

def gpu_mmq(kai, mats, x_dev, bf16=False, stride=0, return_scratch=False):
    m, k = x_dev.shape
    count = len(mats)
    types = (ctypes.c_int * count)(*[t for t, _, _ in mats])
    rows = (ctypes.c_int64 * count)(*[w.shape[0] for _, w, _ in mats])
    ptrs = (ctypes.c_void_p * count)(*[wd.data_ptr() for _, _, wd in mats])
    size = kai.kai_fused_mmq_workspace(0, types, rows, count, k, m, 0 if bf16 else 1)
    assert size > 0, kai.current_direct_error()
    total = sum(w.shape[0] for _, w, _ in mats)
    ld = stride or total
    out = torch.full((m, ld), float("nan"), dtype=torch.bfloat16 if bf16 else torch.float32, device=DEV)
    scratch = torch.empty(size, dtype=torch.uint8, device=DEV)
    code = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[x_dev.dtype]
    st = kai.kai_fused_mmq_run(ptrs, types, rows, count, x_dev.data_ptr(), code, x_dev.stride(0), k, m,
                               out.data_ptr(), 1 if bf16 else 0, stride, scratch.data_ptr(), size, 0, _stream())
    assert st == 0, kai.current_direct_error()
    torch.cuda.synchronize()
    return (out, scratch) if return_scratch else out


def batched_ref(mats, x, dtype_code=None, threads=8):
    """The batched path's result for a group: each matrix on its layout's plane."""
    return np.concatenate([O.mmq_reference(t, w, x, dtype_code, threads) for t, w, *_ in mats], axis=1)


def host_bits(x_dev):
    """x as the oracle takes it: float32/float16 arrays, bf16 as uint16 bits (code 1)."""
    if x_dev.dtype == torch.bfloat16:
        return x_dev.view(torch.int16).cpu().numpy().view(np.uint16), 1
    return x_dev.cpu().numpy(), None


def plane_offsets(m, k, layouts):
    """Scratch offsets of kai_fused_mmq_run: [inverse][D4][DS4][D2S6]..., each a plane, or
    for up to 16 rows the small-M image; above 16 rows (every format of these tests on the fp16
    GEMM) each layout's fp16 image as (codes, mins) offsets."""
    a256 = lambda b: (b + 255) // 256 * 256
    off = a256(4 * m)
    out = {}
    if m <= 16:
        for l in (O.D4, O.DS4, O.D2S6):
            if l in layouts:
                out[l] = off
                off += a256(image_bytes(l, k))
        return out
    for l in (O.D4, O.DS4, O.D2S6):
        if l in layouts:
            codes, mins = (a256(len(part)) for part in h_image_parts(None, l, m, k))
            out[l] = (off, off + codes)
            off += codes + mins
    return out


def h_image_parts(plane, layout, m, k):
    """The fp16 GEMM's activation image (codes, min-pass sums as bytes) that the preparation
    writes above 16 rows, re-laid in numpy from the oracle's plane [K/128][m][144]: rows padded
    to a multiple of 32 and K to 256; codes fp16 [K/16][mpad][16] = half(float32(d * q)) with d
    the scale the block dot takes (D4: the fp32 d, DS4 / D2S6: the stored fp16 d); mins (none
    for D4) per superblock, DS4 fp16 [..][mpad][32] = [S | Xhi | Xlo | 0] (S the 8 stored sums,
    X = half(d) * sum(q) exact, hi = half(X), lo = half(X - hi)), D2S6 [..][mpad][64] =
    [Shi | Slo | Xhi | Xlo] per 16-value group. plane None: zero bytes of each size."""
    mpad, kpad, sbs = (m + 31) // 32 * 32, (k + 255) // 256 * 256, (k + 255) // 256
    codes = np.zeros((kpad // 16, mpad, 16), np.float16)
    mins = np.zeros((sbs, mpad, 0 if layout == O.D4 else 32 if layout == O.DS4 else 64), np.float16)
    if plane is None:
        return codes.view(np.uint8).reshape(-1), mins.view(np.uint8).reshape(-1)
    f32, f16 = np.float32, np.float16
    q, d, sums = O.split_plane(plane, layout)  # q [m, Kpad512], d per 32 (D2S6: 64), sums
    g = 64 if layout == O.D2S6 else 32
    dk = np.repeat(d[:, :kpad // g].astype(f32), g, axis=1)
    if layout != O.D4:
        dk = dk.astype(f16).astype(f32)
    codes[:, :m, :] = (dk * q[:, :kpad].astype(f32)).astype(f16).reshape(m, kpad // 16, 16).transpose(1, 0, 2)

    def parts(v):
        hi = v.astype(f16)
        return hi, (v - hi.astype(f32)).astype(f16)

    if layout == O.DS4:
        dh = d[:, :8 * sbs].astype(f32).astype(f16).astype(f32)
        x = dh * q[:, :256 * sbs].astype(np.int64).reshape(m, 8 * sbs, 32).sum(axis=2).astype(f32)
        xhi, xlo = parts(x)
        mins[:, :m, 0:8] = sums[:, :8 * sbs].astype(f16).reshape(m, sbs, 8).transpose(1, 0, 2)
        mins[:, :m, 8:16] = xhi.reshape(m, sbs, 8).transpose(1, 0, 2)
        mins[:, :m, 16:24] = xlo.reshape(m, sbs, 8).transpose(1, 0, 2)
    elif layout == O.D2S6:
        s16 = sums[:, :16 * sbs].astype(f32).copy()  # NaN where the plane stores none
        d64 = np.repeat(d[:, :4 * sbs].astype(f32), 4, axis=1)
        dh = d64.astype(f16).astype(f32)
        qs = q[:, :256 * sbs].astype(np.int64).reshape(m, 16 * sbs, 16).sum(axis=2).astype(f32)
        s16 = np.where(np.isnan(s16), d64 * qs, s16).astype(f32)
        for at, v in ((0, s16), (32, dh * qs)):
            hi, lo = parts(v)
            mins[:, :m, at:at + 16] = hi.reshape(m, sbs, 16).transpose(1, 0, 2)
            mins[:, :m, at + 16:at + 32] = lo.reshape(m, sbs, 16).transpose(1, 0, 2)
    return codes.view(np.uint8).reshape(-1), mins.view(np.uint8).reshape(-1)


def image_bytes(layout, k):
    return (k + 255) // 256 * (4608 if layout == O.D4 else 5632)


def small_m_image(plane, layout, k):
    """The small-M image a plane [K/128][m][144] re-lays as (the layout the preparation writes
    for up to 16 rows): per 256-value step, codes [8][16][32] with octet o of row r at byte
    8 * (o ^ ((r >> 2) & 3)), d8 [8][16] fp32, then the terms: DS4 the stored fp16 sums and
    d8 * sum(codes), D2S6 one per 16 values (stored sums, d8 * sum(codes) past value 96 of 128)."""
    nb, m, _ = plane.shape
    steps = (k + 255) // 256
    codes = np.zeros((steps, 8, 16, 4, 8), np.uint8)
    d8 = np.zeros((steps, 8, 16), np.float32)
    terms = np.zeros((steps, 16, 16), np.float32)
    for s in range(steps):
        for b in range(8):
            blk, sub = 2 * s + b // 4, b % 4
            hdr = plane[blk, :, :16]
            q = plane[blk, :, 16 + 32 * sub:48 + 32 * sub]
            qs = q.view(np.int8).astype(np.int64)
            for r in range(m):
                for o in range(4):
                    codes[s, b, r, o ^ ((r >> 2) & 3)] = q[r, 8 * o:8 * o + 8]
            if layout == O.D4:
                d8[s, b, :m] = hdr.copy().view(np.float32)[:, sub]
            elif layout == O.DS4:
                halves = hdr.copy().view(np.float16).astype(np.float32)
                d8[s, b, :m] = halves[:, 2 * sub]
                terms[s, b, :m] = halves[:, 2 * sub + 1]
                terms[s, 8 + b, :m] = d8[s, b, :m] * qs.sum(axis=1).astype(np.float32)
            else:
                halves = hdr.copy().view(np.float16).astype(np.float32)
                d8[s, b, :m] = halves[:, sub >> 1]
                for g in range(2):
                    if sub < 3:
                        terms[s, 2 * b + g, :m] = halves[:, 2 + 2 * sub + g]
                    else:
                        terms[s, 2 * b + g, :m] = d8[s, b, :m] * qs[:, 16 * g:16 * g + 16].sum(axis=1).astype(np.float32)
    nterm = 0 if layout == O.D4 else 16
    parts = [codes.reshape(steps, -1), d8.view(np.uint8).reshape(steps, -1),
             terms[:, :nterm].view(np.uint8).reshape(steps, -1)]
    return np.concatenate(parts, axis=1).reshape(-1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,k", [(9, 256), (12, 2080), (16, 4096), (17, 1056), (80, 5120), (130, 2080), (300, 2080),
                                 (1030, 4096), (260, 17408), (256, 32768)])
def test_mmq_planes_bit_exact(kai, dtype, m, k):
    """The batched path's activation (row scale + GGML MMQ quantisation into D4, DS4 and
    D2S6 planes, K padded to 512) read back from the scratch equals the oracle's bytes, in the
    form the GEMMs read it: up to 16 rows the small-M images of the planes, above 16 rows the
    fp16 GEMM's images (h_image_parts); from 256 rows (image rows) a workgroup walks a whole row,
    converting up to 12 chunks from the values of its row-maximum pass (K = 32768: 16 chunks, the
    last 4 read again)."""
    print(f"mmq planes dtype={dtype} m={m} k={k}", flush=True)
    rng = np.random.default_rng(m + k)
    kq = k if k % 256 == 0 else None
    types = [O.Q8_0, O.Q4_0] + ([O.Q2_K] if kq else [])
    mats = []
    # the product check divides each row's error by its largest output: over a thousand rows of
    # 12 outputs per matrix some row's largest is small enough for the fp16 GEMM's operand
    # roundings (~4e-4 of a typical row's largest output) to pass 1e-3, so many rows get 64
    n = 12 if m < 256 else 64
    for qtype in types:
        w = O.random_blocks(qtype, n, k, rng)
        mats.append((qtype, w, to_dev(w)))
    x = (rng.standard_normal((m, k)) * rng.uniform(1e-2, 1e2, (m, 1))).astype(np.float32)
    x[0] = 0.0
    x[1, :64] = 0.0
    x[2, 5] = np.float32(np.finfo(np.float32).tiny) if dtype == torch.float32 else x[2, 5]
    x_dev = to_dev(x).to(dtype)
    out, scratch = gpu_mmq(kai, mats, x_dev, return_scratch=True)
    xs, code = host_bits(x_dev)
    layouts = {O.mmq_layout(t) for t in types}
    offs = plane_offsets(m, k, layouts)
    got = scratch.cpu().numpy()
    for layout in layouts:
        plane, inverse = O.prepare_mmq(xs, layout, code)
        if m <= 16:
            want = small_m_image(plane, layout, k)
            assert np.array_equal(got[offs[layout]:offs[layout] + want.size], want), O.LAYOUT_NAMES[layout]
        else:
            for name, part, at in zip(("codes", "mins"), h_image_parts(plane, layout, m, k), offs[layout]):
                assert np.array_equal(got[at:at + part.size], part), (O.LAYOUT_NAMES[layout], name)
        assert np.array_equal(got[:4 * m].view(np.float32), inverse)
    assert O.normwise_rel(out.cpu().numpy(), batched_ref(mats, xs, code)) <= TOL_F32


@pytest.mark.parametrize("m", [9, 16, 17, 40, 80])
def test_mmq_group_parity(kai, m):
    print(f"mmq group m={m}", flush=True)
    rng = np.random.default_rng(m)
    k = 1024
    mats = []
    for qtype, n in ((O.Q4_K, 96), (O.Q6_K, 64), (O.Q8_0, 36)):
        w = O.random_blocks(qtype, n, k, rng)
        mats.append((qtype, w, to_dev(w)))
    x = rng.standard_normal((m, k)).astype(np.float16)
    ref = batched_ref(mats, x)
    out = gpu_mmq(kai, mats, to_dev(x)).cpu().numpy()
    assert O.normwise_rel(out, ref) <= TOL_F32
    outb = gpu_mmq(kai, mats, to_dev(x), bf16=True, stride=ref.shape[1] + 8).float().cpu().numpy()
    assert O.normwise_rel(outb[:, :ref.shape[1]], ref) <= TOL_BF16
    assert np.isnan(outb[:, ref.shape[1]:]).all()


ALL_TYPES = [O.Q8_0, O.Q4_0, O.Q4_K, O.Q6_K, O.Q2_K, O.IQ3_S]


@pytest.mark.parametrize("qtype", ALL_TYPES)
@pytest.mark.parametrize("m,k,n", [(9, 768, 200), (24, 512, 64), (130, 256, 136), (300, 768, 72),
                                   (20, 1056, 96)])
def test_mmq_each_type(kai, qtype, m, k, n):
    """Every format through the batched path: partial weight tiles (n % 128), several
    activation tiles (m > 128), one K step (k = 256), and k % 256 != 0 (row-block path)."""
    if k % O.BLOCK[qtype][0]:
        pytest.skip("k not a multiple of this format's block")
    print(f"mmq type={qtype} m={m} k={k} n={n}", flush=True)
    rng = np.random.default_rng(qtype * 1000 + m + k)
    w = O.random_blocks(qtype, n, k, rng)
    x = rng.standard_normal((m, k)).astype(np.float32)
    ref = O.mmq_reference(qtype, w, x)
    out = gpu_mmq(kai, [(qtype, w, to_dev(w))], to_dev(x)).cpu().numpy()
    assert O.normwise_rel(out, ref) <= TOL_F32


PAIRED = [(O.Q4_K, 5, 768, 200), (O.Q6_K, 8, 1280, 136), (O.Q2_K, 6, 768, 200), (O.Q8_0, 8, 16384, 72),
          (O.Q4_0, 8, 16384, 40), (O.IQ3_S, 7, 18432, 72)]


@pytest.mark.parametrize("qtype,m,k,n", PAIRED, ids=lambda v: str(v))
@pytest.mark.parametrize("bf16", [False, True])
def test_mmq_paired_tile(kai, qtype, m, k, n, bf16):
    """Up to 8 rows on int8 MFMA (two 32-value blocks per MFMA), reached through
    kai_fused_mmvq above the GEMV's row limit: on these few row sets the persistent paired
    GEMM (one workgroup per set; long K in chunks), ragged row sets, strided bf16 output."""
    print(f"mmq paired {O.NAMES[qtype]} m={m} k={k} n={n} bf16={bf16}", flush=True)
    rng = np.random.default_rng(qtype * 100 + m)
    w = O.random_blocks(qtype, n, k, rng)
    x = rng.standard_normal((m, k)).astype(np.float16)
    act = gpu_prepare(kai, to_dev(x))
    out = gpu_mmvq(kai, qtype, to_dev(w), n, k, act, m, bf16=bf16, stride=n + 8 if bf16 else None)
    ref = O.mul_mat(qtype, w, k, O.prepare(x), m)
    got = out.float().cpu().numpy()
    assert O.normwise_rel(got[:, :n], ref) <= (TOL_BF16 if bf16 else TOL_F32)
    if bf16:
        assert np.isnan(got[:, n:]).all()


# Above the GEMV's rows kai_fused_mmvq runs the persistent paired GEMM where whole 16-row sets
# per workgroup keep the workgroups busy (kai_mmqd.cuh mmqd_suits: under 256 row sets, or
# at least 90 % busy), the tiled paired kernel elsewhere (kai_abi.hip run_decode).
# 1000 row sets on 256 CUs: workgroups of 3 and of 4 sets; k = 61 K steps, staged in two
# chunks of 31 (rounded up to 32 by a zero step) and 30; 15995 rows: the last set ragged.
PERSISTENT = [(O.Q4_K, 7), (O.Q6_K, 5), (O.Q2_K, 8), (O.IQ3_S, 6), (O.Q8_0, 8), (O.Q4_0, 7)]


@pytest.mark.parametrize("qtype,m", PERSISTENT, ids=lambda v: str(v))
def test_persistent_decode_chunks_and_ragged_sets(kai, qtype, m):
    n, k = 15995, 61 * 256
    print(f"persistent decode {O.NAMES[qtype]} m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(qtype * 10 + m)
    w = O.random_blocks(qtype, n, k, rng)
    x = rng.standard_normal((m, k)).astype(np.float16)
    act = gpu_prepare(kai, to_dev(x))
    w_dev = to_dev(w)
    out = gpu_mmvq(kai, qtype, w_dev, n, k, act, m)
    again = gpu_mmvq(kai, qtype, w_dev, n, k, act, m)
    assert torch.equal(out, again), "the slot sums are added in a fixed order"
    ref = O.mul_mat(qtype, w, k, O.prepare(x), m, threads=16)
    assert O.normwise_rel(out.cpu().numpy(), ref) <= TOL_F32


# C3 shapes whose row sets do not balance over the CUs (448 and 320 sets) stay on the tiled
# paired kernel: qkv at 8 rows, o_proj at 5, down at 4 (K split over the waves).
TILED = [(O.Q4_K, 8, 7168, 5120), (O.Q6_K, 5, 5120, 6144), (O.Q6_K, 4, 5120, 17408)]


@pytest.mark.parametrize("qtype,m,n,k", TILED, ids=lambda v: str(v))
def test_tiled_paired_decode_full_shapes(kai, qtype, m, n, k):
    print(f"tiled paired {O.NAMES[qtype]} m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(n + k + m)
    w = O.random_blocks(qtype, n, k, rng)
    x = rng.standard_normal((m, k)).astype(np.float16)
    act = gpu_prepare(kai, to_dev(x))
    out = gpu_mmvq(kai, qtype, to_dev(w), n, k, act, m, bf16=True, stride=n + 8).float().cpu().numpy()
    ref = O.mul_mat(qtype, w, k, O.prepare(x), m, threads=16)
    assert O.normwise_rel(out[:, :n], ref) <= TOL_BF16
    assert np.isnan(out[:, n:]).all()


# The tiled paired kernel on fewer workgroups than about 2 per CU, with K of 32 steps or
# more, splits K across workgroups (pieces of whole K turns); the last piece to arrive adds
# all pieces in K order, so repeated calls agree bit for bit, and each call leaves its
# arrival counts at zero for the next. 321 row sets (the last ragged), 320, 448.
PIECES = [(O.Q6_K, 8, 5128, 17408), (O.IQ3_S, 6, 5120, 17408), (O.Q4_K, 7, 7168, 8192), (O.Q6_K, 5, 5120, 12288)]


@pytest.mark.parametrize("qtype,m,n,k", PIECES, ids=lambda v: str(v))
def test_tiled_paired_k_pieces(kai, qtype, m, n, k):
    print(f"tiled paired K pieces {O.NAMES[qtype]} m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(7 * n + k + m)
    w = O.random_blocks(qtype, n, k, rng)
    x = rng.standard_normal((m, k)).astype(np.float16)
    act = gpu_prepare(kai, to_dev(x))
    w_dev = to_dev(w)
    out = gpu_mmvq(kai, qtype, w_dev, n, k, act, m)
    # a smaller product in between (fewer rows and columns, same slots)
    small_n, small_k = 2048, 2560
    w2 = O.random_blocks(qtype, small_n, small_k, rng)
    x2 = rng.standard_normal((5, small_k)).astype(np.float16)
    act2 = gpu_prepare(kai, to_dev(x2))
    out2 = gpu_mmvq(kai, qtype, to_dev(w2), small_n, small_k, act2, 5)
    again = [gpu_mmvq(kai, qtype, w_dev, n, k, act, m) for _ in range(5)]
    for a in again:
        assert torch.equal(out, a), "K pieces are added in a fixed order"
    ref = O.mul_mat(qtype, w, k, O.prepare(x), m, threads=16)
    assert O.normwise_rel(out.cpu().numpy(), ref) <= TOL_F32
    ref2 = O.mul_mat(qtype, w2, small_k, O.prepare(x2), 5)
    assert O.normwise_rel(out2.cpu().numpy(), ref2) <= TOL_F32


@pytest.mark.parametrize("qtype", [O.Q4_K, O.Q6_K, O.IQ3_S])
def test_mmq_prefill_shape(kai, qtype):
    """A prefill-sized call (m = 512) on a full-width weight, bf16 activations."""
    m, n, k = 512, 1024, 2048
    print(f"mmq prefill type={qtype} m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(qtype + 5)
    w = O.random_blocks(qtype, n, k, rng)
    x_dev = to_dev(rng.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16)
    ref = O.mmq_reference(qtype, w, host_bits(x_dev)[0], 1, threads=16)
    out = gpu_mmq(kai, [(qtype, w, to_dev(w))], x_dev).cpu().numpy()
    assert O.normwise_rel(out, ref) <= TOL_F32


# Prefill-sized products: partial tiles in both dimensions (the last weight tile a 4-row
# group, the last activation tile 40 rows), one to eight superblocks, wire blocks from random
# bytes and from quantised N(0, 0.02) weights (whose min terms cancel: the product is only as
# close to the reference as the fp16 roundings of the weight scales are repeated).
@pytest.mark.parametrize("qtype", [O.Q4_K, O.Q2_K], ids=lambda t: O.NAMES[t])
@pytest.mark.parametrize("weights", ["random", "quantized"])
@pytest.mark.parametrize("m,n,k", [(1000, 4100, 256), (960, 4096, 1280), (1100, 3840, 2048)])
def test_batched_prefill_tiles(kai, qtype, weights, m, n, k):
    print(f"batched prefill tiles {O.NAMES[qtype]} {weights} m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(qtype + m + n + k)
    if weights == "random":
        w = O.random_blocks(qtype, n, k, rng)
    else:
        from kaillm_amd.formats import quantize
        w = quantize(rng.normal(0.0, 0.02, (n, k)).astype(np.float32), qtype)
    x = rng.standard_normal((m, k)).astype(np.float32)
    ref = O.mmq_reference(qtype, w, x, threads=16)
    out = gpu_mmq(kai, [(qtype, w, to_dev(w))], to_dev(x)).cpu().numpy()
    err = O.normwise_rel(out, ref)
    print(f"  normwise rel err {err:.3e}")
    assert err <= TOL_F32


# More tiles than CUs with a short last round: the tiles of a rectangle at the output's end run
# in K pieces whose sums a second kernel adds into that rectangle, in place of an unsplit plan's
# short round or a K split's extra rounds; the other tiles run whole. Rectangles (rows r0.., weight
# rows c0..): Q4_K on 256 x 128 tiles, 2 x 141 tiles, the last 26 in 4 pieces of one 256-value
# step (the last tile 80 wide); Q4_0 at 40 rows on 128 x 96 tiles and IQ3_S and Q2_K at 120 rows
# on 128 x 128 tiles, 258 tiles, the last 2 (232 columns, the last tile 104 wide) in 4 pieces
# over every row; two activation tiles high: Q4_K and Q2_K, 14 x 20 tiles of 256 x 128, the last
# 12 of the last 2 (412 rows, the last tile 68 wide) in 2 pieces.
TAIL = [(O.Q4_K, 300, 18000, 1024, 256, 14720), (O.Q4_0, 40, 33000, 1024, 0, 32768),
        (O.IQ3_S, 120, 33000, 1024, 0, 32768), (O.Q2_K, 120, 33000, 1024, 0, 32768),
        (O.Q4_K, 3484, 2500, 512, 3072, 1024), (O.Q2_K, 3484, 2500, 512, 3072, 1024)]


@pytest.mark.parametrize("qtype,m,n,k,r0,c0", TAIL, ids=[f"{O.NAMES[t]}-{m}x{n}x{k}" for t, m, n, k, _, _ in TAIL])
def test_batched_tail_tiles_in_k_pieces(kai, qtype, m, n, k, r0, c0):
    print(f"batched tail tiles {O.NAMES[qtype]} m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(qtype + m)
    w = O.random_blocks(qtype, n, k, rng)
    x = rng.standard_normal((m, k)).astype(np.float32)
    ref = O.mmq_reference(qtype, w, x, threads=16)
    mats = [(qtype, w, to_dev(w))]
    out = gpu_mmq(kai, mats, to_dev(x)).cpu().numpy()
    assert O.normwise_rel(out, ref) <= TOL_F32
    assert O.normwise_rel(out[r0:, c0:], ref[r0:, c0:]) <= TOL_F32
    assert O.normwise_rel(out[:, :c0], ref[:, :c0]) <= TOL_F32
    again = gpu_mmq(kai, mats, to_dev(x)).cpu().numpy()
    assert np.array_equal(out, again), "the pieces are added in a fixed order"
    outb = gpu_mmq(kai, mats, to_dev(x), bf16=True, stride=n + 3).float().cpu().numpy()
    # the same sums as the f32 output (checked above), rounded to nearest even once, pieces and
    # whole tiles alike (over thousands of rows some row's maximum sits just above a power of
    # two, where that rounding alone approaches TOL_BF16)
    assert np.array_equal(outb[:, :n], torch.from_numpy(out).to(torch.bfloat16).float().numpy())
    assert np.isnan(outb[:, n:]).all()


def test_batched_tail_in_a_group_with_unaligned_columns(kai):
    """A group whose first matrix has a tail of K pieces over 234 columns (33002 rows: 258
    tiles of 128, the last 2 in pieces) and whose second starts at an even but not 16-byte
    aligned column: the pieces' sums and their reduction take the element-wise paths. (Both
    Q4_0: random Q8_0 blocks give outputs several times larger, and two such columns would set
    each row's maximum, making the normwise bound a bound on single outputs.)"""
    print("batched tail in an unaligned group", flush=True)
    rng = np.random.default_rng(33002)
    m, k = 40, 1024
    w1 = O.random_blocks(O.Q4_0, 33002, k, rng)
    w2 = O.random_blocks(O.Q4_0, 2, k, rng)
    mats = [(O.Q4_0, w1, to_dev(w1)), (O.Q4_0, w2, to_dev(w2))]
    x = rng.standard_normal((m, k)).astype(np.float32)
    ref = batched_ref(mats, x, threads=16)
    out = gpu_mmq(kai, mats, to_dev(x)).cpu().numpy()
    assert O.normwise_rel(out, ref) <= TOL_F32
    assert O.normwise_rel(out[:, 32768:], ref[:, 32768:]) <= TOL_F32
    outb = gpu_mmq(kai, mats, to_dev(x), bf16=True, stride=33004 + 5).float().cpu().numpy()
    assert np.array_equal(outb[:, :33004], torch.from_numpy(out).to(torch.bfloat16).float().numpy())
    assert np.isnan(outb[:, 33004:]).all()


def test_batched_heavy_tailed_activations_bf16_out_and_stride(kai):
    """Activations spread over many binades (small-scale blocks beside large ones) and
    exact zeros; bf16 output into a wider matrix, the padding left untouched."""
    rng = np.random.default_rng(5)
    m, n, k = 960, 4096, 512
    w = O.random_blocks(O.Q4_K, n, k, rng)
    x = (rng.standard_normal((m, k)) * np.exp(rng.normal(0.0, 2.0, (m, k)))).astype(np.float32)
    x[3] = 0.0
    x[7, :512] = 0.0
    ref = O.mmq_reference(O.Q4_K, w, x, threads=16)
    out = gpu_mmq(kai, [(O.Q4_K, w, to_dev(w))], to_dev(x)).cpu().numpy()
    assert np.all(out[3] == 0.0)
    assert O.normwise_rel(out, ref) <= TOL_F32
    outb = gpu_mmq(kai, [(O.Q4_K, w, to_dev(w))], to_dev(x), bf16=True, stride=n + 12).float().cpu().numpy()
    assert O.normwise_rel(outb[:, :n], ref) <= TOL_BF16
    assert np.isnan(outb[:, n:]).all()


def test_batched_group_with_unaligned_columns(kai):
    """One group, one scratch, three layouts: Q4_K matrices first and last, a Q6_K between
    them, a Q4_K after a column offset of 2 mod 4 and a narrow Q4_K (n = 2 mod 4)."""
    rng = np.random.default_rng(11)
    m, k = 1000, 512
    mats = []
    for qtype, n in ((O.Q4_K, 4096), (O.Q6_K, 130), (O.Q4_K, 4096), (O.Q2_K, 126), (O.Q4_K, 4096)):
        w = O.random_blocks(qtype, n, k, rng)
        mats.append((qtype, w, to_dev(w)))
    x = rng.standard_normal((m, k)).astype(np.float16)
    ref = batched_ref(mats, x, threads=16)
    out = gpu_mmq(kai, mats, to_dev(x)).cpu().numpy()
    assert O.normwise_rel(out, ref) <= TOL_F32


# Small batches (9..16 rows): K split across the waves of a workgroup (small n), partial
# row tiles, one and an odd number of superblocks.
@pytest.mark.parametrize("qtype", [O.Q4_K, O.Q6_K, O.Q2_K], ids=lambda t: O.NAMES[t])
@pytest.mark.parametrize("weights", ["random", "quantized"])
@pytest.mark.parametrize("m,n,k", [(9, 1000, 256), (12, 200, 1280), (16, 4100, 2304), (13, 64, 5120)])
def test_batched_small_m(kai, qtype, weights, m, n, k):
    print(f"batched small m {O.NAMES[qtype]} m={m} n={n} k={k} {weights}", flush=True)
    rng = np.random.default_rng(m * 7 + n + k)
    if weights == "random":
        w = O.random_blocks(qtype, n, k, rng)
    else:
        from kaillm_amd.formats import quantize
        w = quantize(rng.normal(0.0, 0.02, (n, k)).astype(np.float32), qtype)
    x = rng.standard_normal((m, k)).astype(np.float16)
    ref = O.mmq_reference(qtype, w, x, threads=16)
    out = gpu_mmq(kai, [(qtype, w, to_dev(w))], to_dev(x)).cpu().numpy()
    err = O.normwise_rel(out, ref)
    print(f"  normwise rel err {err:.3e}")
    assert err <= TOL_F32


def test_batched_heavy_tailed_bf16_out_stride_and_group(kai):
    """Heavy-tailed activations, BF16 output into a wider merged tile, and a group of
    Q4_K and Q6_K matrices behind one preparation."""
    m, k = 15, 1536
    print(f"batched group m={m} k={k}", flush=True)
    rng = np.random.default_rng(77)
    mats = []
    for qtype, n in ((O.Q4_K, 520), (O.Q6_K, 72), (O.Q4_K, 36)):
        w = O.random_blocks(qtype, n, k, rng)
        mats.append((qtype, w, to_dev(w)))
    x = (rng.standard_t(2.0, (m, k)) * 3.0).astype(np.float32)
    ref = batched_ref(mats, x)
    out = gpu_mmq(kai, mats, to_dev(x)).cpu().numpy()
    assert O.normwise_rel(out, ref) <= TOL_F32
    outb = gpu_mmq(kai, mats, to_dev(x), bf16=True, stride=ref.shape[1] + 4).float().cpu().numpy()
    assert O.normwise_rel(outb[:, :ref.shape[1]], ref) <= TOL_BF16
    assert np.isnan(outb[:, ref.shape[1]:]).all()


# ----------------------------------------------------------------- full BASELINE shapes

FULL = [
    ("C1 Q8_0 2048x2048", O.Q8_0, 2048, 2048, 1),
    ("C2 Q4_0 gate/up", O.Q4_0, 16384, 2048, 8),
    ("C2 Q4_0 down", O.Q4_0, 2048, 8192, 4),
    ("C3 Q4_K gate/up", O.Q4_K, 34816, 5120, 1),
    ("C3 Q4_K gate/up b8", O.Q4_K, 34816, 5120, 8),
    ("C3 Q4_K qkv", O.Q4_K, 7168, 5120, 16),
    ("C3 Q6_K down", O.Q6_K, 5120, 17408, 2),
    ("C3 Q6_K o_proj", O.Q6_K, 5120, 6144, 8),
    ("C5 Q2_K gate/up", O.Q2_K, 34816, 5120, 1),
    ("C5 IQ3_S down", O.IQ3_S, 5120, 17408, 16),
]


@pytest.mark.parametrize("name,qtype,n,k,m", FULL, ids=[f[0] for f in FULL])
def test_full_size_configs(kai, name, qtype, n, k, m):
    print(f"full {name} m={m}", flush=True)
    rng = np.random.default_rng(n + k + m)
    w = O.random_blocks(qtype, n, k, rng)
    x = rng.standard_normal((m, k)).astype(np.float16)
    x_dev = to_dev(x)
    ref = O.mul_mat(qtype, w, k, O.prepare(x), m, threads=16) if m <= 8 else O.mmq_reference(qtype, w, x, threads=16)
    if m <= 8:
        out = gpu_mmvq(kai, qtype, to_dev(w), n, k, gpu_prepare(kai, x_dev), m)
    else:
        out = gpu_mmq(kai, [(qtype, w, to_dev(w))], x_dev)
    err = O.normwise_rel(out.cpu().numpy(), ref)
    print(f"  normwise rel err {err:.3e}")
    assert err <= TOL_F32


# ----------------------------------------------------------------- torch ops / apply()

def test_fused_projection_torch_ops(kai):
    from kaillm_amd.linear import GGUFLinearMethod, PackedGGUFLinear

    rng = np.random.default_rng(77)
    k = 1024
    parts_np = [(O.Q4_K, O.random_blocks(O.Q4_K, 128, k, rng)), (O.Q6_K, O.random_blocks(O.Q6_K, 64, k, rng))]
    layer = torch.nn.Module()
    layer.gguf_compact = torch.nn.ModuleList(
        [PackedGGUFLinear(to_dev(w), t, torch.bfloat16) for t, w in parts_np])
    method = GGUFLinearMethod()
    for m in (1, 3, 8, 12, 64):
        x = rng.standard_normal((m, k)).astype(np.float32)
        x_dev = to_dev(x).to(torch.bfloat16)
        xb = host_bits(x_dev)[0]
        if m <= 8:
            act = O.prepare(xb, dtype_code=1)
            ref = np.concatenate([O.mul_mat(t, w, k, act, m) for t, w in parts_np], axis=1)
        else:
            ref = batched_ref(parts_np, xb, 1)
        bias = torch.randn(ref.shape[1], device=DEV, dtype=torch.bfloat16)
        y = method.apply(layer, x_dev.reshape(1, m, k), bias)
        assert y.shape == (1, m, ref.shape[1]) and y.dtype == torch.bfloat16
        got = (y.float() - bias.float()).reshape(m, -1).cpu().numpy()
        assert O.normwise_rel(got, ref) <= 2 * TOL_BF16
