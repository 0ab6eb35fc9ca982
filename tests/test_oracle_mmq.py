"""Pin the oracle's batched path (kai_fused_mmq_run, more than 8 rows) before trusting it.

The activation side restates row_scale + quantize_scaled
(current_ggml_direct.cu:978-1092); the block arithmetic restates GGML MMQ. Pins here:
closed forms (power-of-two known answers where every rounding is exact, the per-64
scale of D2S6 against the per-32 scale of D4/DS4, reciprocal quantisation against the
decode path's division), invariants (power-of-two scaling, agreement of the row scale
with the decode preparation), special rows, the byte layout, and a second route through
every format: numpy float64 decoders of the weight bytes dotted with the dequantised
plane, which differs from the oracle only by the stored half sums of the min terms
(bounded exactly from the plane bytes).
"""
import numpy as np
import pytest

import _oracle as O

LAYOUT_OF = {O.Q8_0: O.D4, O.Q6_K: O.D4, O.IQ3_S: O.D4, O.Q4_0: O.DS4, O.Q4_K: O.DS4, O.Q2_K: O.D2S6}


def test_layout_per_type_and_plane_size():
    for t, l in LAYOUT_OF.items():
        assert O.mmq_layout(t) == l
    # K padded to 512 (MATRIX_ROW_PADDING), 128-value blocks of 144 bytes
    assert O.mmq_blocks128(5120) == 40 and O.mmq_blocks128(5121 - 1 + 4) == 44
    assert O.mmq_blocks128(96) == 4
    assert O.lib().oracle_mmq_plane_bytes(3, 1024) == 8 * 3 * 144


def _integer_row(rng, k, group, top=127):
    """Integers in [-top, top] with +-top in every group of `group` values."""
    v = rng.integers(-top, top + 1, k).astype(np.float32)
    for g in range(0, k, group):
        v[g + rng.integers(0, group)] = top * (1 if rng.integers(0, 2) else -1)
    return v


@pytest.mark.parametrize("layout", [O.D4, O.DS4, O.D2S6])
def test_known_answer_power_of_two_rows(layout):
    """Values c * q with q integer, |q| = 127 in every group and c a power of two: the row
    scale maps 127c to 127 (amax in [64, 128)), d_inv = 127/127 = 1, so q comes back
    exactly, d = 1, and every sum is the integer sum (exact in fp16 below 2048)."""
    rng = np.random.default_rng(1)
    m, k = 3, 1024
    g = 64 if layout == O.D2S6 else 32
    q = np.stack([_integer_row(rng, k, g) for _ in range(m)])
    x = q * np.float32(2.0 ** -3)
    x[1] *= np.float32(2.0 ** 20)
    plane, inverse = O.prepare_mmq(x, layout)
    gq, d, sums = O.split_plane(plane, layout)
    assert np.array_equal(gq[:, :k], q.astype(np.int8))
    assert np.array_equal(inverse, np.array([2.0 ** -3, 2.0 ** 17, 2.0 ** -3], dtype=np.float32))
    assert np.all(d[:, :k // g] == 1.0)
    if layout == O.DS4:
        assert np.array_equal(sums[:, :k // 32], q.reshape(m, -1, 32).sum(-1))
    if layout == O.D2S6:
        s16 = q.reshape(m, -1, 16).sum(-1).astype(np.float32)
        stored = sums[:, :k // 16].reshape(m, -1, 8)
        assert np.array_equal(stored[:, :, :6], s16.reshape(m, -1, 8)[:, :, :6])
        assert np.isnan(stored[:, :, 6:]).all()


def test_known_answer_group_max_64():
    """A group whose maximum is 64 (row maximum 127 elsewhere): d_inv = 127/64 = 1.984375 is
    exact, so q = roundf(v * 1.984375) and d = 1/1.984375 rounded once."""
    k = 64
    x = np.zeros((1, k), dtype=np.float32)
    x[0, 0] = 127.0
    x[0, 32:40] = [64, -64, 1, 2, 3, -5, 33, 63]
    plane, inverse = O.prepare_mmq(x, O.D4)
    q, d, _ = O.split_plane(plane, O.D4)
    assert inverse[0] == 1.0
    want = [127, -127, 2, 4, 6, -10, 65, 125]  # 33*1.984375 = 65.48 -> 65; 63*1.984375 = 125.02
    assert list(q[0, 32:40]) == want
    assert d[0, 1] == np.float32(1.0) / np.float32(1.984375)


def test_d2s6_scale_per_64_values_not_32():
    """First 32 values reach 127, the next 32 only ~1/4 of it: D2S6 (one scale per 64) keeps
    the second half's codes near 32, D4/DS4 (one per 32) stretch them to 127."""
    rng = np.random.default_rng(2)
    k = 256
    x = rng.uniform(-1, 1, (1, k)).astype(np.float32)
    x[0, 0] = 127.0
    x[0, 1:32] *= 127.0
    x[0, 32:64] *= 31.0
    x[0, 32] = 31.0
    p6, _ = O.prepare_mmq(x, O.D2S6)
    p4, _ = O.prepare_mmq(x, O.DS4)
    q6 = O.split_plane(p6, O.D2S6)[0]
    q4 = O.split_plane(p4, O.DS4)[0]
    assert np.abs(q6[0, 32:64]).max() == 31 and np.abs(q4[0, 32:64]).max() == 127
    assert np.array_equal(q6[0, :32], q4[0, :32])


def test_reciprocal_quantisation_not_division():
    """quantize_scaled rounds v * (127/amax) (:1053-1058), not v / (amax/127) as the decode
    preparation does: on values where the two differ the batched codes follow the
    reciprocal, and the decode codes the division."""
    rng = np.random.default_rng(3)
    f = np.float32

    def roundf(p):  # C roundf: half-way away from zero
        return int(np.sign(p) * np.floor(abs(np.float64(p)) + 0.5))

    found = None
    while found is None:
        a = f(rng.uniform(64, 128))
        t = rng.integers(1, 126) + 0.5
        v0 = f(t * np.float64(a) / 127)
        for steps in range(-3, 4):  # neighbours of the value that lands on t + 1/2
            v = np.nextafter(v0, f(np.inf if steps > 0 else -np.inf), dtype=np.float32) if steps else v0
            for _ in range(abs(steps) - 1):
                v = np.nextafter(v, f(np.inf if steps > 0 else -np.inf), dtype=np.float32)
            q_mul, q_div = roundf(v * (f(127) / a)), roundf(v / (a / f(127)))
            if q_mul != q_div:
                found = (a, v, q_mul, q_div)
                break
    a, v, q_mul, q_div = found
    x = np.zeros((1, 32), dtype=np.float32)
    x[0, 0], x[0, 1] = a, v
    plane, inv = O.prepare_mmq(x, O.D4)
    assert inv[0] == 1.0
    assert O.split_plane(plane, O.D4)[0][0, 1] == q_mul
    assert O.split_activation(O.prepare(x), 1, 32)[2][0, 1] == q_div


def test_row_scale_matches_decode_preparation_and_scaling_invariance():
    rng = np.random.default_rng(4)
    m, k = 5, 768
    x = (rng.standard_normal((m, k)) * rng.uniform(1e-3, 1e3, (m, 1))).astype(np.float32)
    inv_decode = O.split_activation(O.prepare(x), m, k)[3]
    for layout in (O.D4, O.DS4, O.D2S6):
        plane, inv = O.prepare_mmq(x, layout)
        assert np.array_equal(inv, inv_decode)
        for e in (-30, 5, 44):
            p2, inv2 = O.prepare_mmq(x * np.float32(2.0 ** e), layout)
            assert np.array_equal(p2, plane)
            assert np.array_equal(inv2, inv * np.float32(2.0 ** e))


@pytest.mark.parametrize("layout", [O.D4, O.DS4, O.D2S6])
def test_codes_are_nearest_and_group_max_is_127(layout):
    rng = np.random.default_rng(5 + layout)
    m, k = 4, 512
    x = rng.standard_normal((m, k)).astype(np.float32)
    plane, inv = O.prepare_mmq(x, layout)
    q, d, sums = O.split_plane(plane, layout)
    g = 64 if layout == O.D2S6 else 32
    v = x.astype(np.float64) / inv[:, None]
    vg = v.reshape(m, -1, g)
    a = np.abs(vg).max(-1, keepdims=True)
    qg = q[:, :k].reshape(m, -1, g).astype(np.float64)
    assert np.all(np.abs(qg).max(-1) == 127)
    # q is within half a step (plus the fp32 roundings of 127/amax and the product) of v*127/amax
    assert np.all(np.abs(vg * 127 / a - qg) <= 0.5 + 1e-4)
    # d is 1/d_inv: d * 127 = amax within a few fp32 ulps (in fp16 for DS4/D2S6)
    rel = np.abs(d[:, :k // g].astype(np.float64) * 127 / a[..., 0] - 1)
    assert rel.max() < (2e-6 if layout == O.D4 else 2.0 ** -11)
    if layout == O.DS4:
        s_exact = d[:, :k // 32] * q[:, :k].reshape(m, -1, 32).sum(-1)   # uses fp16 d; stored uses fp32 d
        assert np.all(np.abs(sums[:, :k // 32] - s_exact) <= np.abs(s_exact) * 2.0 ** -9 + 1e-6)


def test_zero_rows_blocks_padding_and_special_values():
    k = 200  # padded to 512: blocks past the row hold zeros
    x = np.zeros((4, k), dtype=np.float32)
    x[1, 5] = 3.0
    x[2, :] = 1.0
    x[2, 40] = np.inf
    x[3, :] = 2.0
    x[3, 7] = np.nan
    for layout in (O.D4, O.DS4, O.D2S6):
        plane, inv = O.prepare_mmq(x, layout)
        q, d, sums = O.split_plane(plane, layout)
        assert q.shape[1] == 512
        assert np.all(q[:, k:] == 0) and np.all(plane[4:, :, :] == 0)
        assert np.all(q[0] == 0) and np.all(d[0] == 0) and inv[0] == 1.0
        assert q[1, 5] == 127 and np.count_nonzero(q[1]) == 1
        # inf row: unit scale; the inf's group has d_inv = 0, so every code is 0 and d = inf
        g = 64 if layout == O.D2S6 else 32
        assert inv[2] == 1.0 and np.all(q[2, (40 // g) * g:(40 // g + 1) * g] == 0) and np.isinf(d[2, 40 // g])
        # NaN is skipped by the maximum and quantises to 0
        assert q[3, 7] == 0 and q[3, 6] == 127


# ----------------------------------------------------------------- second route through the MMQ dots

def _f16(b, off):
    return b[..., off:off + 2].copy().view(np.float16)[..., 0].astype(np.float64)


def _hr(v):
    """Round float64 values to fp16 (the MMQ tile loaders' half products)."""
    return np.asarray(v, dtype=np.float64).astype(np.float32).astype(np.float16).astype(np.float64)


def _decode(qtype, w, k):
    """Weights as float64 [n, k] decoded with numpy from the byte maps (ggml-common.h), with
    the weight-side scales GGML MMQ forms: half(d*sc) and half(dmin*m) for Q4_K/Q2_K."""
    n = w.shape[0]
    qk, bb = O.BLOCK[qtype]
    blk = w.reshape(n, k // qk, bb)
    if qtype == O.Q8_0:
        return (_f16(blk, 0)[..., None] * blk[..., 2:].view(np.int8)).reshape(n, k)
    if qtype == O.Q4_0:
        nib = np.concatenate([blk[..., 2:] & 15, blk[..., 2:] >> 4], axis=-1).astype(np.float64) - 8
        return (_f16(blk, 0)[..., None] * nib).reshape(n, k)
    if qtype == O.Q4_K:
        d, dmin, s = _f16(blk, 0), _f16(blk, 2), blk[..., 4:16].astype(np.int64)
        sc = np.concatenate([s[..., 0:4] & 63, (s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4)], -1)
        mn = np.concatenate([s[..., 4:8] & 63, (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)], -1)
        qs = blk[..., 16:].reshape(n, -1, 4, 32)
        codes = np.stack([qs & 15, qs >> 4], axis=3).reshape(n, -1, 8, 32).astype(np.float64)
        out = _hr(d[..., None] * sc)[..., None] * codes - _hr(dmin[..., None] * mn)[..., None]
        return out.reshape(n, k)
    if qtype == O.Q6_K:
        ql, qh = blk[..., 0:128].astype(np.int64), blk[..., 128:192].astype(np.int64)
        sc, d = blk[..., 192:208].view(np.int8).astype(np.float64), _f16(blk, 208)
        e = np.arange(256)
        h, s, l = e // 128, (e % 128) // 32, e % 32
        lo = (ql[..., 64 * h + 32 * (s % 2) + l] >> (4 * (s // 2))) & 15
        hi = (qh[..., 32 * h + l] >> (2 * s)) & 3
        return (d[..., None] * sc[..., e // 16] * ((lo | (hi << 4)) - 32)).reshape(n, k)
    if qtype == O.Q2_K:
        s, qs = blk[..., 0:16].astype(np.int64), blk[..., 16:80].astype(np.int64)
        d, dmin = _f16(blk, 80), _f16(blk, 82)
        e = np.arange(256)
        h, sh, l = e // 128, (e % 128) // 32, e % 32
        code = (qs[..., 32 * h + l] >> (2 * sh)) & 3
        g = e // 16
        return (_hr(d[..., None] * (s & 15))[..., g] * code - _hr(dmin[..., None] * (s >> 4))[..., g]).reshape(n, k)
    if qtype == O.IQ3_S:
        import json
        from pathlib import Path
        grid = np.array(json.loads((Path(O.ROOT) / "tests/golden/iq3s_grid.json").read_text())["levels"])
        d = _f16(blk, 0)
        e = np.arange(256)
        gg, t = e // 32, e % 32
        i, j = t // 4, t % 4
        idx = blk[..., 2 + 8 * gg + i].astype(np.int64) | (((blk[..., 66 + gg].astype(np.int64) >> i) & 1) << 8)
        sign = np.where((blk[..., 74 + 4 * gg + t // 8] >> (t % 8)) & 1, -1.0, 1.0)
        scale = 1 + 2 * ((blk[..., 106 + gg // 2].astype(np.int64) >> (4 * (gg % 2))) & 15)
        return (d[..., None] * scale * grid[idx, j] * sign).reshape(n, k)
    raise ValueError(qtype)


@pytest.mark.parametrize("qtype", O.WEIGHT_TYPES, ids=lambda t: O.NAMES[t])
@pytest.mark.parametrize("weights", ["random", "quantized"])
def test_mmq_dot_equals_dequantized_dot(qtype, weights):
    """oracle_mul_mat_mmq against numpy: decoded weights (MMQ's weight-side scales) times the
    dequantised plane (q times its group's d). The oracle's min terms use the stored half
    sums where the plane has them; their distance from d * sum(q) bounds the difference."""
    rng = np.random.default_rng(30 + qtype)
    n, k, m = 24, 1024, 5
    if weights == "random":
        w = O.random_blocks(qtype, n, k, rng)
    else:
        from kaillm_amd.formats import quantize
        w = quantize(rng.normal(0, 0.02, (n, k)).astype(np.float32), qtype)
    x = rng.standard_normal((m, k)).astype(np.float16)
    layout = O.mmq_layout(qtype)
    plane, inv = O.prepare_mmq(x, layout)
    got = O.mul_mat_mmq(qtype, w, k, plane, inv)
    q, d, sums = O.split_plane(plane, layout)
    g = 64 if layout == O.D2S6 else 32
    xd = (np.repeat(d, g, axis=1)[:, :k].astype(np.float64) * q[:, :k])
    wd = _decode(qtype, w, k)
    route = (xd @ wd.T) * inv[:, None]
    bound = np.zeros_like(route)
    if qtype in (O.Q4_K, O.Q2_K):
        # min-term weights (|half(dmin*m)| per 32 or 16 values) times |stored sum - d*sum(q)|
        if qtype == O.Q4_K:
            blk = w.reshape(n, k // 256, 144)
            s = blk[..., 4:16].astype(np.int64)
            mn = np.concatenate([s[..., 4:8] & 63, (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)], -1)
            wm = _hr(_f16(blk, 2)[..., None] * mn).reshape(n, -1)
            exact = d[:, :k // 32] * q[:, :k].reshape(m, -1, 32).sum(-1)
            gap = np.abs(sums[:, :k // 32] - exact)
        else:
            blk = w.reshape(n, k // 256, 84)
            wm = _hr(_f16(blk, 82)[..., None] * (blk[..., 0:16].astype(np.int64) >> 4)).reshape(n, -1)
            exact = np.repeat(d, 4, axis=1)[:, :k // 16] * q[:, :k].reshape(m, -1, 16).sum(-1)
            gap = np.nan_to_num(np.abs(sums[:, :k // 16] - exact), nan=0.0)
        bound = (gap @ wm.T) * inv[:, None]
        assert bound.max() > 0  # the stored sums do differ from the exact ones
    scale = np.abs(route).max()
    assert np.all(np.abs(got - route) <= bound * (1 + 1e-9) + 1e-12 * scale)


def test_q2_k_min_terms_use_stored_sums_then_computed_ones():
    """One Q2_K superblock with zero scales (only min terms): the result is
    -sum_g half(dmin*m_g) * S_g, S_g the stored half sum for the first 96 values of each
    128-block and d64 * sum(q) for the last 32."""
    rng = np.random.default_rng(6)
    k = 256
    b = np.zeros(84, dtype=np.uint8)
    mins = rng.integers(1, 16, 16)
    b[0:16] = (mins << 4).astype(np.uint8)
    b[16:80] = rng.integers(0, 256, 64, dtype=np.uint8)
    b[80:82] = np.array([0.25], dtype=np.float16).view(np.uint8)
    b[82:84] = np.array([0.0371], dtype=np.float16).view(np.uint8)
    x = rng.uniform(-1, 1, (1, k)).astype(np.float32) * np.float32(3.3)
    plane, inv = O.prepare_mmq(x, O.D2S6)
    got = O.mul_mat_mmq(O.Q2_K, b[None], k, plane, inv)[0, 0]
    q, d, sums = O.split_plane(plane, O.D2S6)
    dmin = float(np.float16(0.0371))
    want = 0.0
    for g in range(16):
        slot = g % 8
        s = sums[0, g] if slot < 6 else float(d[0, g // 4]) * float(q[0, 16 * g:16 * g + 16].astype(np.int64).sum())
        want -= float(_hr(dmin * mins[g])) * float(s)
    assert got == pytest.approx(want * float(inv[0]), rel=1e-12)


def test_batched_differs_from_decode_arithmetic_for_q2_k():
    """The reason the batched path needs its own oracle: on N(0,1) activations the D2S6
    per-64 scales move a Q2_K product by more than the 1e-3 tolerance from the per-32 Q8_1
    arithmetic of the decode path."""
    from kaillm_amd.formats import quantize
    rng = np.random.default_rng(7)
    n, k, m = 64, 5120, 4
    w = quantize(rng.normal(0, 0.02, (n, k)).astype(np.float32), O.Q2_K)
    x = rng.standard_normal((m, k)).astype(np.float16)
    batched = O.mmq_reference(O.Q2_K, w, x)
    decode = O.mul_mat(O.Q2_K, w, k, O.prepare(x), m)
    assert O.normwise_rel(batched, decode) > 1e-3
