"""Pin the CPU oracle before trusting it as the checker.

Each check is independent of the oracle's own code: numpy's IEEE half
conversion, closed-form values of the Q8_1 row normalisation and rounding,
known-answer blocks assembled by hand from each format's byte map, and the
agreement of two different routes through every layout (integer block dots vs
dequantize-then-dot). The reference holds no golden vectors for this path, so
these are the pins.
"""
import json
from pathlib import Path

import numpy as np
import pytest

import _oracle as O

ROOT = Path(__file__).resolve().parents[1]


# ----------------------------------------------------------------- fp16 conversion

def test_half_to_float_all_65536_match_numpy():
    o = O.lib()
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([o.oracle_half_to_float(int(b)) for b in bits], dtype=np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    assert np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])


def test_float_to_half_rne_matches_numpy():
    o = O.lib()
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        # exact ties and neighbours around every binade edge, subnormals, overflow
        (np.arange(1, 2049, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -24),
        np.array([65504, 65519.99, 65520, 1e6, 6.1035156e-05, 5.9604645e-08, 2.9802322e-08,
                  2.9802326e-08, 0.0, -0.0, 1.0009766, 1.00048828125], dtype=np.float32),
    ])
    vals = np.concatenate([vals, -vals])
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([o.oracle_float_to_half(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, want)


# ----------------------------------------------------------------- Q8_1 preparation

def _scale_exponent(amax):
    """Closed form of kai_dual_mmvq.cuh:202-211 on the IEEE exponent field."""
    biased = int(np.float32(amax).view(np.uint32) >> 23) & 255
    se = 127 if biased in (0, 255) else min(max(260 - biased, 1), 253)
    return se


@pytest.mark.parametrize("amax,expected_inverse", [
    (1.0, 2.0 ** -6), (127.0, 1.0), (64.0, 1.0), (63.99, 0.5), (3.0, 2.0 ** -5),
    (1e-30, None), (1e30, None), (2.0 ** -126, 2.0 ** -126), (2.0 ** 127, 2.0 ** 121),
])
def test_row_normalisation_closed_form(amax, expected_inverse):
    k = 64
    x = np.zeros((1, k), dtype=np.float32)
    x[0, 5] = amax
    x[0, 40] = -amax / 3
    buf = O.prepare(x)
    d, s, q, inverse, _ = O.split_activation(buf, 1, k)
    se = _scale_exponent(amax)
    assert inverse[0] == np.float32(2.0 ** (127 - se))
    if expected_inverse is not None:
        assert inverse[0] == np.float32(expected_inverse)
    scaled = np.float32(amax) * np.float32(2.0 ** (se - 127))
    if 1 < se < 253:
        assert 64.0 <= scaled < 128.0  # amax lands in [64, 128)
    assert q[0, 5] == 127  # the block maximum always quantises to 127


@pytest.mark.parametrize("special", ["zero", "subnormal", "inf", "nan_only_elsewhere"])
def test_special_rows_keep_unit_scale(special):
    k = 64
    x = np.zeros((1, k), dtype=np.float32)
    if special == "subnormal":
        x[0, 3] = np.float32(1e-41)
    elif special == "inf":
        x[0, 40] = np.inf   # second block holds the inf; first block stays finite
        x[0, 3] = 2.0
    elif special == "nan_only_elsewhere":
        x[0, 3] = 100.0     # fmaxf ignores NaN, so the scale comes from 100
        x[0, 40] = np.nan
    buf = O.prepare(x)
    d, s, q, inverse, _ = O.split_activation(buf, 1, k)
    if special == "nan_only_elsewhere":
        assert inverse[0] == 1.0  # 100 already lies in [64, 128)
        assert q[0, 3] == 127
        return
    assert inverse[0] == 1.0
    if special == "zero":
        assert np.all(q == 0) and np.all(d == 0) and np.all(s == 0)
    if special == "subnormal":
        assert q[0, 3] == 127  # IEEE subnormal arithmetic: a/127 and v/d are exact enough
    if special == "inf":
        assert q[0, 3] == 127 and d[0, 0] == np.float32(np.float16(2.0 / 127))


def test_round_half_away_from_zero_and_zero_block():
    k = 64
    x = np.zeros((1, k), dtype=np.float32)
    # row max 127 -> scale 1, d = 127/127 = 1 exactly, so q = roundf(x)
    x[0, :8] = [127, 2.5, -2.5, 3.5, 0.5, -0.5, 1.49999, -126.5]
    buf = O.prepare(x)
    d, s, q, inverse, _ = O.split_activation(buf, 1, k)
    assert inverse[0] == 1.0 and d[0, 0] == 1.0
    assert list(q[0, :8]) == [127, 3, -3, 4, 1, -1, 1, -127]
    assert d[0, 1] == 0 and np.all(q[0, 32:] == 0)  # all-zero block inside a nonzero row
    assert s[0, 0] == np.float32(np.float16(1.0 * q[0, :32].astype(np.int64).sum()))


def test_q8_1_properties_random_rows():
    rng = np.random.default_rng(1)
    m, k = 6, 512
    x = (rng.standard_normal((m, k)) * rng.uniform(1e-3, 1e3, (m, 1))).astype(np.float32)
    d, s, q, inverse, _ = O.split_activation(O.prepare(x), m, k)
    for j in range(m):
        se = _scale_exponent(np.abs(x[j]).max())
        v = x[j] * np.float32(2.0 ** (se - 127))
        assert inverse[j] == np.float32(2.0 ** (127 - se))
        for b in range(k // 32):
            vb = v[32 * b:32 * b + 32]
            qb = q[j, 32 * b:32 * b + 32].astype(np.int64)
            a = np.float32(np.abs(vb).max())
            dexact = a / np.float32(127)
            assert d[j, b] == np.float32(np.float16(dexact))
            assert np.abs(qb).max() == 127
            # |v/d - q| <= 1/2: the nearest integer
            assert np.all(np.abs(vb / dexact - qb) <= 0.5 + 1e-5)
            assert s[j, b] == np.float32(np.float16(dexact * np.float32(qb.sum())))


def test_q8_1_invariant_to_power_of_two_scaling():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    base = O.split_activation(O.prepare(x), 3, 256)
    for e in (-40, -3, 7, 60):
        other = O.split_activation(O.prepare(x * np.float32(2.0 ** e)), 3, 256)
        assert np.array_equal(base[2], other[2])           # q unchanged
        assert np.array_equal(base[0], other[0])           # d unchanged
        assert np.allclose(other[3], base[3] * 2.0 ** e, rtol=0)  # inverse carries the scale


def test_input_dtypes_decode_identically():
    rng = np.random.default_rng(3)
    x16 = rng.standard_normal((2, 128)).astype(np.float16)
    a = O.prepare(x16)
    b = O.prepare(x16.astype(np.float32))
    assert np.array_equal(a, b)
    bf = (rng.standard_normal((2, 128)).astype(np.float32).view(np.uint32) & 0xFFFF0000).astype(np.uint32)
    bf_bits = (bf >> 16).astype(np.uint16)
    c = O.prepare(bf_bits, dtype_code=1)
    e = O.prepare(bf.view(np.float32))
    assert np.array_equal(c, e)


def test_two_pass_residual_property():
    rng = np.random.default_rng(4)
    m, k = 2, 128
    x = rng.standard_normal((m, k)).astype(np.float32)
    d1, s1, q1, inv, p2 = O.split_activation(O.prepare(x, two_pass=1), m, k, two_pass=1)
    d2, s2, q2 = p2
    for j in range(m):
        se = _scale_exponent(np.abs(x[j]).max())
        v = x[j].astype(np.float64) * 2.0 ** (se - 127)
        resid = v - np.repeat(d1[j], 32) * q1[j] - np.repeat(d2[j], 32) * q2[j]
        # the second pass leaves half a step of d2, plus the fp16 rounding of d2 (2^-11
        # relative) times |q2| <= 127; a single pass leaves up to half a step of d1 >> d2
        bound = np.repeat(d2[j].astype(np.float64), 32) * (0.5 + 127 * 2.0 ** -11) + 1e-9
        assert np.all(np.abs(resid) <= bound)
        assert np.abs(resid).max() < 0.05 * np.abs(v - np.repeat(d1[j], 32) * q1[j]).max()


def test_activation_layout():
    assert O.activation_bytes(3, 64, 0) == 256 + 256
    assert O.activation_bytes(1, 5120, 0) == (160 * 36 + 255) // 256 * 256 + 256
    assert O.activation_bytes(2, 64, 1) == 256 * 2 + 256


# ----------------------------------------------------------------- dequant known answers

def _half(v):
    return np.array([v], dtype=np.float16).view(np.uint8)


def test_kat_q8_0():
    b = np.zeros(34, dtype=np.uint8)
    b[0:2] = _half(0.5)
    b[2:34] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    out = O.dequantize(O.Q8_0, b[None], 32)[0]
    assert np.array_equal(out, 0.5 * np.arange(-16, 16, dtype=np.float32))


def test_kat_q4_0_nibble_positions():
    b = np.zeros(18, dtype=np.uint8)
    b[0:2] = _half(2.0)
    b[2:] = 0x88                   # every nibble 8 -> value 0
    b[2 + 3] = 0x8B                # low nibble of qs[3] = 11 -> element 3 = (11-8)*2
    b[2 + 7] = 0x28                # high nibble of qs[7] = 2 -> element 23 = (2-8)*2
    out = O.dequantize(O.Q4_0, b[None], 32)[0]
    want = np.zeros(32, dtype=np.float32)
    want[3], want[23] = 6.0, -12.0
    assert np.array_equal(out, want)


def _q4k_block(sc, mn, codes, d=1.0, dmin=1.0):
    """Assemble a Q4_K block from 8 scales, 8 mins (6-bit) and 256 codes (4-bit)."""
    b = np.zeros(144, dtype=np.uint8)
    b[0:2], b[2:4] = _half(d), _half(dmin)
    s = np.zeros(12, dtype=np.uint8)
    for i in range(4):
        s[i] = (sc[i] & 63) | ((sc[i + 4] >> 4) << 6)
        s[4 + i] = (mn[i] & 63) | ((mn[i + 4] >> 4) << 6)
        s[8 + i] = (sc[i + 4] & 15) | ((mn[i + 4] & 15) << 4)
    b[4:16] = s
    for j in range(4):
        b[16 + 32 * j:16 + 32 * j + 32] = codes[64 * j:64 * j + 32] | (codes[64 * j + 32:64 * j + 64] << 4)
    return b


def test_kat_q4_k_scales_mins_and_codes():
    rng = np.random.default_rng(5)
    sc = np.array([1, 63, 17, 32, 48, 5, 62, 33], dtype=np.uint8)   # >= 16 exercises the top bits
    mn = np.array([0, 9, 63, 31, 16, 47, 2, 60], dtype=np.uint8)
    codes = rng.integers(0, 16, 256, dtype=np.uint8)
    b = _q4k_block(sc, mn, codes, d=0.25, dmin=0.5)
    out = O.dequantize(O.Q4_K, b[None], 256)[0]
    want = 0.25 * np.repeat(sc, 32).astype(np.float32) * codes - 0.5 * np.repeat(mn, 32).astype(np.float32)
    assert np.array_equal(out, want.astype(np.float32))


def _q6k_block(codes, scales, d=1.0):
    b = np.zeros(210, dtype=np.uint8)
    for e in range(256):
        h, s, l = e // 128, (e % 128) // 32, e % 32
        b[64 * h + 32 * (s % 2) + l] |= (codes[e] & 15) << (4 * (s // 2))
        b[128 + 32 * h + l] |= (codes[e] >> 4) << (2 * s)
    b[192:208] = scales.astype(np.int8).view(np.uint8)
    b[208:210] = _half(d)
    return b


def test_kat_q6_k_offset_sign_and_positions():
    codes = np.full(256, 32, dtype=np.uint8)   # code 32 -> value 0
    codes[0], codes[77], codes[130], codes[255] = 0, 63, 33, 1
    scales = np.arange(-8, 8, dtype=np.int8)
    scales[0] = -3
    b = _q6k_block(codes, scales, d=0.5)
    out = O.dequantize(O.Q6_K, b[None], 256)[0]
    want = np.zeros(256, dtype=np.float32)
    for e in (0, 77, 130, 255):
        want[e] = 0.5 * float(scales[e // 16]) * (int(codes[e]) - 32)
    assert np.array_equal(out, want)


def test_kat_q2_k_scale_nibbles_and_positions():
    b = np.zeros(84, dtype=np.uint8)
    scales = np.array([(g % 16) | (((15 - g) % 16) << 4) for g in range(16)], dtype=np.uint8)
    b[0:16] = scales
    codes = np.zeros(256, dtype=np.uint8)
    codes[[1, 40, 100, 129, 200, 255]] = [3, 1, 2, 3, 1, 2]
    for e in range(256):
        h, s, l = e // 128, (e % 128) // 32, e % 32
        b[16 + 32 * h + l] |= codes[e] << (2 * s)
    b[80:82], b[82:84] = _half(0.5), _half(0.25)
    out = O.dequantize(O.Q2_K, b[None], 256)[0]
    g = np.arange(256) // 16
    want = 0.5 * (scales[g] & 15).astype(np.float32) * codes - 0.25 * (scales[g] >> 4).astype(np.float32)
    assert np.array_equal(out, want.astype(np.float32))


def test_kat_iq3_s_index_bit8_signs_scale_and_top_level():
    grid = json.loads((ROOT / "tests/golden/iq3s_grid.json").read_text())["levels"]
    b = np.zeros(110, dtype=np.uint8)
    b[0:2] = _half(0.5)
    # group 2, index slot 5: grid entry 300 (needs bit 8 from qh[2] bit 5)
    b[2 + 8 * 2 + 5] = 300 & 0xFF
    b[66 + 2] = 1 << 5
    # group 2 values t = 20..23 come from slot 5; flip the sign of t = 21 (byte 4*2 + 21//8, bit 21%8)
    b[74 + 4 * 2 + 21 // 8] = 1 << (21 % 8)
    # scale nibble of group 2 (low nibble of scales[1]) = 7 -> d*(1+14); group 3 (high nibble) = 15
    b[106 + 1] = 7 | (15 << 4)
    # group 3 slot 0 -> an entry containing level 15
    e15 = next(i for i, e in enumerate(grid) if e[0] == 15)
    b[2 + 8 * 3 + 0] = e15 & 0xFF
    b[66 + 3] = (e15 >> 8) << 0
    out = O.dequantize(O.IQ3_S, b[None], 256)[0]
    want = np.zeros(256, dtype=np.float32)
    for g in range(8):
        scale = 0.5 * (1 + 2 * ((b[106 + g // 2] >> (4 * (g % 2))) & 15))
        for i in range(8):
            idx = int(b[2 + 8 * g + i]) | (((int(b[66 + g]) >> i) & 1) << 8)
            for j in range(4):
                t = 4 * i + j
                sign = -1 if (b[74 + 4 * g + t // 8] >> (t % 8)) & 1 else 1
                want[32 * g + t] = scale * grid[idx][j] * sign
    assert np.array_equal(out, want)
    assert out[32 * 2 + 21] == -0.5 * 15 * grid[300][1]
    assert out[32 * 3 + 0] == 0.5 * 31 * 15  # top level is 15, not 15.5


# ----------------------------------------------------------------- two routes through each layout

@pytest.mark.parametrize("qtype", O.WEIGHT_TYPES, ids=lambda t: O.NAMES[t])
def test_block_dot_equals_dequantized_dot(qtype):
    """Integer block dots (oracle_mul_mat) == dense dot of the dequantized weights with the
    dequantized Q8_1 activation. Q4_0 uses the stored fp16 s8 for its offset term, so its
    dense route adds d_w * 8 * (d8 * sum(q8) - s8) exactly."""
    rng = np.random.default_rng(10 + qtype)
    n, k, m = 24, 512, 3
    w = O.random_blocks(qtype, n, k, rng)
    x = rng.standard_normal((m, k)).astype(np.float32)
    act = O.prepare(x)
    got = O.mul_mat(qtype, w, k, act, m)
    wd = O.dequantize(qtype, w, k).astype(np.float64)
    d, s, q, inverse, _ = O.split_activation(act, m, k)
    xd = np.repeat(d, 32, axis=1).astype(np.float64) * q
    dense = (xd @ wd.T) * inverse[:, None]
    if qtype == O.Q4_0:
        dw = w.reshape(n, k // 32, 18)[:, :, 0:2].copy().view(np.float16).reshape(n, k // 32).astype(np.float64)
        corr = 8.0 * (d.astype(np.float64) * q.reshape(m, k // 32, 32).sum(-1) - s)   # [m, nb]
        dense += (corr @ dw.T) * inverse[:, None]
    assert O.normwise_rel(got, dense) < 1e-6


def test_oracle_f32_baseline_matches_f64():
    rng = np.random.default_rng(20)
    n, k, m = 16, 256, 2
    w = O.random_blocks(O.Q4_K, n, k, rng)
    act = O.prepare(rng.standard_normal((m, k)).astype(np.float32))
    ref = O.mul_mat(O.Q4_K, w, k, act, m)
    out = np.empty((m, n), dtype=np.float32)
    assert O.lib().oracle_mul_mat_f32(O.Q4_K, O._p(w), n, k, m, O._p(act), 0, O._p(out), n, 2) == 0
    assert O.normwise_rel(out, ref) < 1e-6


# ----------------------------------------------------------------- IQ3_S grid tables

def test_iq3s_grid_tables_agree_with_fixture():
    fx = json.loads((ROOT / "tests/golden/iq3s_grid.json").read_text())
    levels = fx["levels"]
    assert len(levels) == 512 and all(len(e) == 4 for e in levels)
    assert {v for e in levels for v in e} == {1, 3, 5, 7, 9, 11, 13, 15}
    assert len({tuple(e) for e in levels}) == 512
    assert fx["entries_with_level_15"] > 0
    import hashlib
    assert hashlib.sha256(json.dumps(levels).encode()).hexdigest() == fx["sha256_levels_json"]
    text = (ROOT / "kaillm_amd/csrc/kai_iq3s_grid.h").read_text()
    import re
    product = [int(v, 16) for v in re.findall(r"0x([0-9a-f]{8})u", text)]
    assert product == fx["packed_u32"]
    otext = (ROOT / "oracle/oracle_iq3s_grid.h").read_text()
    oracle_levels = [[int(v) for v in e.split(",")] for e in re.findall(r"\{(\d+,\d+,\d+,\d+)\}", otext)]
    assert oracle_levels == levels
