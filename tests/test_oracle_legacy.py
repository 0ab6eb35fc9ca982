"""Pin the oracle's restatement of the legacy _C_gguf ops (gguf_kernel.cu:32-290).

The activation (quantize_q8_1, :32-69) is pinned by closed forms: values whose codes and
scales are known exactly, round-half-away ties, the all-negative-zero block, fp16
overflow and underflow of the stored scale and sum, and two inputs whose fp32 sum
depends on the grouping of the 32-lane butterfly, so that a sequential or an
adjacent-pair sum fails. The products are pinned by routes that do not share the
oracle's block formulas: the dense dot of dequantized weights with the dequantized
activation (every format whose legacy dot uses only d8 and the codes), and, for the two
forms that take the stored sum half(sum x) (Q4_0 on both ops, Q4_K on ggml_mul_mat_a8),
weights whose scale terms vanish, leaving the dense dot with the unquantised x.
"""
import numpy as np
import pytest

import _oracle as O


def _blocks(buf, m, k):
    """-> (d bits [m, nb], s bits [m, nb], q [m, k], inverse [m])."""
    nb = k // 32
    blocks = buf[:m * nb * 36].reshape(m, nb, 36)
    d = blocks[:, :, 0:2].copy().view(np.uint16).reshape(m, nb)
    s = blocks[:, :, 2:4].copy().view(np.uint16).reshape(m, nb)
    q = blocks[:, :, 4:].copy().view(np.int8).reshape(m, k)
    off = (m * nb * 36 + 255) // 256 * 256
    inverse = buf[off:off + 4 * m].copy().view(np.float32)
    return d, s, q, inverse


def _h(v):
    return int(np.float16(v).view(np.uint16))


def test_integer_block_has_unit_scale_and_exact_codes():
    rng = np.random.default_rng(1)
    x = rng.integers(-126, 127, size=(2, 64)).astype(np.float32)
    x[0, 5], x[0, 40], x[1, 0], x[1, 63] = 127, -127, -127, 127
    d, s, q, inverse = _blocks(O.prepare_legacy(x), 2, 64)
    assert (d == _h(1.0)).all()
    assert np.array_equal(q, x.astype(np.int8))
    sums = x.reshape(2, 2, 32).sum(-1)   # integers below 2048: exact in fp32 and fp16
    assert np.array_equal(s, np.vectorize(_h)(sums).astype(np.uint16))
    assert np.array_equal(inverse, np.ones(2, np.float32))   # no row normalisation


def test_round_half_away_from_zero():
    x = np.zeros((1, 32), np.float32)
    x[0, :6] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5]    # d = 1: x / d is the tie itself
    _, _, q, _ = _blocks(O.prepare_legacy(x), 1, 32)
    assert q[0, :6].tolist() == [127, 3, -3, 1, -1, 2]


def test_butterfly_grouping_of_the_sum():
    # 2^25 + 1 rounds to 2^25 in fp32 (ulp 4). Butterfly: (x0 + x16) = 0 first, then + 1.
    a = np.zeros((2, 32), np.float32)
    a[0, 0], a[0, 16], a[0, 1] = 2.0 ** 25, -2.0 ** 25, 1.0
    # Here x0 + x16 = 2^25 + 1 -> 2^25 is rounded first, and x1 = -2^25 cancels it later: 0.
    # (An adjacent-pair tree would give 1, a left-to-right sum 1 as well.)
    a[1, 0], a[1, 1], a[1, 16] = 2.0 ** 25, -2.0 ** 25, 1.0
    _, s, _, _ = _blocks(O.prepare_legacy(a), 2, 32)
    assert int(s[0, 0]) == _h(1.0)      # a left-to-right sum gives 0 here
    assert int(s[1, 0]) == 0x0000


def test_zero_blocks_and_signed_zero_sum():
    x = np.zeros((2, 32), np.float32)
    x[1] = -0.0
    d, s, q, _ = _blocks(O.prepare_legacy(x), 2, 32)
    assert (d == 0).all() and (q == 0).all()
    assert int(s[0, 0]) == 0x0000 and int(s[1, 0]) == 0x8000   # (-0) + (-0) stays -0


def test_fp16_overflow_and_underflow_are_kept():
    x = np.zeros((2, 32), np.float32)
    x[0] = 4000.0                        # sum 128000 > 65504: stored sum is +inf
    x[1, 0], x[1, 1] = 1e-6, -2e-7       # d = 7.9e-9 underflows fp16 to 0
    d, s, q, _ = _blocks(O.prepare_legacy(x), 2, 32)
    assert int(s[0, 0]) == 0x7C00 and int(d[0, 0]) == _h(np.float32(4000.0) / np.float32(127.0))
    assert (q[0] == 127).all()
    assert int(d[1, 0]) == 0x0000 and q[1, 0] == 127 and q[1, 1] == -25
    assert int(s[1, 0]) == _h(np.float32(1e-6) + np.float32(-2e-7))


def test_input_dtypes_decode_identically():
    rng = np.random.default_rng(4)
    x16 = rng.standard_normal((3, 96)).astype(np.float16)
    b16 = (x16.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    xb = (b16.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(O.prepare_legacy(x16), O.prepare_legacy(x16.astype(np.float32)))
    assert np.array_equal(O.prepare_legacy(b16, dtype_code=1), O.prepare_legacy(xb))


def _exact_rows(rng, m, k, c):
    """Rows that the legacy quantisation carries exactly: x = c * q, |q| <= 127, a +-127 in
    every block (so d = c), block sums below 2048 * c (exact in fp16)."""
    x = np.empty((m, k), np.float32)
    for r in range(m):
        for b in range(k // 32):
            while True:
                q = rng.integers(-127, 128, 32)
                q[rng.integers(0, 32)] = 127 * rng.choice([-1, 1])
                if abs(q.sum()) < 2048:
                    break
            x[r, 32 * b:32 * b + 32] = c * q
    return x


@pytest.mark.parametrize("qtype", O.WEIGHT_TYPES, ids=lambda t: O.NAMES[t])
@pytest.mark.parametrize("batched", [0, 1])
def test_exact_activation_gives_dense_product(qtype, batched):
    rng = np.random.default_rng(20 + qtype)
    n, k, m = 16, 512, 3
    w = O.random_blocks(qtype, n, k, rng)
    x = _exact_rows(rng, m, k, 2.0 ** -5)
    got = O.legacy_reference(qtype, w, x, batched)
    dense = x.astype(np.float64) @ O.dequantize(qtype, w, k).astype(np.float64).T
    assert O.normwise_rel(got, dense) < 1e-6


@pytest.mark.parametrize("qtype", [O.Q8_0, O.Q6_K, O.Q2_K, O.IQ3_S, O.Q4_K], ids=lambda t: O.NAMES[t])
def test_code_only_forms_equal_dequantized_dot(qtype):
    """ggml_mul_mat_vec_a8 (and ggml_mul_mat_a8 except for Q4_K): d8 and the codes only."""
    rng = np.random.default_rng(40 + qtype)
    n, k, m = 16, 512, 4
    w = O.random_blocks(qtype, n, k, rng)
    x = rng.standard_normal((m, k)).astype(np.float32)
    act = O.prepare_legacy(x)
    d, _, q, _ = _blocks(act, m, k)
    xd = np.repeat(d.view(np.float16).astype(np.float64), 32, axis=1) * q
    dense = xd @ O.dequantize(qtype, w, k).astype(np.float64).T
    for batched in ((0, 1) if qtype != O.Q4_K else (0,)):
        assert O.normwise_rel(O.mul_mat_legacy(qtype, w, k, act, m, batched), dense) < 1e-6


def _sixteenths(rng, m, k):
    """Values on a 1/16 grid in [-2, 2]: block sums are exact in fp16, the codes are not."""
    return (rng.integers(-32, 33, size=(m, k)) / 16.0).astype(np.float32)


@pytest.mark.parametrize("batched", [0, 1])
def test_q4_0_offset_uses_stored_sum_of_x(batched):
    """All nibbles 0: the weight is -8 d per block, and both legacy ops give it against the
    unquantised x, because the offset term reads half(sum x)."""
    rng = np.random.default_rng(7)
    n, k, m = 12, 256, 3
    w = O.random_blocks(O.Q4_0, n, k, rng).reshape(n, k // 32, 18)
    w[:, :, 2:] = 0
    w = w.reshape(n, -1)
    x = _sixteenths(rng, m, k)
    got = O.legacy_reference(O.Q4_0, w, x, batched)
    dense = x.astype(np.float64) @ O.dequantize(O.Q4_0, w, k).astype(np.float64).T
    assert O.normwise_rel(got, dense) < 1e-12


def test_q4_k_min_term_per_op():
    """Scales 0, mins non-zero: the weight is -dmin * m per 32 values. ggml_mul_mat_a8's min
    term reads half(sum x) and matches the unquantised x; ggml_mul_mat_vec_a8's reads
    d8 * sum q and matches the dequantized activation."""
    rng = np.random.default_rng(8)
    n, k, m = 10, 512, 2
    w = O.random_blocks(O.Q4_K, n, k, rng).reshape(n, k // 256, 144)
    # scales of blocks 0-3: low 6 bits of bytes 4-7; of blocks 4-7: low nibbles of bytes 12-15
    # and the top 2 bits of bytes 4-7 (the mins live in bytes 8-11 and the high nibbles)
    w[:, :, 4:8] = 0
    w[:, :, 12:16] &= 0xF0
    w = w.reshape(n, -1)
    wd = O.dequantize(O.Q4_K, w, k).astype(np.float64)
    assert np.all(wd.reshape(n, -1, 32).std(-1) == 0)      # constant per 32 values
    x = _sixteenths(rng, m, k)
    act = O.prepare_legacy(x)
    mmq = O.mul_mat_legacy(O.Q4_K, w, k, act, m, 1)
    assert O.normwise_rel(mmq, x.astype(np.float64) @ wd.T) < 1e-12
    d, _, q, _ = _blocks(act, m, k)
    xd = np.repeat(d.view(np.float16).astype(np.float64), 32, axis=1) * q
    mmvq = O.mul_mat_legacy(O.Q4_K, w, k, act, m, 0)
    assert O.normwise_rel(mmvq, xd @ wd.T) < 1e-12
    assert O.normwise_rel(mmvq, mmq) > 1e-4                 # the two ops differ here
