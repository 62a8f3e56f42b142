"""The exact-integer affine projection of the oracle (oracle/xq.c), pinned on
the CPU against what the mathematics fixes:
  * the float64 closed form sum_k x_k (s q_k + b) of the affine layout
    (reference kernels/verify_qmv.h:112, matrix_verify.h:7-29), within a
    rigorous bound: the activation grid's truncation (< 2^(Eb - 156) per
    value) times sum |w|, plus half an fp32 ulp of the result;
  * exactness: with small integer activations, power-of-two scales and
    biases, every step is exact and y equals the exact rational sum;
  * the truncation rule: a value 22 binades below its group's largest is
    kept exactly, one more binade down it truncates toward zero;
  * the grid integers stay below 2^30, so four signed int8 digits hold them
    (the GPU's operands);
  * planted mistakes (the bias term dropped, the slices merged into one
    sequential sum, the grid anchored at the row's exponent instead of the
    group's) change the result.
"""
import numpy as np
import pytest


def _bf(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _dense_w(orc, codes, s, b, k, bits):
    q = orc.unpack_codes(codes, k, bits).astype(np.float64)
    g = np.repeat(np.arange(k // 64), 64)
    return _bf(s)[:, g] * q + _bf(b)[:, g]


def _group_exp(x):
    e = (np.asarray(x, np.uint16) >> 7) & 0xFF
    return np.maximum(e.reshape(x.shape[0], -1, 64).max(axis=2), 1)


@pytest.mark.parametrize("k,bits", [(256, 4), (512, 5), (2048, 4), (2048, 6), (2048, 8), (8192, 4)])
def test_xq_within_rigorous_bound_of_float64_closed_form(orc, k, bits):
    n, m = 48, 3
    codes, s, b = orc.random_qweight(n, k, bits, 64, seed=k + bits)
    rng = np.random.default_rng(k * 7 + bits)
    xf = rng.standard_normal((m, k)).astype(np.float32)
    xf[:, ::37] *= 2.0 ** rng.integers(-30, -10, xf[:, ::37].shape)  # wide exponents in groups
    x = orc.f32_to_bf16(xf)
    y = orc.xq(codes, s, b, k, bits, x).astype(np.float64)
    w = _dense_w(orc, codes, s, b, k, bits)
    y64 = _bf(x) @ w.T
    eb = _group_exp(x)  # [m, G]
    grid = 2.0 ** (eb - 156.0)
    wabs = np.abs(w).reshape(n, -1, 64).sum(axis=2)  # [n, G]
    bound = grid @ wabs.T * 64 / 64 + np.abs(y64) * 2.0 ** -24 + 1e-300
    assert np.all(np.abs(y - y64) <= bound), np.max(np.abs(y - y64) / bound)
    # and far tighter than bf16 needs
    assert np.max(np.abs(y - y64) / (np.abs(y64) + 1e-6)) < 1e-5


def test_xq_exact_on_integer_inputs(orc):
    """Integer activations |x| <= 100, scales 2^-3, biases -2^-1: no value is
    truncated and every product and sum is exact, so y is the exact sum."""
    n, k, bits = 16, 1024, 4
    codes = orc.fill_codes(n, k, bits, 5)
    s = np.full((n, k // 64), orc.f32_to_bf16(np.float32(0.125)), np.uint16)
    b = np.full((n, k // 64), orc.f32_to_bf16(np.float32(-0.5)), np.uint16)
    xi = np.random.default_rng(2).integers(-100, 101, (2, k))
    x = orc.f32_to_bf16(xi.astype(np.float32))
    y = orc.xq(codes, s, b, k, bits, x)
    q = orc.unpack_codes(codes, k, bits).astype(np.int64)
    exact8 = xi @ (q.T * 1 - 4)  # 8 y = sum x (q - 4)
    assert (y.astype(np.float64) * 8 == exact8).all()


def test_xq_truncation_rule(orc):
    """One group: 2^10 at position 0; a value 22 binades down is exact, a value
    23 binades down with an odd significand loses its last bit."""
    k, bits, n = 64, 8, 1
    codes = np.zeros((n, k * bits // 32), np.uint32)
    codes[0, 0] = 1  # q_0 = 1
    codes[0, 1] = 1  # q_4 = 1
    s = orc.f32_to_bf16(np.array([[1.0]], np.float32))
    b = orc.f32_to_bf16(np.array([[0.0]], np.float32))
    for shift, keeps in ((22, True), (23, False)):
        x = np.zeros((1, k), np.float32)
        x[0, 0] = 2.0 ** 10
        x[0, 4] = 2.0 ** (10 - shift) * (1 + 2 ** -7)  # significand 0x81
        xb = orc.f32_to_bf16(x)
        y = float(orc.xq(codes, s, b, k, bits, xb)[0, 0])
        want = 2.0 ** 10 + float(_bf(xb)[0, 4])
        if keeps:
            assert y == np.float32(want)
        else:
            trunc = 2.0 ** 10 + 2.0 ** (10 - shift) * (1 + 2 ** -7) - 2.0 ** (10 - shift - 7)
            assert np.float64(orc.xq(codes, s, b, k, bits, xb)[0, 0]) == np.float32(trunc)
    # the grid integer of the group's largest value, and of the smallest kept
    assert orc.lib.mxo_xq_int(0x4480, 137) == 0x80 << 22
    assert orc.lib.mxo_xq_int(0x8001, 137) == 0  # a denormal far below
    assert orc.lib.mxo_xq_int(orc.f32_to_bf16(np.float32(-3.0)).item(), 128) == -(0xC0 << 22)


def test_xq_grid_integers_fit_four_int8_digits(orc):
    """Every bf16 value on the grid of any exponent field at or above its own
    stays below 2^30 in magnitude (the top signed base-256 digit is then
    within [-64, 64])."""
    worst = 0
    for h in range(0, 0x10000, 7):
        e = max((h >> 7) & 0xFF, 1)
        for eb in (e, e + 1, e + 22, e + 30):
            v = abs(orc.lib.mxo_xq_int(h, eb))
            worst = max(worst, v)
    assert worst < 2 ** 30


def test_xq_planted_mistakes_fail(orc):
    """A dropped bias term misses the closed form; merging the slices of a
    K = 1024 row into one sequential double sum, and anchoring the grid at the
    row's largest exponent, give other bits on inputs built to show them."""
    n, k, bits = 4, 1024, 4
    codes, s, b = orc.random_qweight(n, k, bits, 64, seed=9)
    x = orc.f32_to_bf16(np.random.default_rng(9).standard_normal((1, k)).astype(np.float32))
    y = orc.xq(codes, s, b, k, bits, x).astype(np.float64)
    w = _dense_w(orc, codes, s, b, k, bits)
    no_bias = _bf(x) @ (w - np.repeat(_bf(b), 64, axis=1)).T
    assert np.max(np.abs(y - no_bias)) > 1e-2
    # slices of two groups: group 0 = +2^60 (slice 0); groups 8 = -2^60 and
    # 9 = +1 share slice 4
    codes1 = np.zeros((1, k * 8 // 32), np.uint32)
    for g in (0, 8, 9):
        codes1[0, g * 16] = 1  # q at value 64 g = 1 (8-bit codes: 4 per word)
    s1 = orc.f32_to_bf16(np.ones((1, k // 64), np.float32))
    b1 = orc.f32_to_bf16(np.zeros((1, k // 64), np.float32))
    xf = np.zeros((1, k), np.float32)
    xf[0, 0], xf[0, 512], xf[0, 576] = 2.0 ** 60, -(2.0 ** 60), 1.0
    y1 = float(orc.xq(codes1, s1, b1, k, 8, orc.f32_to_bf16(xf))[0, 0])
    assert orc.lib.mxo_xq_slices(k) == 8
    assert orc.lib.mxo_xq_slices(448) == 4 and orc.lib.mxo_xq_slices(64) == 1
    assert y1 == 0.0  # slice 4 rounds -2^60 + 1 to -2^60; one sequential sum would give 1
    # grid per group, not per row: a group of small values next to a group
    # holding 2^20 keeps all its bits
    xg = np.full((1, 128), 1.0 + 2 ** -7, np.float32)
    xg[0, 64] = 2.0 ** 20
    c2 = np.zeros((1, 128 * 8 // 32), np.uint32)
    c2[0, 0] = 1
    y2 = float(orc.xq(c2, s1[:, :2], b1[:, :2], 128, 8, orc.f32_to_bf16(xg))[0, 0])
    assert y2 == np.float32(1.0 + 2 ** -7)
