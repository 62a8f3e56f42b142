"""Pins the oracle's scalar arithmetic, bit layout, dequantisation and QMV
against what the mathematics and the reference's own formulas fix (no GPU)."""
import numpy as np
import pytest


def ulp_err(got, want):
    """Error in units of fp32 ulp of the exact (double) value."""
    want = np.asarray(want, np.float64)
    spacing = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - want) / spacing


def test_expf_accuracy(orc):
    x = np.linspace(-103.0, 88.7, 200001, dtype=np.float32)
    got = orc.eval_math(0, x)
    want = np.exp(x.astype(np.float64))
    normal = want > 1.2e-38
    assert ulp_err(got[normal], want[normal]).max() <= 2.0
    # special values
    sp = orc.eval_math(0, np.array([0.0, -0.0, 89.0, -104.0, np.inf, -np.inf], np.float32))
    assert sp[0] == 1.0 and sp[1] == 1.0 and np.isinf(sp[2]) and sp[3] == 0.0
    assert np.isinf(sp[4]) and sp[5] == 0.0
    assert np.isnan(orc.eval_math(0, np.array([np.nan], np.float32))[0])


def test_log1p_softplus_sigmoid_accuracy(orc):
    u = np.concatenate([np.geomspace(1e-30, 1.0, 50000), np.linspace(-0.9, 30.0, 50000)]).astype(np.float32)
    got = orc.eval_math(1, u)
    assert ulp_err(got, np.log1p(u.astype(np.float64))).max() <= 3.0
    x = np.linspace(-60.0, 60.0, 100001, dtype=np.float32)
    xd = x.astype(np.float64)
    sp = orc.eval_math(3, x)
    want = np.logaddexp(xd, 0.0)
    assert (np.abs(sp - want) <= 4 * np.spacing(want.astype(np.float32)) + 1e-30).all()
    sg = orc.eval_math(2, x)
    want = 1.0 / (1.0 + np.exp(-xd))
    assert np.abs(sg - want).max() <= 1.2e-7
    # the MLX form computes the negative side directly: sigma(x) = fl32(1 - sigma(-x)) for x > 0
    pos = x[x > 0]
    assert (orc.eval_math(2, pos) == np.float32(1.0) - orc.eval_math(2, -pos)).all()


def test_bf16_round_to_nearest_even(orc):
    u = np.array([0x3F808000, 0x3F818000, 0x3F808001, 0x7F7FFFFF, 0x7F800000, 0xFF800000,
                  0x7FC00001, 0x00000001, 0x80000000], np.uint32)
    got = orc.f32_to_bf16(u.view(np.float32))
    # halfway 1.00390625 -> even 1.0; halfway above odd -> up; above halfway -> up;
    # FLT_MAX -> +inf; infinities keep; NaN -> quiet NaN; tiny denormal -> +0; -0 keeps.
    assert list(got) == [0x3F80, 0x3F82, 0x3F81, 0x7F80, 0x7F80, 0xFF80, 0x7FC0, 0x0000, 0x8000]
    for h in [0x0001, 0x3F80, 0x7F7F, 0xC2F7]:
        f = orc.bf16_to_f32(np.array([h], np.uint16))
        assert orc.f32_to_bf16(f)[0] == h
    # the C scalar agrees with the numpy helper on random patterns
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    c = np.array([orc.lib.mxo_f32_to_bf16(float(v)) for v in f[:2000]], np.uint16)
    assert (c == orc.f32_to_bf16(f[:2000])).all()


def _ref_unpack_bytes(row_bytes: bytes, k: int, bits: int):
    """Decode codes with the reference's byte masks (kernels/verify_qmv.h:60-116)."""
    b = np.frombuffer(row_bytes, np.uint8).astype(np.uint32)
    out = []
    if bits == 4:
        for i in range(k // 2):
            out += [b[i] & 0xF, b[i] >> 4]
    elif bits == 8:
        out = list(b[:k])
    elif bits == 5:
        for p in range(k // 8):
            w = b[5 * p:5 * p + 5]
            out += [w[0] & 0x1F, (w[0] & 0xE0) >> 5 | (w[1] & 0x3) << 3, (w[1] & 0x7C) >> 2,
                    (w[1] & 0x80) >> 7 | (w[2] & 0xF) << 1, (w[2] & 0xF0) >> 4 | (w[3] & 0x1) << 4,
                    (w[3] & 0x3E) >> 1, (w[3] & 0xC0) >> 6 | (w[4] & 0x7) << 2, (w[4] & 0xF8) >> 3]
    elif bits == 6:
        for p in range(k // 4):
            w = b[3 * p:3 * p + 3]
            out += [w[0] & 0x3F, (w[0] & 0xC0) >> 6 | (w[1] & 0xF) << 2,
                    (w[1] & 0xF0) >> 4 | (w[2] & 0x3) << 4, (w[2] & 0xFC) >> 2]
    return np.array(out, np.uint32)


@pytest.mark.parametrize("bits", [4, 5, 6, 8])
def test_code_layout_matches_reference_byte_masks(orc, bits):
    k, rows = 256, 16
    codes = orc.fill_codes(rows, k, bits, seed=77 + bits)
    un = orc.unpack_codes(codes, k, bits)
    for r in range(rows):
        ref = _ref_unpack_bytes(codes[r].tobytes(), k, bits)
        assert (un[r] == ref).all()
    # the generator covers every code value
    assert set(np.unique(un)) == set(range(2 ** bits))


@pytest.mark.parametrize("bits", [4, 5, 6, 8])
def test_dequant_closed_form_every_code(orc, bits):
    gs, k = 32, 2 ** bits * 2 if bits < 8 else 512
    k = max(k, 64)
    n = 6
    codes_vals = (np.arange(n * k) % (2 ** bits)).reshape(n, k).astype(np.uint32)
    # pack codes into MLX layout by hand (bitstream, little endian)
    words = np.zeros((n, k * bits // 32), np.uint32)
    for r in range(n):
        acc = 0
        for c in range(k):
            acc |= int(codes_vals[r, c]) << (c * bits)
        for w in range(words.shape[1]):
            words[r, w] = (acc >> (32 * w)) & 0xFFFFFFFF
    s = orc.f32_to_bf16(np.linspace(-0.07, 0.05, n * (k // gs)).astype(np.float32)).reshape(n, k // gs)
    b = orc.f32_to_bf16(np.linspace(-0.3, 0.2, n * (k // gs)).astype(np.float32)).reshape(n, k // gs)
    ids = np.array([3, 0, 5, 1], np.uint32)
    got = orc.dequant_rows(words, s, b, k, bits, gs, ids)
    sf = orc.bf16_to_f32(s)[ids][:, np.arange(k) // gs]
    bf = orc.bf16_to_f32(b)[ids][:, np.arange(k) // gs]
    want = orc.f32_to_bf16((sf * codes_vals[ids].astype(np.float32)) + bf)
    assert (got == want).all()


@pytest.mark.parametrize("bits,gs,k,n,m", [(4, 64, 2048, 96, 1), (5, 64, 512, 64, 3),
                                           (6, 32, 1024, 40, 2), (8, 128, 2560, 48, 4),
                                           (4, 32, 256, 72, 8)])
def test_qmv_oracle_against_closed_form(orc, bits, gs, k, n, m):
    codes, s, b = orc.random_qweight(n, k, bits, gs, seed=1000 + bits)
    x = orc.fill_bf16(m * k, 5, 1, 1.0, 0.0).reshape(m, k)
    y = orc.bf16_to_f32(orc.qmv(codes, s, b, k, bits, gs, x))
    y64 = orc.qmv_f64(codes, s, b, k, bits, gs, x)
    mag = np.abs(orc.bf16_to_f32(x)).sum(axis=1, keepdims=True) * 0.23  # bound of |s q + b| sums
    # bf16 rounding (2^-9 relative) plus fp32 accumulation error
    assert (np.abs(y - y64) <= np.abs(y64) * 2.0 ** -8 + mag * 2.0 ** -18 + 1e-30).all()
    # a plausible indexing mistake (scales of the wrong group) is outside the bound
    s_bad = np.roll(s, 1, axis=1)
    y_bad = orc.qmv_f64(codes, s_bad, b, k, bits, gs, x)
    assert (np.abs(y_bad - y64) > np.abs(y64) * 2.0 ** -8 + mag * 2.0 ** -18).any()


def test_qmv_special_cases(orc):
    k, n, bits, gs = 512, 32, 4, 64
    codes, s, b = orc.random_qweight(n, k, bits, gs, seed=3)
    zero_x = np.zeros((2, k), np.uint16)
    assert (orc.qmv(codes, s, b, k, bits, gs, zero_x) == 0).all()
    # all codes zero: y = sum_g b_g * sum(x in g) up to rounding
    z = np.zeros_like(codes)
    x = orc.fill_bf16(k, 9, 1, 1.0, 0.0).reshape(1, k)
    y = orc.bf16_to_f32(orc.qmv(z, s, b, k, bits, gs, x))[0]
    xs = orc.bf16_to_f32(x)[0].astype(np.float64).reshape(-1, gs).sum(axis=1)
    want = (orc.bf16_to_f32(b).astype(np.float64) * xs[None, :]).sum(axis=1)
    assert np.allclose(y, want, rtol=2 ** -8, atol=1e-5)


def test_generator_statistics(orc):
    v = orc.bf16_to_f32(orc.fill_bf16(400000, 11, 1, 1.0, 0.0)).astype(np.float64)
    assert abs(v.mean()) < 0.01 and abs(v.std() - 1.0) < 0.01
    u = orc.bf16_to_f32(orc.fill_bf16(100000, 12, 0, 0.005, 0.03))
    # bf16 rounding may move the endpoints by half an ulp (2^-9 relative)
    assert u.min() >= 0.005 * (1 - 2 ** -9) and u.max() <= 0.03 * (1 + 2 ** -9)
    assert abs(u.mean() - 0.0175) < 2e-4
