"""The exact-integer projection on the int8 matrix cores (mx_xq) equals the
CPU oracle's mxo_xq bit for bit: config 0's matrix, the decode step's
projection shapes (router 513 x 2048, GDN input 12352 x 2048, K = 4096 rows
staged in 137 KiB of LDS, K = 8192 hyper-connection rows built in registers,
K = 256 up-projections), every code width at each of those depths, 1..8
activation rows, and
activations with exponents spread over many binades (the grid truncation)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _run(mx, orc, n, k, bits, m, seed, spread=False):
    w = mx.QWeight.random(n, k, bits, 64, seed=seed)
    codes, s, b = orc.random_qweight(n, k, bits, 64, seed=seed)
    rng = np.random.default_rng(seed)
    xf = rng.standard_normal((m, k)).astype(np.float32)
    if spread:
        xf *= (2.0 ** rng.integers(-40, 8, (m, k))).astype(np.float32)
    x = orc.f32_to_bf16(xf)
    dx = mx.DeviceArray.from_numpy(x)
    dy = mx.DeviceArray((m, n), np.uint16)
    qc = w.c()
    mx.check(mx.lib.mx_xq(C.byref(qc), dx.ptr, m, dy.ptr, None))
    got = dy.numpy()
    want = orc.f32_to_bf16(orc.xq(codes, s, b, k, bits, x))
    return got, want


@pytest.mark.parametrize("n,k,bits,m", [
    (4096, 2048, 4, 1),    # config 0
    (513, 2048, 4, 8),     # router + shared gate
    (12352, 2048, 4, 3),   # GDN qkv | z | a | b
    (2048, 4096, 4, 8),    # GDN / attention output (LDS staging of K = 4096)
    (260, 8192, 4, 5),     # hyper-connection down (register operands)
    (8192, 256, 4, 8),     # hyper-connection up
    (2048, 512, 5, 2),     # expert down width
    (512, 2048, 5, 8),
    (640, 1024, 6, 4),
    (512, 2048, 8, 7),
    (1000, 2048, 8, 1),    # head width, ragged n
    (64, 448, 4, 6),       # short rows: one slice of 7 groups
    # every width through the other row-major read forms: 8-bit batches of
    # four and eight (K = 1024, K = 2048 with n > 2048), and 5 / 6 / 8-bit at
    # K = 4096 (LDS staging) and K = 8192 (register and block operands)
    (4096, 2048, 8, 8),
    (640, 1024, 8, 4),
    (2048, 4096, 6, 3),
    (2048, 4096, 5, 8),
    (2048, 4096, 8, 2),
    (260, 8192, 5, 5),
    (260, 8192, 6, 8),
    (260, 8192, 8, 2),
    (8192, 256, 5, 8),
    (8192, 256, 6, 3),
])
def test_xq_bit_exact_with_oracle(mx, orc, n, k, bits, m):
    got, want = _run(mx, orc, n, k, bits, m, seed=n + k + bits + m)
    bad = np.argwhere(got != want)
    assert bad.size == 0, (bad[:5], got[tuple(bad[0])], want[tuple(bad[0])])


@pytest.mark.parametrize("bits", [4, 5, 8])
def test_xq_bit_exact_with_spread_exponents(mx, orc, bits):
    got, want = _run(mx, orc, 384, 2048, bits, 8, seed=77 + bits, spread=True)
    assert (got == want).all()


def test_xq_rows_are_independent(mx, orc):
    """Row r of an 8-row call equals a 1-row call on row r (batch invariance)."""
    n, k, bits = 1024, 2048, 4
    w = mx.QWeight.random(n, k, bits, 64, seed=5)
    x = orc.fill_bf16(8 * k, 6, 1, 1.0, 0.0).reshape(8, k)
    dx = mx.DeviceArray.from_numpy(x)
    y8 = mx.DeviceArray((8, n), np.uint16)
    qc = w.c()
    mx.check(mx.lib.mx_xq(C.byref(qc), dx.ptr, 8, y8.ptr, None))
    all8 = y8.numpy()
    for r in (0, 3, 7):
        d1 = mx.DeviceArray.from_numpy(np.ascontiguousarray(x[r:r + 1]))
        y1 = mx.DeviceArray((1, n), np.uint16)
        mx.check(mx.lib.mx_xq(C.byref(qc), d1.ptr, 1, y1.ptr, None))
        assert (y1.numpy()[0] == all8[r]).all()
