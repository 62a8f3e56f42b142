"""The oracle's unquantised bf16 GEMV (A16, src/gemv_kernel.rs:30-90) pinned
independently of its summation order: the float64 closed form within fp32-sum
plus bf16-output tolerance; a one-hot x selects one weight column exactly;
small-integer inputs (every partial sum exact in fp32) give the exact integer
dot product, which any dropped term, wrong index or transposed operand breaks."""
import numpy as np
import pytest


def bf(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("n,k,rows", [(64, 128, 1), (512, 2048, 8), (100, 640, 3)])
def test_gemv_closed_form(orc, n, k, rows):
    rng = np.random.default_rng(n + k)
    w = orc.f32_to_bf16(rng.standard_normal((n, k)).astype(np.float32) * 0.05)
    x = orc.f32_to_bf16(rng.standard_normal((rows, k)).astype(np.float32))
    y = bf(orc.gemv_bf16(w, x)).astype(np.float64)
    ref = bf(x).astype(np.float64) @ bf(w).astype(np.float64).T
    mag = np.abs(bf(x)).astype(np.float64) @ np.abs(bf(w)).astype(np.float64).T
    assert np.all(np.abs(y - ref) <= 2.0 ** -8 * np.abs(ref) + 2.0 ** -20 * mag + 1e-30)


def test_gemv_one_hot_and_integer_exact(orc):
    rng = np.random.default_rng(5)
    n, k = 48, 384
    w = orc.f32_to_bf16(rng.standard_normal((n, k)).astype(np.float32))
    x = np.zeros((3, k), np.uint16)
    for r, kk in enumerate((0, 131, 383)):
        x[r, kk] = orc.f32_to_bf16(np.array([1.0], np.float32))[0]
    y = orc.gemv_bf16(w, x)
    for r, kk in enumerate((0, 131, 383)):
        assert (y[r] == w[:, kk]).all()
    wi = rng.integers(-8, 9, (n, k)).astype(np.float32)
    xi = rng.integers(-8, 9, (4, k)).astype(np.float32)
    y = bf(orc.gemv_bf16(orc.f32_to_bf16(wi), orc.f32_to_bf16(xi)))
    # |partial sums| <= 384 * 64 < 2^24: exact in fp32, so the only rounding
    # is the final one to bf16
    exact = xi.astype(np.int64) @ wi.astype(np.int64).T
    want = bf(orc.f32_to_bf16(exact.astype(np.float32)))
    assert (y == want).all()
