"""Unquantised bf16 GEMV (mx_gemv_bf16, A16): bit-exact with the oracle's
restated order for 1..8 rows, and each row of a batched call equals the
single-row call (the reference's shared_unquantized_rows_preserve_native_
singleton_tree property, src/gemv_kernel.rs tests)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,k", [(512, 2048), (64, 128), (1000, 2560), (13, 256)])
def test_gemv_bit_exact_and_row_invariant(mx, orc, n, k):
    rng = np.random.default_rng(n * 7 + k)
    w = orc.f32_to_bf16(rng.standard_normal((n, k)).astype(np.float32) * 0.05)
    x = orc.f32_to_bf16(rng.standard_normal((8, k)).astype(np.float32))
    dw = mx.DeviceArray.from_numpy(w)
    single = []
    for r in range(8):
        dx = mx.DeviceArray.from_numpy(np.ascontiguousarray(x[r:r + 1]))
        dy = mx.DeviceArray((1, n), np.uint16)
        mx.check(mx.lib.mx_gemv_bf16(dw.ptr, n, k, dx.ptr, 1, dy.ptr, None))
        single.append(dy.numpy()[0])
    for rows in (1, 2, 5, 8):
        dx = mx.DeviceArray.from_numpy(np.ascontiguousarray(x[:rows]))
        dy = mx.DeviceArray((rows, n), np.uint16)
        mx.check(mx.lib.mx_gemv_bf16(dw.ptr, n, k, dx.ptr, rows, dy.ptr, None))
        got = dy.numpy()
        assert (got == orc.gemv_bf16(w, x[:rows])).all(), rows
        for r in range(rows):
            assert (got[r] == single[r]).all(), (rows, r)
