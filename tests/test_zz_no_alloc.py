"""mx_head_argmax_noalloc (partials in a static device array, no workspace,
no allocation) against mx_head_argmax (partials in a caller workspace)
through the C ABI, bit for bit: two calls in a row on the static array, the
second with a smaller head and fewer rows (the array keeps the first call's
partials; the second reads only what it writes)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# (vocabulary rows, k, bits, activation rows, seed): config 3's head, then a
# smaller one
CASES = [(151936, 2048, 8, 8, 31), (40000, 1024, 4, 3, 32)]


def _inputs(mx, orc, n, k, bits, m, seed):
    w = mx.QWeight.random(n, k, bits, 64, seed=seed)
    x = mx.DeviceArray.from_numpy(orc.fill_bf16(m * k, seed + 1, 1, 1.0, 0.0).reshape(m, k))
    return w, x


def test_noalloc_head_equals_workspace_head_on_two_calls(mx, orc):
    assert mx.lib.mx_head_noalloc_max_bytes() == 1 << 20
    ins = [_inputs(mx, orc, *c) for c in CASES]
    got = []
    for (n, k, bits, m, seed), (w, x) in zip(CASES, ins):
        print(f"noalloc head n={n} k={k} bits={bits} m={m}", flush=True)
        assert mx.lib.mx_head_workspace_bytes(n, k, m) <= mx.lib.mx_head_noalloc_max_bytes()
        qc = w.c()
        toks = mx.DeviceArray((m,), np.uint32)
        mx.check(mx.lib.mx_head_argmax_noalloc(C.byref(qc), x.ptr, m, toks.ptr, None))
        mx.sync()
        got.append(toks.numpy())
    for (n, k, bits, m, seed), (w, x), g in zip(CASES, ins, got):
        qc = w.c()
        toks = mx.DeviceArray((m,), np.uint32)
        ws = mx.DeviceArray((mx.lib.mx_head_workspace_bytes(n, k, m),), np.uint8)
        mx.check(mx.lib.mx_head_argmax(C.byref(qc), x.ptr, m, toks.ptr, ws.ptr, None))
        mx.sync()
        assert (g == toks.numpy()).all(), (n, g, toks.numpy())
