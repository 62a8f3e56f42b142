"""Chunked GatedDeltaNet prefill (mx_gdn_prefill_chunked) against the
sequential fp32 delta rule of the CPU oracle (the reference's recurrent
kernel, token by token) and the GPU sequential scan (mx_gdn_scan): the fp32
state within 1e-4 relative (max norm) and y within 2e-2 relative / 1e-2
absolute, the north star's tolerances.  Covers a single chunk, a partial last
chunk, two sequences at once, a non-zero initial state, decays down to zero
(a reset inside a chunk) and benchmark config 1's prefill (T = 2048, 16 key /
32 value heads)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def bf(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def inputs(orc, rows, hk, hv, seed, zero_decay_at=None):
    """Config-1 style inputs: L2-normalised q, k; beta = sigmoid(N(0,1));
    g = exp(-softplus(N(0,1)) * A) with A ~ U(0, 16) per head."""
    rng = np.random.default_rng(seed)

    def l2n(x):
        return x / np.linalg.norm(x, axis=-1, keepdims=True)

    q = orc.f32_to_bf16(l2n(rng.standard_normal((rows, hk, 128))).astype(np.float32))
    k = orc.f32_to_bf16(l2n(rng.standard_normal((rows, hk, 128))).astype(np.float32))
    v = orc.f32_to_bf16(rng.standard_normal((rows, hv, 128)).astype(np.float32))
    beta = orc.f32_to_bf16((1 / (1 + np.exp(-rng.standard_normal((rows, hv))))).astype(np.float32))
    A = rng.uniform(0, 16, hv)
    g = np.exp(-np.log1p(np.exp(rng.standard_normal((rows, hv)))) * A).astype(np.float32)
    if zero_decay_at is not None:
        g[zero_decay_at] = 0.0
    return q, k, v, g, beta


def run_chunked(mx, q, k, v, g, beta, hk, hv, groups, t, slots, state):
    dims = mx.GdnDimsC(hk, hv, 128, 128, 4)
    dq, dk, dv_, dg, db, dsl, dst = (mx.DeviceArray.from_numpy(np.ascontiguousarray(a))
                                     for a in (q, k, v, g, beta, slots, state))
    y = mx.DeviceArray((groups * t, hv, 128), np.uint16)
    ws = mx.DeviceArray((mx.lib.mx_gdn_prefill_workspace_bytes(groups, hv, t),), np.uint8)
    mx.check(mx.lib.mx_gdn_prefill_chunked(dq.ptr, dk.ptr, dv_.ptr, dg.ptr, db.ptr, C.byref(dims),
                                           groups, t, dsl.ptr, dst.ptr, y.ptr, ws.ptr, None))
    return y.numpy(), dst.numpy()


def check(y, st, y_w, st_w):
    assert np.abs(st - st_w).max() <= 1e-4 * np.abs(st_w).max(), np.abs(st - st_w).max()
    a, b = bf(y).astype(np.float64), bf(y_w).astype(np.float64)
    assert np.all(np.abs(a - b) <= 2e-2 * np.abs(b) + 1e-2), np.abs(a - b).max()


@pytest.mark.parametrize("hk,hv,groups,t,init", [(2, 4, 1, 64, False), (2, 4, 1, 100, True),
                                                 (1, 2, 2, 200, True), (2, 2, 1, 129, True)])
def test_prefill_chunked_matches_sequential_oracle(mx, orc, hk, hv, groups, t, init):
    rows = groups * t
    q, k, v, g, beta = inputs(orc, rows, hk, hv, 500 + t, zero_decay_at=(min(70, rows - 1), 0))
    S = 3
    rng = np.random.default_rng(7)
    state = ((rng.standard_normal((S, hv, 128, 128)) * 0.1) if init
             else np.zeros((S, hv, 128, 128))).astype(np.float32)
    slots = np.array([2, 0][:groups], np.int32)
    y_w, st_w, _ = orc.gdn_scan(q, k, v, g, beta, hk, hv, groups, t, slots, state)
    y, st = run_chunked(mx, q, k, v, g, beta, hk, hv, groups, t, slots, state)
    check(y, st, y_w, st_w)
    # slots not named stay untouched
    untouched = [s for s in range(S) if s not in slots]
    assert (st[untouched] == state[untouched]).all()


def test_prefill_chunked_config1_t2048(mx, orc):
    """benchmark config 1 prefill: T = 2048, B = 1, 16 key / 32 value heads,
    zero initial state; against the oracle and the GPU sequential scan."""
    hk, hv, t = 16, 32, 2048
    q, k, v, g, beta = inputs(orc, t, hk, hv, 2048)
    state = np.zeros((1, hv, 128, 128), np.float32)
    slots = np.zeros(1, np.int32)
    y_w, st_w, _ = orc.gdn_scan(q, k, v, g, beta, hk, hv, 1, t, slots, state)
    y, st = run_chunked(mx, q, k, v, g, beta, hk, hv, 1, t, slots, state)
    check(y, st, y_w, st_w)
    # the GPU sequential scan on the same inputs
    dims = mx.GdnDimsC(hk, hv, 128, 128, 4)
    dq, dk, dv_, dg, db, dsl, dst = (mx.DeviceArray.from_numpy(np.ascontiguousarray(a))
                                     for a in (q, k, v, g, beta, slots, state))
    ys = mx.DeviceArray((t, hv, 128), np.uint16)
    mx.check(mx.lib.mx_gdn_scan(dq.ptr, dk.ptr, dv_.ptr, dg.ptr, db.ptr, C.byref(dims), 1, t,
                                dsl.ptr, dst.ptr, None, ys.ptr, None))
    check(y, st, ys.numpy(), dst.numpy())
