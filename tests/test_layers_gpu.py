"""GPU parity of the MoE, GatedDeltaNet and greedy-head kernels against the CPU
oracle, through the C ABI.  Bit-exact: kernels and oracle share one fixed
operation order.  Also checks the reference's own GDN fixture (tolerance) and
expert deduplication / batch invariance properties."""
import ctypes as C
import os

import numpy as np
import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(ROOT, "tests", "golden")


def bf(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def dev(mx, a):
    return mx.DeviceArray.from_numpy(np.ascontiguousarray(a))


# ------------------------------------------------------------------ routing --
@pytest.mark.parametrize("rows", [1, 3, 8])
@pytest.mark.parametrize("experts,top_k", [(512, 10), (64, 4), (128, 8)])
def test_route_bit_exact(mx, orc, rows, experts, top_k):
    lg = orc.fill_bf16(rows * experts, 300 + rows, 1, 2.0, 0.0).reshape(rows, experts)
    lg[0, :] = 0  # an all-tied row
    sl = orc.fill_bf16(rows, 301, 1, 2.0, 0.0)
    ids_w, sc_w, f_w = orc.moe_route(lg, sl, top_k)
    d_lg, d_sl = dev(mx, lg), dev(mx, sl)
    ids = mx.DeviceArray((rows, top_k), np.uint32)
    sc = mx.DeviceArray((rows, top_k), np.uint16)
    fa = mx.DeviceArray((rows,), np.uint16)
    mx.check(mx.lib.mx_moe_route(d_lg.ptr, experts, d_sl.ptr, 1, rows, experts, top_k, ids.ptr,
                                 sc.ptr, fa.ptr, None))
    assert (ids.numpy() == ids_w).all()
    assert (sc.numpy() == sc_w).all()
    assert (fa.numpy() == f_w).all()


# ------------------------------------------------------------------ experts --
class Moe:
    def __init__(self, mx, orc, E, I, H, seed, sI=None, gbits=4, dbits=5):
        sI = sI or I
        self.E, self.I, self.H = E, I, H
        self.gate = mx.QBank.random(E, I, H, gbits, 64, seed)
        self.up = mx.QBank.random(E, I, H, gbits, 64, seed + 10)
        self.down = mx.QBank.random(E, H, I, dbits, 64, seed + 20)
        self.sg = mx.QWeight.random(sI, H, gbits, 64, seed + 30)
        self.su = mx.QWeight.random(sI, H, gbits, 64, seed + 40)
        self.sd = mx.QWeight.random(H, sI, dbits, 64, seed + 50)
        self.h_host = [b.host() for b in (self.gate, self.up, self.down)]
        self.s_host = [w.host() for w in (self.sg, self.su, self.sd)]
        g, u, d = self.h_host
        self.o_banks = [orc.qbank(*g, E, I, H, gbits, 64), orc.qbank(*u, E, I, H, gbits, 64),
                        orc.qbank(*d, E, H, I, dbits, 64)]
        sg, su, sd = self.s_host
        self.o_shared = [orc.qw(*sg, sI, H, gbits, 64), orc.qw(*su, sI, H, gbits, 64),
                         orc.qw(*sd, H, sI, dbits, 64)]
        self.ws_bytes = mx.lib.mx_moe_workspace_bytes(8, 16, max(I, sI))
        self.ws = mx.DeviceArray((self.ws_bytes,), np.uint8)

    def run(self, mx, x, ids, scores, top_k):
        rows = x.shape[0]
        p = mx.DeviceArray((rows, top_k + 1, self.H), np.uint16)
        qb = [b.c() for b in (self.gate, self.up, self.down)]
        qs = [w.c() for w in (self.sg, self.su, self.sd)]
        dx, di, ds = dev(mx, x), dev(mx, ids), dev(mx, scores)
        mx.check(mx.lib.mx_moe_experts(dx.ptr, di.ptr, ds.ptr, rows, top_k, C.byref(qb[0]),
                                       C.byref(qb[1]), C.byref(qb[2]), C.byref(qs[0]),
                                       C.byref(qs[1]), C.byref(qs[2]), self.ws.ptr, p.ptr, None))
        return p.numpy()

    def oracle(self, orc, x, ids, scores, top_k):
        return orc.moe_experts(x, ids, scores, top_k, *self.o_banks, *self.o_shared, self.H)


@pytest.mark.parametrize("rows", [1, 2, 5, 8])
def test_experts_bit_exact_with_shared_experts_across_rows(mx, orc, rows):
    E, I, H, top_k = 16, 64, 512, 4
    m = Moe(mx, orc, E, I, H, seed=400, sI=128)
    rng = np.random.default_rng(rows)
    # few experts for many routes: heavy deduplication across rows
    ids = np.stack([rng.choice(6, top_k, replace=False) for _ in range(rows)]).astype(np.uint32)
    scores = orc.f32_to_bf16(rng.uniform(0.05, 0.5, (rows, top_k)).astype(np.float32))
    x = orc.fill_bf16(rows * H, 410 + rows, 1, 1.0, 0.0).reshape(rows, H)
    got = m.run(mx, x, ids, scores, top_k)
    want = m.oracle(orc, x, ids, scores, top_k)
    assert (got == want).all(), np.argwhere(got != want)[:5]


def test_experts_config2_shapes_and_batch_invariance(mx, orc):
    """benchmark config 2 geometry: 512 experts, inter 512, hidden 2048, top-10,
    4-bit gate/up, 5-bit down; rows routed by the router tail."""
    E, I, H, top_k = 512, 512, 2048, 10
    m = Moe(mx, orc, E, I, H, seed=500)
    rows = 8
    x = orc.fill_bf16(rows * H, 501, 1, 1.0, 0.0).reshape(rows, H)
    router = mx.QWeight.random(E + 1, H, 4, 64, 502)
    logits = mx.DeviceArray((rows, E + 1), np.uint16)
    dx = dev(mx, x)
    mx.qmv(router, dx, rows, logits)
    lg = logits.numpy()
    ids, scores, factor = orc.moe_route(np.ascontiguousarray(lg[:, :E]), lg[:, E], top_k)
    got = m.run(mx, x, ids, scores, top_k)
    want = m.oracle(orc, x, ids, scores, top_k)
    assert (got == want).all()
    # each row alone gives the same bits as inside the batch of eight
    for r in (0, 5):
        one = m.run(mx, x[r:r + 1], ids[r:r + 1], scores[r:r + 1], top_k)
        assert (one[0] == got[r]).all()


def test_reduce_and_epilogue_bit_exact(mx, orc):
    rows, top_k, H, hc = 5, 10, 2048, 4
    rng = np.random.default_rng(13)
    p = orc.f32_to_bf16(rng.standard_normal((rows, top_k + 1, H)).astype(np.float32))
    factor = orc.f32_to_bf16(rng.uniform(0, 1, rows).astype(np.float32))
    residual = orc.f32_to_bf16(rng.standard_normal((rows, hc * H)).astype(np.float32) * 3)
    gate = orc.f32_to_bf16(rng.uniform(0, 2, (rows, hc)).astype(np.float32))
    routed_w = orc.moe_reduce(p, top_k)
    shared = np.ascontiguousarray(p[:, top_k, :])
    out_w = orc.moe_hc_epilogue(routed_w, shared, factor, residual, gate, hc)
    dp, df, dr, dg = dev(mx, p), dev(mx, factor), dev(mx, residual), dev(mx, gate)
    routed = mx.DeviceArray((rows, H), np.uint16)
    mx.check(mx.lib.mx_moe_reduce(dp.ptr, rows, top_k, H, routed.ptr, None))
    assert (routed.numpy() == routed_w).all()
    out = mx.DeviceArray((rows, hc * H), np.uint16)
    dsh = dev(mx, shared)
    mx.check(mx.lib.mx_moe_hc_epilogue(routed.ptr, dsh.ptr, df.ptr, dr.ptr, dg.ptr, rows, hc, H,
                                       out.ptr, None))
    assert (out.numpy() == out_w).all()
    fused = mx.DeviceArray((rows, hc * H), np.uint16)
    mx.check(mx.lib.mx_moe_reduce_hc_epilogue(dp.ptr, df.ptr, dr.ptr, dg.ptr, rows, top_k, hc, H,
                                              fused.ptr, None))
    assert (fused.numpy() == out_w).all()
    # in place (out aliases residual), as the engine uses it
    mx.check(mx.lib.mx_moe_reduce_hc_epilogue(dp.ptr, df.ptr, dr.ptr, dg.ptr, rows, top_k, hc, H,
                                              dr.ptr, None))
    assert (dr.numpy() == out_w).all()


# ---------------------------------------------------------------------- GDN --
def gdn_dims(mx, hk, hv, conv_k=4):
    return mx.GdnDimsC(hk, hv, 128, 128, conv_k)


@pytest.mark.parametrize("groups,t", [(1, 1), (8, 1), (1, 4), (2, 3)])
def test_gdn_conv_bit_exact(mx, orc, groups, t):
    C_, K, S = 8192, 4, 10
    rng = np.random.default_rng(groups * 10 + t)
    stride = C_ + 96  # rows of a fused projection output
    qkv = orc.f32_to_bf16(rng.standard_normal((groups * t, stride)).astype(np.float32))
    state = orc.f32_to_bf16(rng.standard_normal((S, K - 1, C_)).astype(np.float32))
    w = (rng.standard_normal((K, C_)) * 0.4).astype(np.float32)
    slots = rng.choice(S, groups, replace=False).astype(np.int32)
    out_w, st_w, hist_w = orc.gdn_conv(np.ascontiguousarray(qkv[:, :C_]), groups, t, slots, state,
                                       w, window_history=True)
    dq, dst, dw, ds = dev(mx, qkv), dev(mx, state), dev(mx, w), dev(mx, slots)
    out = mx.DeviceArray((groups * t, C_), np.uint16)
    hist = mx.DeviceArray((groups, K - 1 + t, C_), np.uint16)
    mx.check(mx.lib.mx_gdn_conv(dq.ptr, stride, groups, t, ds.ptr, dst.ptr, dw.ptr, C_, K, out.ptr,
                                C_, hist.ptr, None))
    assert (out.numpy() == out_w).all()
    assert (dst.numpy() == st_w).all()
    assert (hist.numpy() == hist_w).all()


@pytest.mark.parametrize("groups,t,K", [(1, 256, 4), (2, 100, 4), (1, 17, 8), (1, 40, 2)])
def test_gdn_conv_long_runs_bit_exact(mx, orc, groups, t, K):
    """Runs longer than 16 tokens without a window history (prefill chunks)
    spread their tokens over workgroups; same bits as the oracle's sequential
    conv, cached window included."""
    C_, S = 8192, 6
    rng = np.random.default_rng(groups * 1000 + t + K)
    stride = C_ + 32
    qkv = orc.f32_to_bf16(rng.standard_normal((groups * t, stride)).astype(np.float32))
    state = orc.f32_to_bf16(rng.standard_normal((S, K - 1, C_)).astype(np.float32))
    w = (rng.standard_normal((K, C_)) * 0.4).astype(np.float32)
    slots = rng.choice(S, groups, replace=False).astype(np.int32)
    out_w, st_w, _ = orc.gdn_conv(np.ascontiguousarray(qkv[:, :C_]), groups, t, slots, state, w)
    dq, dst, dw, ds = dev(mx, qkv), dev(mx, state), dev(mx, w), dev(mx, slots)
    out = mx.DeviceArray((groups * t, C_), np.uint16)
    mx.check(mx.lib.mx_gdn_conv(dq.ptr, stride, groups, t, ds.ptr, dst.ptr, dw.ptr, C_, K, out.ptr,
                                C_, None, None))
    assert (out.numpy() == out_w).all()
    assert (dst.numpy() == st_w).all()


def _gdn_inputs(orc, rows, hk, hv, seed):
    rng = np.random.default_rng(seed)
    conv = orc.f32_to_bf16(rng.standard_normal((rows, 2 * hk * 128 + hv * 128)).astype(np.float32))
    z = orc.f32_to_bf16(rng.standard_normal((rows, hv * 128)).astype(np.float32))
    a = orc.f32_to_bf16(rng.standard_normal((rows, hv)).astype(np.float32))
    b = orc.f32_to_bf16(rng.standard_normal((rows, hv)).astype(np.float32))
    a_log = np.log(rng.uniform(0.01, 16, hv)).astype(np.float32)
    dt = orc.f32_to_bf16(rng.uniform(-1, 1, hv).astype(np.float32))
    norm_w = orc.f32_to_bf16(rng.uniform(0.5, 1.5, 128).astype(np.float32))
    return conv, z, a, b, a_log, dt, norm_w


@pytest.mark.parametrize("groups,t,history", [(1, 1, False), (2, 1, False), (4, 1, False),
                                              (8, 1, False), (1, 4, True), (2, 3, True)])
def test_gdn_recurrence_bit_exact(mx, orc, groups, t, history):
    hk, hv, S = 16, 32, 9
    rows = groups * t
    conv, z, a, b, a_log, dt, norm_w = _gdn_inputs(orc, rows, hk, hv, groups * 7 + t)
    rng = np.random.default_rng(99)
    state = (rng.standard_normal((S, hv, 128, 128)) * 0.05).astype(np.float32)
    slots = rng.choice(S, groups, replace=False).astype(np.int32)
    eps = 1e-6
    y_w, st_w, h_w = orc.gdn_recurrence(conv, z, a, b, a_log, dt, norm_w, eps, hk, hv, groups, t,
                                        slots, state, history=history)
    zab = np.ascontiguousarray(np.concatenate([z, a, b], axis=1))
    dzab = dev(mx, zab)
    zs = zab.shape[1]
    dconv, dal, ddt, dnw, dsl, dst = (dev(mx, v) for v in (conv, a_log, dt, norm_w, slots, state))
    y = mx.DeviceArray((rows, hv * 128), np.uint16)
    hist = mx.DeviceArray((rows, hv, 128, 128), np.float32) if history else None
    dims = gdn_dims(mx, hk, hv)
    mx.check(mx.lib.mx_gdn_recurrence(dconv.ptr, conv.shape[1], dzab.ptr, dzab.ptr + 2 * hv * 128,
                                      dzab.ptr + 2 * (hv * 128 + hv), zs, dal.ptr, ddt.ptr,
                                      dnw.ptr, eps, C.byref(dims), groups, t, dsl.ptr, dst.ptr,
                                      hist.ptr if hist else None, y.ptr, None))
    assert (y.numpy() == y_w).all(), np.argwhere(y.numpy() != y_w)[:5]
    assert (dst.numpy() == st_w).all()
    if history:
        assert (hist.numpy() == h_w).all()


def test_gdn_scan_reference_fixture_and_oracle(mx, orc):
    f = np.load(os.path.join(GOLDEN, "gdn_native_kernels_subset.npz"))
    hk, hv = 2, 6
    init = np.ascontiguousarray(f["initial"][0].transpose(0, 2, 1))[None]
    args = [f["q"].reshape(1, hk, 128), f["k"].reshape(1, hk, 128), f["v"].reshape(1, hv, 128),
            f["g"].reshape(1, hv), f["beta"].reshape(1, hv)]
    y_w, st_w, _ = orc.gdn_scan(*args, hk, hv, 1, 1, np.zeros(1, np.int32), init)
    dq, dk, dv, dg, db = (dev(mx, np.ascontiguousarray(a)) for a in args)
    dst, dsl = dev(mx, init), dev(mx, np.zeros(1, np.int32))
    y = mx.DeviceArray((1, hv, 128), np.uint16)
    dims = gdn_dims(mx, hk, hv)
    mx.check(mx.lib.mx_gdn_scan(dq.ptr, dk.ptr, dv.ptr, dg.ptr, db.ptr, C.byref(dims), 1, 1,
                                dsl.ptr, dst.ptr, None, y.ptr, None))
    assert (y.numpy() == y_w).all()
    assert (dst.numpy() == st_w).all()
    # against the reference's MLX/Metal outputs: fp32 state 1e-4 relative,
    # bf16 y within 2e-2 relative / 1e-2 absolute
    want_state = f["state"][0].transpose(0, 2, 1)
    assert np.abs(dst.numpy()[0] - want_state).max() <= 1e-4 * np.abs(want_state).max()
    yw = bf(f["y"].reshape(hv, 128))
    assert np.all(np.abs(bf(y.numpy().reshape(hv, 128)) - yw) <= 1e-2 + 2e-2 * np.abs(yw))


# --------------------------------------------------------------------- head --
@pytest.mark.parametrize("m", [1, 3, 8])
def test_head_argmax_bit_exact(mx, orc, m):
    n, k = 151936, 2048
    w = mx.QWeight.random(n, k, 8, 64, 600)
    c, s, b = w.host()
    x = orc.fill_bf16(m * k, 601 + m, 1, 1.0, 0.0).reshape(m, k)
    dx = dev(mx, x)
    ws = mx.DeviceArray((mx.lib.mx_head_workspace_bytes(n, k, m),), np.uint8)
    tok = mx.DeviceArray((m,), np.uint32)
    qc = w.c()
    mx.check(mx.lib.mx_head_argmax(C.byref(qc), dx.ptr, m, tok.ptr, ws.ptr, None))
    want = orc.head_argmax(orc.qw(c, s, b, n, k, 8, 64), x)
    assert (tok.numpy() == want).all()
    # the logits path (QMV + argmax over bf16 logits) selects the same tokens
    logits = mx.DeviceArray((m, n), np.uint16)
    mx.qmv(w, dx, m, logits)
    tok2 = mx.DeviceArray((m,), np.uint32)
    mx.check(mx.lib.mx_argmax_bf16(logits.ptr, m, n, tok2.ptr, None))
    assert (tok2.numpy() == want).all()


def test_argmax_extremes(mx, orc):
    n = 31040
    rows = np.zeros((4, n), np.float32)
    rows[0] = -np.inf
    rows[1] = np.nan
    rows[1, 777] = 2.0
    rows[2, 50] = np.inf
    rows[2, 1000] = np.inf
    rows[3] = -0.0
    lg = orc.f32_to_bf16(rows)
    d = dev(mx, lg)
    tok = mx.DeviceArray((4,), np.uint32)
    mx.check(mx.lib.mx_argmax_bf16(d.ptr, 4, n, tok.ptr, None))
    assert list(tok.numpy()) == [0, 777, 50, 0]


@pytest.mark.parametrize("groups", [1, 8])
def test_gdn_recurrence_fast_within_tolerance(mx, orc, groups):
    """Fast-mode single-token step (hardware exp2 / log2 / rsqrt, wave-local q/k
    norms) against the oracle's fixed-order step on the same inputs: the fp32
    state within 1e-4 relative per element (|d| <= 1e-4 max(|w|, 1e-2 rms)
    per head, the floor covering entries that cancel to near zero), y within
    2e-2 relative / 1e-2 absolute."""
    hk, hv, S = 16, 32, 9
    conv, z, a, b, a_log, dt, norm_w = _gdn_inputs(orc, groups, hk, hv, 900 + groups)
    rng = np.random.default_rng(98)
    state = (rng.standard_normal((S, hv, 128, 128)) * 0.05).astype(np.float32)
    slots = rng.choice(S, groups, replace=False).astype(np.int32)
    eps = 1e-6
    y_w, st_w, _ = orc.gdn_recurrence(conv, z, a, b, a_log, dt, norm_w, eps, hk, hv, groups, 1,
                                      slots, state)
    zab = np.ascontiguousarray(np.concatenate([z, a, b], axis=1))
    dzab = dev(mx, zab)
    dconv, dal, ddt, dnw, dsl, dst = (dev(mx, v) for v in (conv, a_log, dt, norm_w, slots, state))
    y = mx.DeviceArray((groups, hv * 128), np.uint16)
    dims = gdn_dims(mx, hk, hv)
    mx.check(mx.lib.mx_gdn_recurrence_fast(dconv.ptr, conv.shape[1], dzab.ptr,
                                           dzab.ptr + 2 * hv * 128, dzab.ptr + 2 * (hv * 128 + hv),
                                           zab.shape[1], dal.ptr, ddt.ptr, dnw.ptr, eps,
                                           C.byref(dims), groups, 1, dsl.ptr, dst.ptr, None, y.ptr,
                                           None))
    st = dst.numpy().astype(np.float64)
    w64 = st_w.astype(np.float64)
    rms = np.sqrt((w64 ** 2).mean(axis=(2, 3), keepdims=True))
    ratio = np.abs(st - w64) / (1e-4 * np.maximum(np.abs(w64), 1e-2 * rms))
    print(f"fast GDN state: worst error / bound {ratio.max():.3f}, "
          f"entries above 1e-4 relative {(np.abs(st - w64) > 1e-4 * np.abs(w64)).mean():.2e}")
    assert ratio.max() <= 1.0
    got, want = bf(y.numpy()).astype(np.float64), bf(y_w).astype(np.float64)
    assert np.all(np.abs(got - want) <= 2e-2 * np.abs(want) + 1e-2)


@pytest.mark.parametrize("groups,t", [(1, 4), (2, 3), (1, 8)])
def test_gdn_recurrence_fast_block_equals_one_token_steps(mx, orc, groups, t):
    """A fast-mode block of t tokens per group (the engine's verify and prefill
    form, the kernel's looping instance) gives the bits of t one-token fast
    calls (the decode step, its loop-free instance): every y row, the history's
    state after every token, and the final cached state.  Speculative
    decoding's greedy acceptance is lossless only with this."""
    hk, hv, S = 16, 32, 6
    rows = groups * t
    conv, z, a, b, a_log, dt, norm_w = _gdn_inputs(orc, rows, hk, hv, 700 + rows)
    rng = np.random.default_rng(97)
    state = (rng.standard_normal((S, hv, 128, 128)) * 0.05).astype(np.float32)
    slots = rng.choice(S, groups, replace=False).astype(np.int32)
    zab = np.ascontiguousarray(np.concatenate([z, a, b], axis=1))
    cs, zs = conv.shape[1], zab.shape[1]
    dims = gdn_dims(mx, hk, hv)
    eps = 1e-6
    dconv, dzab, dal, ddt, dnw, dsl = (dev(mx, v) for v in (conv, zab, a_log, dt, norm_w, slots))

    def call(r0, g, tt, slot_ptr, st, hist, y):
        zp = dzab.ptr + 2 * r0 * zs
        mx.check(mx.lib.mx_gdn_recurrence_fast(dconv.ptr + 2 * r0 * cs, cs, zp, zp + 2 * hv * 128,
                                               zp + 2 * (hv * 128 + hv), zs, dal.ptr, ddt.ptr,
                                               dnw.ptr, eps, C.byref(dims), g, tt, slot_ptr,
                                               st.ptr, hist, y.ptr, None))

    st_b = dev(mx, state)
    hist = mx.DeviceArray((rows, hv, 128, 128), np.float32)
    y_b = mx.DeviceArray((rows, hv * 128), np.uint16)
    call(0, groups, t, dsl.ptr, st_b, hist.ptr, y_b)
    st_s = dev(mx, state)
    y_s = mx.DeviceArray((1, hv * 128), np.uint16)
    y_want = np.empty((rows, hv * 128), np.uint16)
    h_want = np.empty((rows, hv, 128, 128), np.float32)
    for step in range(t):
        for g in range(groups):
            r = g * t + step
            call(r, 1, 1, dsl.ptr + 4 * g, st_s, None, y_s)
            y_want[r] = y_s.numpy()[0]
            h_want[r] = st_s.numpy()[slots[g]]
    assert (y_b.numpy() == y_want).all()
    assert (hist.numpy() == h_want).all()
    assert (st_b.numpy() == st_s.numpy()).all()
    assert not (st_b.numpy()[slots] == state[slots]).all()
