"""Pins the oracle's MoE, GatedDeltaNet and greedy-head restatements (CPU only)
against the reference's held fixture, closed forms in float64, special cases
and an independent restatement of the reference kernels' control flow."""
import os

import numpy as np
import pytest

from conftest import ROOT

GOLDEN = os.path.join(ROOT, "tests", "golden")


def bf(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_bf(orc, f):
    return orc.f32_to_bf16(np.asarray(f, np.float32))


# ------------------------------------------------------------------ routing --
def test_route_all_equal_logits_pick_highest_ids(orc):
    """Equal gates tie in bf16: the (value, index) key picks the ten highest
    expert ids, slot k-1 the largest (kernels/moe_route_tail.metal:80-100)."""
    logits = np.zeros((3, 512), np.uint16)
    ids, scores, factor = orc.moe_route(logits, np.zeros(3, np.uint16), 10)
    assert (ids == np.arange(502, 512, dtype=np.uint32)[None, :]).all()
    # each gate is bf16(1/512) = 2^-9; ten bf16 adds are exact; 1/10 -> bf16(0.1)
    assert (scores == 0x3DCD).all()
    assert (factor == to_bf(orc, [0.5])[0]).all()


def test_route_phase_pattern_and_monotone_logits(orc):
    # strictly increasing logits: the top ten are the last ten ids, ascending
    lg = to_bf(orc, np.linspace(-4, 4, 512)).reshape(1, 512)
    ids, scores, _ = orc.moe_route(lg, to_bf(orc, [0.0]), 10)
    assert (ids[0] == np.arange(502, 512)).all()
    assert (np.diff(bf(scores[0])) >= 0).all()
    # phase pattern in the spirit of the reference test (moe_route.rs:91-98)
    rows = 8
    x = np.array([[np.sin(0.37 * e + 1.3 * r) * 3.0 + 0.01 * e for e in range(512)]
                  for r in range(rows)])
    lg = to_bf(orc, x)
    sl = to_bf(orc, np.linspace(-3, 3, rows))
    ids, scores, factor = orc.moe_route(lg, sl, 10)
    g64 = np.exp(bf(lg).astype(np.float64) - bf(lg).max(axis=1, keepdims=True))
    g64 /= g64.sum(axis=1, keepdims=True)
    gb = bf(to_bf(orc, g64.astype(np.float32)))
    for r in range(rows):
        # the selection is the top ten under (bf16 gate, id); allow a one-ulp
        # disagreement of the f64 gates only exactly at the tenth-place boundary
        key = gb[r].astype(np.float64) * 1024 + np.arange(512) / 1024.0
        want = np.sort(np.argsort(key)[-10:])
        got = np.sort(ids[r])
        if not (got == want).all():
            tenth = np.sort(gb[r])[-10]
            diff = set(got) ^ set(want)
            assert all(abs(gb[r][d] - tenth) <= tenth * 2 ** -7 for d in diff)
        # slot order ascending by key and scores sum to ~1
        assert (np.diff(bf(scores[r])) >= 0).all()
        assert abs(bf(scores[r]).astype(np.float64).sum() - 1.0) < 0.03
    want_f = 1 / (1 + np.exp(-bf(sl).astype(np.float64)))
    assert np.allclose(bf(factor), want_f, rtol=2 ** -7, atol=2 ** -9)


# ------------------------------------------------------------------ experts --
def _bank(orc, experts, n, k, bits, gs, seed):
    c, s, b = orc.random_qweight(experts * n, k, bits, gs, seed)
    return (c, s, b), orc.qbank(c, s, b, experts, n, k, bits, gs)


def _qw(orc, n, k, bits, gs, seed):
    c, s, b = orc.random_qweight(n, k, bits, gs, seed)
    return (c, s, b), orc.qw(c, s, b, n, k, bits, gs)


def _mlp64(orc, g3, u3, d3, xrow, H, I, gbits, dbits):
    """SwiGLU expert in float64 with only h rounded to bf16 (the down input)."""
    g = orc.qmv_f64(*g3, H, gbits, 64, xrow)[0]
    u = orc.qmv_f64(*u3, H, gbits, 64, xrow)[0]
    hb = orc.f32_to_bf16((g / (1 + np.exp(-g)) * u).astype(np.float32)).reshape(1, I)
    return orc.qmv_f64(*d3, I, dbits, 64, hb)[0]


def test_experts_against_float64_closed_form(orc):
    E, I, H, top_k, rows = 8, 64, 256, 3, 2
    (gc, gs_, gb), gate = _bank(orc, E, I, H, 4, 64, 11)
    (uc, us, ub), up = _bank(orc, E, I, H, 4, 64, 12)
    (dc, ds, db), down = _bank(orc, E, H, I, 5, 64, 13)
    sg3, sgate = _qw(orc, I, H, 4, 64, 14)
    su3, sup = _qw(orc, I, H, 4, 64, 15)
    sd3, sdown = _qw(orc, H, I, 5, 64, 16)
    x = orc.fill_bf16(rows * H, 17, 1, 1.0, 0.0).reshape(rows, H)
    ids = np.array([[1, 5, 7], [5, 0, 2]], np.uint32)
    scores = to_bf(orc, [[0.2, 0.3, 0.5], [0.6, 0.1, 0.3]])
    p = orc.moe_experts(x, ids, scores, top_k, gate, up, down, sgate, sup, sdown, H)
    for r in range(rows):
        for j in range(top_k + 1):
            if j < top_k:
                e = int(ids[r, j])
                ri, rh = slice(e * I, (e + 1) * I), slice(e * H, (e + 1) * H)
                want = _mlp64(orc, (gc[ri], gs_[ri], gb[ri]), (uc[ri], us[ri], ub[ri]),
                              (dc[rh], ds[rh], db[rh]), x[r:r + 1], H, I, 4, 5)
                want = want * bf(scores[r, j])
            else:
                want = _mlp64(orc, sg3, su3, sd3, x[r:r + 1], H, I, 4, 5)
            got = bf(p[r, j]).astype(np.float64)
            # bf16 roundings of g, u, silu, h, down and the product: a few ulps
            assert np.abs(got - want).max() <= 0.03 * np.abs(want).max(), (r, j)
    # a planted mistake (gate and up swapped) leaves the bound
    bad = orc.moe_experts(x, ids, scores, top_k, up, gate, down, sup, sgate, sdown, H)
    assert np.abs(bf(bad) - bf(p)).max() > 0.03 * np.abs(bf(p)).max()


def _reduce_reference_control_flow(prod):
    """kernels/moe_down_tail.metal:83-99 restated literally for TOP_K = 10:
    SLOT_ORDER {0,8,1,9,2,3,4,5,6,7}, pending/routed bf16 registers."""
    order = [0, 8, 1, 9, 2, 3, 4, 5, 6, 7]
    pending = routed = None
    for oi, slot in enumerate(order):
        product = prod[slot]
        if oi in (0, 2):
            pending = product
        elif oi == 1:
            routed = _rb(pending + product)
        elif oi == 3:
            second = _rb(pending + product)
            routed = _rb(second + routed)
        else:
            routed = _rb(product + routed)
    return routed


def _rb(v):
    v = np.float32(v)
    u = np.array([v], np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) << 16
    return r.view(np.float32)[0]


def test_reduce_matches_reference_slot_order(orc):
    rng = np.random.default_rng(3)
    rows, H, k = 3, 96, 10
    p = to_bf(orc, rng.standard_normal((rows, k + 1, H)).astype(np.float32) * 10 ** rng.uniform(-2, 2, (rows, k + 1, H)))
    got = bf(orc.moe_reduce(p, k))
    pf = bf(p)
    for r in range(rows):
        for c in range(H):
            want = _reduce_reference_control_flow(pf[r, :, c])
            assert got[r, c] == want, (r, c)
    # the order matters: a naive ascending sum differs somewhere
    naive = np.zeros((rows, H), np.float32)
    for r in range(rows):
        for c in range(H):
            acc = np.float32(0)
            for s in range(k):
                acc = _rb(acc + pf[r, s, c])
            naive[r, c] = acc
    assert (naive != got).any()


def test_hc_epilogue_four_rounding_points(orc):
    rng = np.random.default_rng(5)
    rows, H, hc = 2, 64, 4
    routed, shared = (to_bf(orc, rng.standard_normal((rows, H)).astype(np.float32)) for _ in range(2))
    factor = to_bf(orc, rng.uniform(0, 1, rows).astype(np.float32))
    residual = to_bf(orc, rng.standard_normal((rows, hc * H)).astype(np.float32) * 4)
    gate = to_bf(orc, rng.uniform(0, 2, (rows, hc)).astype(np.float32))
    got = orc.moe_hc_epilogue(routed, shared, factor, residual, gate, hc)
    for r in range(rows):
        for s in range(hc):
            for c in range(H):
                w = _rb(bf(shared[r, c]) * bf(factor[r]))
                cmb = _rb(bf(routed[r, c]) + w)
                inj = _rb(cmb * bf(gate[r, s]))
                want = _rb(bf(residual[r, s * H + c]) + inj)
                assert bf(got[r, s * H + c]) == want


# ---------------------------------------------------------------------- GDN --
def _silu64(v):
    return v / (1 + np.exp(-v))


def test_conv_window_and_state_update(orc):
    rng = np.random.default_rng(7)
    C_, K, groups, t = 40, 4, 2, 3
    qkv = to_bf(orc, rng.standard_normal((groups * t, C_)).astype(np.float32))
    state = to_bf(orc, rng.standard_normal((3, K - 1, C_)).astype(np.float32))
    w = rng.standard_normal((K, C_)).astype(np.float32) * 0.5
    slots = np.array([2, 0], np.int32)
    out, st2, hist = orc.gdn_conv(qkv, groups, t, slots, state, w, window_history=True)
    for g in range(groups):
        win = np.concatenate([bf(state[slots[g]]), bf(qkv[g * t:(g + 1) * t])], axis=0)
        assert (to_bf(orc, win) == hist[g]).all()
        for i in range(t):
            acc = (win[i:i + K].astype(np.float64) * w).sum(axis=0)
            got = bf(out[g * t + i]).astype(np.float64)
            assert np.allclose(got, _silu64(acc), rtol=2 ** -6, atol=2 ** -8)
        assert (st2[slots[g]] == to_bf(orc, win[-(K - 1):])).all()
    assert (st2[1] == state[1]).all()  # untouched slot
    # w = e_{K-1}: the output is silu of the new token alone
    w1 = np.zeros((K, C_), np.float32)
    w1[K - 1] = 1
    out1, _, _ = orc.gdn_conv(qkv, groups, t, slots, state, w1)
    # four bf16 roundings inside the bf16 sigmoid plus the product: <= 2^-6 relative
    assert np.allclose(bf(out1), _silu64(bf(qkv).astype(np.float64)), rtol=2 ** -6, atol=1e-6)


def _gdn_reference64(q, k, v, g, beta, state):
    """gdn_reference (src/hybrid.rs:457-498) in float64; state [Hv, Dv, Dk]."""
    hv, hk = v.shape[0], q.shape[0]
    s = state.astype(np.float64).copy()
    y = np.zeros((hv, 128))
    for h in range(hv):
        kk = k[h // (hv // hk)].astype(np.float64)
        qq = q[h // (hv // hk)].astype(np.float64)
        s[h] *= g[h]
        mem = s[h] @ kk
        delta = (v[h] - mem) * beta[h]
        s[h] += np.outer(delta, kk)
        y[h] = s[h] @ qq
    return y, s


def test_scan_matches_reference_fixture(orc):
    f = np.load(os.path.join(GOLDEN, "gdn_native_kernels_subset.npz"))
    hk, hv = 2, 6
    init = f["initial"][0]                            # [Hv, Dv, Dk]
    ours = np.ascontiguousarray(init.transpose(0, 2, 1))[None]  # [1, Hv, Dk, Dv]
    y, st, hist = orc.gdn_scan(f["q"].reshape(1, hk, 128), f["k"].reshape(1, hk, 128),
                               f["v"].reshape(1, hv, 128), f["g"].reshape(1, hv),
                               f["beta"].reshape(1, hv), hk, hv, 1, 1, np.zeros(1, np.int32),
                               ours, history=True)
    want_state = f["state"][0].transpose(0, 2, 1)
    scale = np.abs(want_state).max()
    assert np.abs(st[0] - want_state).max() <= 1e-4 * scale
    yw = bf(f["y"].reshape(hv, 128)).astype(np.float64)
    yg = bf(y.reshape(hv, 128)).astype(np.float64)
    assert np.all(np.abs(yg - yw) <= 1e-2 + 2e-2 * np.abs(yw))
    assert (hist[0] == st[0]).all()
    # and the float64 restatement of gdn_reference agrees with both
    y64, s64 = _gdn_reference64(bf(f["q"].reshape(hk, 128)), bf(f["k"].reshape(hk, 128)),
                                bf(f["v"].reshape(hv, 128)), f["g"].reshape(hv),
                                bf(f["beta"].reshape(hv)), init)
    assert np.abs(s64.transpose(0, 2, 1) - st[0]).max() <= 1e-5 * scale
    assert np.all(np.abs(y64 - yg) <= 1e-2 + 2e-2 * np.abs(y64))


def test_scan_identity_when_decay_one_and_beta_zero(orc):
    rng = np.random.default_rng(9)
    hk, hv = 1, 2
    state = rng.standard_normal((1, hv, 128, 128)).astype(np.float32)
    q, k = (to_bf(orc, rng.standard_normal((1, hk, 128)).astype(np.float32)) for _ in range(2))
    v = to_bf(orc, rng.standard_normal((1, hv, 128)).astype(np.float32))
    _, st, _ = orc.gdn_scan(q, k, v, np.ones((1, hv), np.float32), np.zeros((1, hv), np.uint16),
                            hk, hv, 1, 1, np.zeros(1, np.int32), state)
    assert (st == state).all()


def _fused64(orc, conv, z, a, b, a_log, dt, norm_w, eps, hk, hv, state):
    """Gdn::forward_reference (src/hybrid.rs:401-453) in float64 for one row."""
    kd = hk * 128
    q = conv[:kd].reshape(hk, 128).astype(np.float64)
    k = conv[kd:2 * kd].reshape(hk, 128).astype(np.float64)
    v = conv[2 * kd:].reshape(hv, 128).astype(np.float64)
    q = q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6) * 128 ** -0.5
    k = k / np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
    beta = 1 / (1 + np.exp(-b.astype(np.float64)))
    sp = np.logaddexp(a.astype(np.float64) + dt, 0)
    g = np.exp(-np.exp(a_log.astype(np.float64)) * sp)
    y, s = _gdn_reference64(q, k, v, g, beta, state)
    inv = 1 / np.sqrt((y * y).mean(-1, keepdims=True) + eps)
    y = y * inv * norm_w * (1 / (1 + np.exp(-z.reshape(hv, 128).astype(np.float64))))
    return y.reshape(-1), s


def test_fused_recurrence_against_float64(orc):
    rng = np.random.default_rng(11)
    hk, hv, groups, t = 2, 4, 2, 2
    rows = groups * t
    conv = to_bf(orc, rng.standard_normal((rows, 2 * hk * 128 + hv * 128)).astype(np.float32))
    z = to_bf(orc, rng.standard_normal((rows, hv * 128)).astype(np.float32))
    a = to_bf(orc, rng.standard_normal((rows, hv)).astype(np.float32))
    b = to_bf(orc, rng.standard_normal((rows, hv)).astype(np.float32))
    a_log = np.log(rng.uniform(0.5, 16, hv)).astype(np.float32)
    dt = to_bf(orc, rng.uniform(-1, 1, hv).astype(np.float32))
    norm_w = to_bf(orc, rng.uniform(0.5, 1.5, 128).astype(np.float32))
    eps = 1e-6
    state = (rng.standard_normal((3, hv, 128, 128)) * 0.1).astype(np.float32)
    slots = np.array([2, 0], np.int32)
    y, st, hist = orc.gdn_recurrence(conv, z, a, b, a_log, dt, norm_w, eps, hk, hv, groups, t,
                                     slots, state, history=True)
    for g in range(groups):
        s64 = state[slots[g]].transpose(0, 2, 1).astype(np.float64)  # -> [Hv, Dv, Dk]
        for i in range(t):
            r = g * t + i
            y64, s64 = _fused64(orc, bf(conv[r]), bf(z[r]), bf(a[r]), bf(b[r]), a_log,
                                bf(dt).astype(np.float64), bf(norm_w).astype(np.float64), eps,
                                hk, hv, s64)
            assert np.all(np.abs(bf(y[r]) - y64) <= 1e-2 + 2e-2 * np.abs(y64)), (g, i)
            sc = np.abs(s64).max()
            # bf16 q/k normalisation (vs exact f64) moves the state by ~2^-8 relative
            assert np.abs(hist[r].transpose(0, 2, 1) - s64).max() <= 2e-2 * sc
        assert (st[slots[g]] == hist[g * t + t - 1]).all()
    assert (st[1] == state[1]).all()


# --------------------------------------------------------------------- head --
def test_argmax_extremes_match_reference_convention(orc):
    """The cases of the reference's reduction test (tests/greedy_head.rs:109-147)."""
    n = 31040
    rows = np.zeros((4, n), np.float32)
    rows[0] = -np.inf
    rows[1] = np.nan
    rows[1, 777] = 2.0
    rows[2] = 0.0
    rows[2, 50] = np.inf
    rows[2, 1000] = np.inf
    rows[3] = -0.0
    got = orc.argmax_bf16(to_bf(orc, rows))
    assert list(got) == [0, 777, 50, 0]
    nan_only = to_bf(orc, np.full((1, 100), np.nan, np.float32))
    assert orc.argmax_bf16(nan_only)[0] == 0


def test_head_argmax_is_argmax_of_bf16_logits(orc):
    n, k = 3000, 512
    c, s, b = orc.random_qweight(n, k, 8, 64, 21)
    w = orc.qw(c, s, b, n, k, 8, 64)
    x = orc.fill_bf16(3 * k, 22, 1, 1.0, 0.0).reshape(3, k)
    logits = orc.qmv(c, s, b, k, 8, 64, x)
    got = orc.head_argmax(w, x)
    lf = bf(logits)
    for m in range(3):
        best = lf[m].max()
        assert got[m] == np.flatnonzero(lf[m] == best)[0]
    # ties in bf16 are common at vocabulary scale: lowest id wins
    assert (got == orc.argmax_bf16(logits)).all()
