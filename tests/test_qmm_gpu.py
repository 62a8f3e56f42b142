"""Matrix-core (MFMA) projections: within the north star's tolerance of the
float64 closed form and of the exact fixed-order kernels, for every code
width, depth and row count the engine uses (including partial 16-row tiles
and matrices split along k across workgroups)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def bf(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("bits", [4, 5, 6, 8])
@pytest.mark.parametrize("k,n", [(256, 72), (512, 2048), (2048, 1000), (4096, 264), (8192, 260)])
def test_qmm_against_closed_form_and_exact(mx, orc, bits, k, n):
    gs = 64
    seed = 7000 + bits * 100 + k // 64
    w = mx.QWeight.random(n, k, bits, gs, seed)
    codes, s, b = orc.random_qweight(n, k, bits, gs, seed)
    for m in (1, 3, 8, 16, 40, 200):  # beyond 16: the staged prefill GEMM
        x = orc.fill_bf16(m * k, seed + m, 1, 1.0, 0.0).reshape(m, k)
        dx = mx.DeviceArray.from_numpy(x)
        dy = mx.DeviceArray((m, n), np.uint16)
        qc = w.c()
        mx.check(mx.lib.mx_qmm(C.byref(qc), dx.ptr, m, dy.ptr, None))
        got = bf(dy.numpy()).astype(np.float64)
        y64 = orc.qmv_f64(codes, s, b, k, bits, gs, x)
        mag = np.abs(bf(x)).astype(np.float64).sum(axis=1, keepdims=True) * 0.05
        assert np.all(np.abs(got - y64) <= 2.0 ** -8 * np.abs(y64) + 2.0 ** -16 * mag + 1e-6), (m,)
        if m <= 8:
            ex = mx.DeviceArray((m, n), np.uint16)
            mx.qmv(w, dx, m, ex)
            e = bf(ex.numpy()).astype(np.float64)
            # fp32 summation order only: at most a bf16 ulp or two apart
            assert np.all(np.abs(got - e) <= 2.0 ** -7 * np.abs(e) + 2.0 ** -16 * mag + 1e-6)


def test_moe_experts_mfma_within_tolerance(mx, orc):
    from test_layers_gpu import Moe, dev

    E, I, H, top_k, rows = 64, 512, 2048, 10, 8
    m = Moe(mx, orc, E, I, H, seed=800)
    rng = np.random.default_rng(8)
    ids = np.stack([rng.choice(12, top_k, replace=False) for _ in range(rows)]).astype(np.uint32)
    scores = orc.f32_to_bf16(rng.uniform(0.02, 0.3, (rows, top_k)).astype(np.float32))
    x = orc.fill_bf16(rows * H, 801, 1, 1.0, 0.0).reshape(rows, H)
    want = bf(m.oracle(orc, x, ids, scores, top_k)).astype(np.float64)
    p = mx.DeviceArray((rows, top_k + 1, H), np.uint16)
    qb = [b.c() for b in (m.gate, m.up, m.down)]
    qs = [w.c() for w in (m.sg, m.su, m.sd)]
    dx, di, ds = dev(mx, x), dev(mx, ids), dev(mx, scores)
    mx.check(mx.lib.mx_moe_experts_mfma(dx.ptr, di.ptr, ds.ptr, rows, top_k, C.byref(qb[0]),
                                        C.byref(qb[1]), C.byref(qb[2]), C.byref(qs[0]),
                                        C.byref(qs[1]), C.byref(qs[2]), m.ws.ptr, p.ptr, None))
    got = bf(p.numpy()).astype(np.float64)
    scale = np.abs(want).max(axis=2, keepdims=True)
    assert np.all(np.abs(got - want) <= 2e-2 * np.abs(want) + 1e-2 * scale)
    assert np.mean(got == want) > 0.5  # mostly identical after bf16 rounding


def _experts_mfma(mx, m, x, ids, scores, top_k):
    from test_layers_gpu import dev

    rows = x.shape[0]
    p = mx.DeviceArray((rows, top_k + 1, m.H), np.uint16)
    qb = [b.c() for b in (m.gate, m.up, m.down)]
    qs = [w.c() for w in (m.sg, m.su, m.sd)]
    dx, di, ds = dev(mx, x), dev(mx, ids), dev(mx, scores)
    mx.check(mx.lib.mx_moe_experts_mfma(dx.ptr, di.ptr, ds.ptr, rows, top_k, C.byref(qb[0]),
                                        C.byref(qb[1]), C.byref(qb[2]), C.byref(qs[0]),
                                        C.byref(qs[1]), C.byref(qs[2]), m.ws.ptr, p.ptr, None))
    return p.numpy()


@pytest.mark.parametrize("bits", [4, 5, 6, 8])
def test_moe_experts_mfma_every_width(mx, orc, bits):
    """Hidden 2048 takes the persistent gate/up kernel (three items in flight
    per wave at <= 5-bit codes, two above) and 512-deep experts the
    fixed-depth down kernel."""
    from test_layers_gpu import Moe

    E, I, H, top_k, rows = 40, 512, 2048, 8, 8
    m = Moe(mx, orc, E, I, H, seed=700 + bits, gbits=bits, dbits=bits)
    rng = np.random.default_rng(bits)
    ids = np.stack([rng.choice(E, top_k, replace=False) for _ in range(rows)]).astype(np.uint32)
    scores = orc.f32_to_bf16(rng.uniform(0.05, 0.5, (rows, top_k)).astype(np.float32))
    x = orc.fill_bf16(rows * H, 710 + bits, 1, 1.0, 0.0).reshape(rows, H)
    want = bf(m.run(mx, x, ids, scores, top_k)).astype(np.float64)
    got = bf(_experts_mfma(mx, m, x, ids, scores, top_k)).astype(np.float64)
    scale = np.abs(want).max(axis=2, keepdims=True)
    assert np.all(np.abs(got - want) <= 2e-2 * np.abs(want) + 1e-2 * scale)
    assert np.mean(got == want) > 0.5


@pytest.mark.parametrize("rows,E,top_k,H", [(40, 64, 10, 2048), (128, 64, 10, 2048),
                                            (128, 512, 10, 2048), (17, 32, 6, 512)])
def test_moe_experts_mfma_prefill_chunk_rows(mx, orc, rows, E, top_k, H):
    """Beyond eight rows (a prefill chunk): routes grouped by expert into
    16-route tiles.  At 128 rows over 64 experts most experts take more than
    16 routes (several tiles each); against the exact kernels run eight rows
    at a time, within the north star's tolerance."""
    from test_layers_gpu import Moe

    I = 512
    m = Moe(mx, orc, E, I, H, seed=650 + rows + E)
    m.ws = mx.DeviceArray((mx.lib.mx_moe_workspace_bytes(rows, top_k, I),), np.uint8)
    rng = np.random.default_rng(rows + E)
    ids = np.stack([rng.choice(E, top_k, replace=False) for _ in range(rows)]).astype(np.uint32)
    scores = orc.f32_to_bf16(rng.uniform(0.05, 0.5, (rows, top_k)).astype(np.float32))
    x = orc.fill_bf16(rows * H, 660 + rows, 1, 1.0, 0.0).reshape(rows, H)
    got = bf(_experts_mfma(mx, m, x, ids, scores, top_k)).astype(np.float64)
    ws = m.ws
    m.ws = mx.DeviceArray((mx.lib.mx_moe_workspace_bytes(8, top_k, I),), np.uint8)
    want = np.concatenate([m.run(mx, x[r:r + 8], ids[r:r + 8], scores[r:r + 8], top_k)
                           for r in range(0, rows, 8)])
    m.ws = ws
    want = bf(want).astype(np.float64)
    scale = np.abs(want).max(axis=2, keepdims=True)
    assert np.all(np.abs(got - want) <= 2e-2 * np.abs(want) + 1e-2 * scale)
    assert np.mean(got == want) > 0.5


@pytest.mark.parametrize("gbits,dbits,H,I", [(5, 6, 512, 512), (6, 8, 1024, 256),
                                              (8, 4, 512, 768), (4, 5, 256, 1280)])
def test_moe_experts_mfma_prefill_chunk_widths(mx, orc, gbits, dbits, H, I):
    """The prefill chunk's expert kernels for every code width (4/8-bit: the
    32-row tile forms, each lane reading a group's 32 codes of its half with
    16-byte loads; 5/6-bit: the 16-row forms), at depths of 4..20 groups,
    against the exact kernels eight rows at a time within the north star's
    tolerance."""
    from test_layers_gpu import Moe

    E, top_k, rows = 32, 6, 40
    m = Moe(mx, orc, E, I, H, seed=700 + gbits * 10 + dbits, gbits=gbits, dbits=dbits)
    m.ws = mx.DeviceArray((mx.lib.mx_moe_workspace_bytes(rows, top_k, I),), np.uint8)
    rng = np.random.default_rng(gbits * 10 + dbits)
    ids = np.stack([rng.choice(E, top_k, replace=False) for _ in range(rows)]).astype(np.uint32)
    scores = orc.f32_to_bf16(rng.uniform(0.05, 0.5, (rows, top_k)).astype(np.float32))
    x = orc.fill_bf16(rows * H, 710 + gbits, 1, 1.0, 0.0).reshape(rows, H)
    got = bf(_experts_mfma(mx, m, x, ids, scores, top_k)).astype(np.float64)
    ws = m.ws
    m.ws = mx.DeviceArray((mx.lib.mx_moe_workspace_bytes(8, top_k, I),), np.uint8)
    want = np.concatenate([m.run(mx, x[r:r + 8], ids[r:r + 8], scores[r:r + 8], top_k)
                           for r in range(0, rows, 8)])
    m.ws = ws
    want = bf(want).astype(np.float64)
    scale = np.abs(want).max(axis=2, keepdims=True)
    assert np.all(np.abs(got - want) <= 2e-2 * np.abs(want) + 1e-2 * scale)
    assert np.mean(got == want) > 0.5


@pytest.mark.parametrize("I,sI", [(1024, 512), (256, 768), (512, 512)])
def test_moe_experts_mfma_mixed_depths(mx, orc, I, sI):
    """Routed and shared experts of different 256-multiple depths (the down
    kernel's general form, depth read per expert) and of equal 512 depth (its
    fixed-depth form), at hidden 512 (the per-route gate/up kernel)."""
    from test_layers_gpu import Moe

    E, H, top_k, rows = 32, 512, 6, 8
    m = Moe(mx, orc, E, I, H, seed=600 + I, sI=sI)
    rng = np.random.default_rng(I + sI)
    ids = np.stack([rng.choice(E, top_k, replace=False) for _ in range(rows)]).astype(np.uint32)
    scores = orc.f32_to_bf16(rng.uniform(0.05, 0.5, (rows, top_k)).astype(np.float32))
    x = orc.fill_bf16(rows * H, 610, 1, 1.0, 0.0).reshape(rows, H)
    want = bf(m.run(mx, x, ids, scores, top_k)).astype(np.float64)
    got = bf(_experts_mfma(mx, m, x, ids, scores, top_k)).astype(np.float64)
    scale = np.abs(want).max(axis=2, keepdims=True)
    assert np.all(np.abs(got - want) <= 2e-2 * np.abs(want) + 1e-2 * scale)
    assert np.mean(got == want) > 0.5


@pytest.mark.parametrize("n,k", [(260, 8192), (2048, 4096), (513, 2048), (12352, 2048)])
def test_qmm_k_split_shapes_deterministic(mx, orc, n, k):
    """Shapes whose k is split among a workgroup's waves (the engine's HC,
    output and router projections): repeated calls give identical bits, and
    the result is within tolerance of the float64 closed form."""
    bits, gs, m = 4, 64, 8
    w = mx.QWeight.random(n, k, bits, gs, 9100 + n)
    x = orc.fill_bf16(m * k, 9102, 1, 1.0, 0.0).reshape(m, k)
    dx = mx.DeviceArray.from_numpy(x)
    outs = []
    for _ in range(3):
        dy = mx.DeviceArray((m, n), np.uint16)
        qc = w.c()
        mx.check(mx.lib.mx_qmm(C.byref(qc), dx.ptr, m, dy.ptr, None))
        outs.append(dy.numpy())
    assert (outs[0] == outs[1]).all() and (outs[1] == outs[2]).all()
    codes, s, b = orc.random_qweight(n, k, bits, gs, 9100 + n)
    y64 = orc.qmv_f64(codes, s, b, k, bits, gs, x)
    got = bf(outs[0]).astype(np.float64)
    mag = np.abs(bf(x)).astype(np.float64).sum(axis=1, keepdims=True) * 0.05
    assert np.all(np.abs(got - y64) <= 2.0 ** -8 * np.abs(y64) + 2.0 ** -16 * mag + 1e-6)


@pytest.mark.parametrize("m", [1, 5, 8])
def test_head_argmax_mfma_matches_exact_head(mx, orc, m):
    """The matrix-core head picks the exact head's token unless the two best
    bf16 logits of a row are within the summation-order tolerance."""
    n, k, bits, gs = 151936, 2048, 8, 64
    w = mx.QWeight.random(n, k, bits, gs, 9200)
    x = orc.fill_bf16(m * k, 9201 + m, 1, 1.0, 0.0).reshape(m, k)
    dx = mx.DeviceArray.from_numpy(x)
    wsb = mx.lib.mx_head_workspace_bytes(n, k, m)
    ws = mx.DeviceArray((wsb,), np.uint8)
    got = mx.DeviceArray((m,), np.uint32)
    exact = mx.DeviceArray((m,), np.uint32)
    qc = w.c()
    mx.check(mx.lib.mx_head_argmax_mfma(C.byref(qc), dx.ptr, m, got.ptr, ws.ptr, None))
    mx.check(mx.lib.mx_head_argmax(C.byref(qc), dx.ptr, m, exact.ptr, ws.ptr, None))
    logits = mx.DeviceArray((m, n), np.uint16)
    mx.qmv(w, dx, m, logits)
    lg = bf(logits.numpy()).astype(np.float64)
    g, e = got.numpy(), exact.numpy()
    for r in range(m):
        if g[r] != e[r]:
            assert abs(lg[r, g[r]] - lg[r, e[r]]) <= 2.0 ** -7 * abs(lg[r, e[r]]) + 1e-3, r
    assert np.mean(g == e) >= 0.5


@pytest.mark.parametrize("E,rows", [(512, 8), (512, 1), (512, 5), (256, 8)])
def test_moe_routed_experts_mfma_matches_route_then_experts(mx, orc, E, rows):
    """The fused routing + matrix-core experts call gives the bits of
    mx_moe_route (bit-exact with the oracle) followed by mx_moe_experts_mfma:
    with 512 routed experts the persistent gate/up kernel routes its rows
    itself, with 256 the call routes first."""
    from test_layers_gpu import dev

    I, H, top_k = 256, 2048, 10
    gate = mx.QBank.random(E, I, H, 4, 64, 900)
    up = mx.QBank.random(E, I, H, 4, 64, 910)
    down = mx.QBank.random(E, H, I, 5, 64, 920)
    sg = mx.QWeight.random(I, H, 4, 64, 930)
    su = mx.QWeight.random(I, H, 4, 64, 940)
    sd = mx.QWeight.random(H, I, 5, 64, 950)
    stride = E + 1
    lg = orc.fill_bf16(rows * stride, 960 + rows, 1, 2.0, 0.0).reshape(rows, stride)
    lg[0, :E] = 0  # an all-tied row
    x = orc.fill_bf16(rows * H, 970 + rows, 1, 1.0, 0.0).reshape(rows, H)
    d_lg, dx = dev(mx, lg), dev(mx, x)
    ws = mx.DeviceArray((mx.lib.mx_moe_workspace_bytes(8, 16, I),), np.uint8)
    qb = [b.c() for b in (gate, up, down)]
    qs = [w.c() for w in (sg, su, sd)]
    lg_ptr, sh_ptr = d_lg.ptr, d_lg.ptr + 2 * E

    ids_w = mx.DeviceArray((rows, top_k), np.uint32)
    sc_w = mx.DeviceArray((rows, top_k), np.uint16)
    fa_w = mx.DeviceArray((rows,), np.uint16)
    mx.check(mx.lib.mx_moe_route(lg_ptr, stride, sh_ptr, stride, rows, E, top_k, ids_w.ptr,
                                 sc_w.ptr, fa_w.ptr, None))
    p_w = mx.DeviceArray((rows, top_k + 1, H), np.uint16)
    mx.check(mx.lib.mx_moe_experts_mfma(dx.ptr, ids_w.ptr, sc_w.ptr, rows, top_k,
                                        C.byref(qb[0]), C.byref(qb[1]), C.byref(qb[2]),
                                        C.byref(qs[0]), C.byref(qs[1]), C.byref(qs[2]), ws.ptr,
                                        p_w.ptr, None))

    ids = mx.DeviceArray((rows, top_k), np.uint32)
    sc = mx.DeviceArray((rows, top_k), np.uint16)
    fa = mx.DeviceArray((rows,), np.uint16)
    p = mx.DeviceArray((rows, top_k + 1, H), np.uint16)
    mx.check(mx.lib.mx_moe_routed_experts_mfma(lg_ptr, stride, sh_ptr, stride, E, dx.ptr, rows,
                                               top_k, C.byref(qb[0]), C.byref(qb[1]),
                                               C.byref(qb[2]), C.byref(qs[0]), C.byref(qs[1]),
                                               C.byref(qs[2]), ws.ptr, ids.ptr, sc.ptr, fa.ptr,
                                               p.ptr, None))
    assert (ids.numpy() == ids_w.numpy()).all()
    assert (sc.numpy() == sc_w.numpy()).all()
    assert (fa.numpy() == fa_w.numpy()).all()
    assert (p.numpy() == p_w.numpy()).all()
    # and the routes themselves are the oracle's
    want_ids, want_sc, want_fa = orc.moe_route(np.ascontiguousarray(lg[:, :E]), lg[:, E], top_k)
    assert (ids.numpy() == want_ids).all() and (sc.numpy() == want_sc).all()
    assert (fa.numpy() == want_fa).all()


@pytest.mark.parametrize("E,rows,top_k,dbits", [(512, 8, 10, 5), (512, 1, 10, 5), (512, 5, 10, 4),
                                                (256, 8, 8, 6), (256, 3, 15, 8), (128, 8, 3, 4),
                                                (64, 2, 4, 5)])
def test_moe_routed_experts_hc_mfma_matches_experts_then_epilogue(mx, orc, E, rows, top_k, dbits):
    """The MoE sublayer call (down projection, slot sum and stream write in
    one kernel) gives the bits of mx_moe_routed_experts_mfma followed by
    mx_moe_reduce_hc_epilogue: ids, scores, factor and the updated streams.
    top_k 3 .. 15 covers one to four slots per wave."""
    from test_layers_gpu import dev

    I, H = 512, 2048
    sd0 = 1000 * top_k + E
    gate = mx.QBank.random(E, I, H, 4, 64, sd0)
    up = mx.QBank.random(E, I, H, 4, 64, sd0 + 1)
    down = mx.QBank.random(E, H, I, dbits, 64, sd0 + 2)
    sg = mx.QWeight.random(I, H, 4, 64, sd0 + 3)
    su = mx.QWeight.random(I, H, 4, 64, sd0 + 4)
    sd = mx.QWeight.random(H, I, dbits, 64, sd0 + 5)
    stride = E + 1
    lg = orc.fill_bf16(rows * stride, sd0 + 6, 1, 2.0, 0.0).reshape(rows, stride)
    x = orc.fill_bf16(rows * H, sd0 + 7, 1, 1.0, 0.0).reshape(rows, H)
    res = orc.fill_bf16(rows * 4 * H, sd0 + 8, 1, 1.0, 0.0).reshape(rows, 4, H)
    hg = orc.fill_bf16(rows * 4, sd0 + 9, 1, 1.0, 1.0).reshape(rows, 4)
    d_lg, dx, dhg = dev(mx, lg), dev(mx, x), dev(mx, hg)
    ws = mx.DeviceArray((mx.lib.mx_moe_workspace_bytes(8, 16, I),), np.uint8)
    qb = [b.c() for b in (gate, up, down)]
    qs = [w.c() for w in (sg, su, sd)]
    lg_ptr, sh_ptr = d_lg.ptr, d_lg.ptr + 2 * E

    ids_w = mx.DeviceArray((rows, top_k), np.uint32)
    sc_w = mx.DeviceArray((rows, top_k), np.uint16)
    fa_w = mx.DeviceArray((rows,), np.uint16)
    p_w = mx.DeviceArray((rows, top_k + 1, H), np.uint16)
    mx.check(mx.lib.mx_moe_routed_experts_mfma(lg_ptr, stride, sh_ptr, stride, E, dx.ptr, rows,
                                               top_k, C.byref(qb[0]), C.byref(qb[1]),
                                               C.byref(qb[2]), C.byref(qs[0]), C.byref(qs[1]),
                                               C.byref(qs[2]), ws.ptr, ids_w.ptr, sc_w.ptr,
                                               fa_w.ptr, p_w.ptr, None))
    dres = dev(mx, res)
    out_w = mx.DeviceArray((rows, 4, H), np.uint16)
    mx.check(mx.lib.mx_moe_reduce_hc_epilogue(p_w.ptr, fa_w.ptr, dres.ptr, dhg.ptr, rows, top_k,
                                              4, H, out_w.ptr, None))

    ids = mx.DeviceArray((rows, top_k), np.uint32)
    sc = mx.DeviceArray((rows, top_k), np.uint16)
    fa = mx.DeviceArray((rows,), np.uint16)
    hcs = dev(mx, res)
    mx.check(mx.lib.mx_moe_routed_experts_hc_mfma(lg_ptr, stride, sh_ptr, stride, E, dx.ptr, rows,
                                                  top_k, 4, C.byref(qb[0]), C.byref(qb[1]),
                                                  C.byref(qb[2]), C.byref(qs[0]), C.byref(qs[1]),
                                                  C.byref(qs[2]), ws.ptr, ids.ptr, sc.ptr, fa.ptr,
                                                  dhg.ptr, hcs.ptr, None))
    assert (ids.numpy() == ids_w.numpy()).all()
    assert (sc.numpy() == sc_w.numpy()).all()
    assert (fa.numpy() == fa_w.numpy()).all()
    got, want = hcs.numpy(), out_w.numpy()
    assert (got == want).all(), np.argwhere(got != want)[:8]
    assert not (got == res).all()


@pytest.mark.parametrize("n,k,ch,taps,m", [(12352, 2048, 8192, 4, 8), (640, 512, 384, 3, 3),
                                           (300, 1024, 300, 2, 1), (49152, 512, 1000, 4, 2)])
def test_qmm_conv_matches_qmm_then_conv(mx, orc, n, k, ch, taps, m):
    """The projection with the GDN conv in its epilogue gives the bits of
    mx_qmm followed by mx_gdn_conv: conv outputs, the updated window (other
    slots untouched) and the plain columns.  The last shape has more outputs
    per workgroup than threads (conv operands fetched in the epilogue)."""
    from test_layers_gpu import dev

    w = mx.QWeight.random(n, k, 4, 64, 9300 + n)
    qc = w.c()
    x = orc.fill_bf16(m * k, 9301 + m, 1, 1.0, 0.0).reshape(m, k)
    S = 10
    rng = np.random.default_rng(n + taps)
    slots = rng.choice(S, m, replace=False).astype(np.int32)
    state = orc.f32_to_bf16(rng.standard_normal((S, taps - 1, ch)).astype(np.float32))
    cw = (rng.standard_normal((taps, ch)) * 0.4).astype(np.float32)
    dx, dsl, dcw = dev(mx, x), dev(mx, slots), dev(mx, cw)
    y_ref = mx.DeviceArray((m, n), np.uint16)
    mx.check(mx.lib.mx_qmm(C.byref(qc), dx.ptr, m, y_ref.ptr, None))
    st1 = dev(mx, state)
    conv_ref = mx.DeviceArray((m, ch), np.uint16)
    mx.check(mx.lib.mx_gdn_conv(y_ref.ptr, n, m, 1, dsl.ptr, st1.ptr, dcw.ptr, ch, taps,
                                conv_ref.ptr, ch, None, None))
    st2 = dev(mx, state)
    y2 = dev(mx, np.zeros((m, n), np.uint16))
    conv2 = mx.DeviceArray((m, ch), np.uint16)
    mx.check(mx.lib.mx_qmm_conv(C.byref(qc), dx.ptr, m, ch, taps, dsl.ptr, st2.ptr, dcw.ptr,
                                conv2.ptr, ch, y2.ptr, n, None))
    assert (conv2.numpy() == conv_ref.numpy()).all()
    assert (st2.numpy() == st1.numpy()).all()
    got = y2.numpy()
    assert (got[:, ch:] == y_ref.numpy()[:, ch:]).all()
    assert (got[:, :ch] == 0).all()  # conv channels are not written to y
    other = np.setdiff1d(np.arange(S), slots)
    assert (st2.numpy()[other] == state[other]).all()


@pytest.mark.parametrize("hidden,rank,inject,rows", [(2048, 256, True, 8), (2048, 256, False, 3),
                                                     (1024, 256, True, 5), (512, 256, True, 1),
                                                     (2048, 512, False, 2)])
def test_hc_forward_mfma_within_tolerance_of_oracle(mx, orc, hidden, rank, inject, rows):
    """The matrix-core hyper-connection projection (norm factored out of the
    down projection, hardware exp2 / rsqrt) against the oracle's fixed-order
    HC (norm, down + activation, up + mix): the north star's 2e-2 relative /
    1e-2 of the row's largest magnitude; repeated calls give the same bits."""
    from test_layers_gpu import dev

    hc = 4
    n_down = rank + (hc if inject else 0)
    down = mx.QWeight.random(n_down, hc * hidden, 4, 64, 9500 + hidden + rows)
    up = mx.QWeight.random(hc * hidden, rank, 4, 64, 9501 + hidden)
    rng = np.random.default_rng(hidden + rows)
    h = orc.f32_to_bf16(rng.standard_normal((rows, hc * hidden)).astype(np.float32))
    scale = orc.f32_to_bf16(rng.uniform(-0.5, 0.5, hc * hidden).astype(np.float32))
    eps = 1e-6
    dh, ds = dev(mx, h), dev(mx, scale)
    ws = mx.DeviceArray((mx.lib.mx_hc_workspace_bytes(n_down),), np.uint8)
    dc, uc = down.c(), up.c()
    outs = []
    for _ in range(2):
        mixed = mx.DeviceArray((rows, hidden), np.uint16)
        inj = mx.DeviceArray((rows, hc), np.uint16)
        mx.check(mx.lib.mx_hc_forward_mfma(C.byref(dc), C.byref(uc), dh.ptr, ds.ptr, rows, hc,
                                           hidden, rank, eps, ws.ptr, mixed.ptr, inj.ptr, None))
        outs.append((mixed.numpy(), inj.numpy()))
    assert (outs[0][0] == outs[1][0]).all()
    m1, i1 = outs[0]
    dcodes, dsc, dbi = down.host()
    ucodes, usc, ubi = up.host()
    dq = orc.qw(dcodes, dsc, dbi, n_down, hc * hidden, 4, 64)
    uq = orc.qw(ucodes, usc, ubi, hc * hidden, rank, 4, 64)
    xn = np.empty_like(h)
    orc.lib.mxo_hc_norm(orc._p(h), orc._p(scale), rows, hc, hidden, eps, orc._p(xn))
    lo = np.empty((rows, rank), np.uint16)
    inj_w = np.zeros((rows, hc), np.uint16)
    orc.lib.mxo_hc_down(C.byref(dq), orc._p(xn), rows, rank, hc, orc._p(lo), orc._p(inj_w))
    mixed_w = np.empty((rows, hidden), np.uint16)
    orc.lib.mxo_hc_up_mix(C.byref(uq), orc._p(lo), orc._p(xn), rows, hidden, orc._p(mixed_w))
    got, want = bf(m1).astype(np.float64), bf(mixed_w).astype(np.float64)
    scale_w = np.abs(want).max(axis=1, keepdims=True)
    assert np.all(np.abs(got - want) <= 2e-2 * np.abs(want) + 1e-2 * scale_w)
    if inject:
        gi, wi = bf(i1).astype(np.float64), bf(inj_w).astype(np.float64)
        assert np.all(np.abs(gi - wi) <= 2e-2 * np.abs(wi) + 1e-2)
