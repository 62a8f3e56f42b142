"""Pins the oracle's hyper-connection and attention restatements (CPU only)
against float64 forms of the reference's own formulas and against properties
the mathematics fixes (a one-position softmax returns v; rotate-half RoPE
preserves each pair's norm and leaves the dimensions past rotary_dim alone).
Each check is chosen so that a plausible slip (a dropped (1 + scale), a
missing 1 / hc, a wrong stream or head mapping, a rotation sign) fails it."""
import ctypes as C

import ctypes as C
import ctypes.util

import numpy as np

HC, EPS = 4, 1e-6


def bf(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def dense(orc, codes, scales, biases, k, bits, gs=64):
    """float64 W = s q + b of an MLX affine matrix (value c at bit c * bits)."""
    q = orc.unpack_codes(codes, k, bits).astype(np.float64)
    s = np.repeat(bf(scales), gs, axis=1)
    b = np.repeat(bf(biases), gs, axis=1)
    return s * q + b


def within(got, want, rel=2e-2, frac=1e-2):
    scale = np.abs(want).max()
    return np.all(np.abs(got - want) <= rel * np.abs(want) + frac * scale)


def test_hc_forward_against_float64_reference(orc):
    """HyperConnection::forward_reference (src/hybrid.rs:78-99): grouped norm
    x_s / sqrt(mean(x_s^2) + eps) * (1 + scale_s) (compiled::norm,
    src/compiled.rs:22-28), lo = silu(down(xn) / hc), p = up(lo), mixed =
    mean_s sigmoid(p_s) * xn_s, inject = 2 sigmoid(inject(xn) / hc)
    (compiled.rs:46-86), in float64 from the same bf16 inputs."""
    rows, hidden, rank = 3, 256, 64
    n_down = rank + HC
    rng = np.random.default_rng(31)
    x = orc.f32_to_bf16(rng.standard_normal((rows, HC * hidden)).astype(np.float32) *
                        np.array([0.5, 1.0, 2.0, 4.0], np.float32).repeat(hidden))
    scale = orc.f32_to_bf16(rng.uniform(-0.6, 0.6, HC * hidden).astype(np.float32))
    dc, dsc, dbi = orc.random_qweight(n_down, HC * hidden, 4, 64, seed=311, s_range=(0.02, 0.08),
                                      b_range=(-0.5, 0.0))
    uc, usc, ubi = orc.random_qweight(HC * hidden, rank, 4, 64, seed=312, s_range=(0.02, 0.08),
                                      b_range=(-0.5, 0.0))
    dq = orc.qw(dc, dsc, dbi, n_down, HC * hidden, 4, 64)
    uq = orc.qw(uc, usc, ubi, HC * hidden, rank, 4, 64)
    xn = np.empty_like(x)
    orc.lib.mxo_hc_norm(orc._p(x), orc._p(scale), rows, HC, hidden, EPS, orc._p(xn))
    lo = np.empty((rows, rank), np.uint16)
    inj = np.zeros((rows, HC), np.uint16)
    orc.lib.mxo_hc_down(C.byref(dq), orc._p(xn), rows, rank, HC, orc._p(lo), orc._p(inj))
    mixed = np.empty((rows, hidden), np.uint16)
    orc.lib.mxo_hc_up_mix(C.byref(uq), orc._p(lo), orc._p(xn), rows, hidden, orc._p(mixed))

    xf = bf(x).reshape(rows, HC, hidden)
    inv = 1.0 / np.sqrt((xf * xf).mean(axis=2, keepdims=True) + EPS)
    xn_w = (xf * inv * (1.0 + bf(scale).reshape(HC, hidden))).reshape(rows, HC * hidden)
    assert within(bf(xn), xn_w, rel=1e-2, frac=1e-3)
    wd = dense(orc, dc, dsc, dbi, HC * hidden, 4)
    v = xn_w @ wd.T
    lo_in = v[:, :rank] / HC
    lo_w = lo_in * sigmoid(lo_in)
    inj_w = 2.0 * sigmoid(v[:, rank:] / HC)
    assert within(bf(lo), lo_w)
    assert within(bf(inj), inj_w)
    p = lo_w @ dense(orc, uc, usc, ubi, rank, 4).T
    mixed_w = (sigmoid(p).reshape(rows, HC, hidden) * xn_w.reshape(rows, HC, hidden)).mean(axis=1)
    assert within(bf(mixed), mixed_w)
    # the streams enter with their own weights: a mix over the wrong stream fails
    swapped = (sigmoid(p).reshape(rows, HC, hidden)[:, ::-1] *
               xn_w.reshape(rows, HC, hidden)).mean(axis=1)
    assert not within(bf(mixed), swapped)


def test_hc_write_against_float64_reference(orc):
    """HyperConnection::write (src/hybrid.rs:100-105): residual stream s gains
    y * gate_s, with y the output projection of the layer."""
    rows, hidden, k = 2, 128, 192
    rng = np.random.default_rng(32)
    wc, ws, wb = orc.random_qweight(hidden, k, 4, 64, seed=321)
    w = orc.qw(wc, ws, wb, hidden, k, 4, 64)
    y = orc.f32_to_bf16(rng.standard_normal((rows, k)).astype(np.float32))
    gate = orc.f32_to_bf16(rng.uniform(0.0, 2.0, (rows, HC)).astype(np.float32))
    res0 = orc.f32_to_bf16(rng.standard_normal((rows, HC * hidden)).astype(np.float32))
    res = res0.copy()
    orc.lib.mxo_hc_write(C.byref(w), orc._p(y), rows, HC, orc._p(res), orc._p(gate))
    proj = bf(y) @ dense(orc, wc, ws, wb, k, 4).T
    want = bf(res0).reshape(rows, HC, hidden) + proj[:, None, :] * bf(gate)[:, :, None]
    assert within(bf(res).reshape(rows, HC, hidden), want)


# attention: 4 query heads over 2 KV heads (query head h reads KV head h // 2),
# head dim 256 with (q, gate) interleaved per head, partial RoPE on 64 dims
HEADS, KVH, HD, ROT, THETA, MAXC = 4, 2, 256, 64, 1e6, 640


def _prep(orc, rows, pos, seed):
    rng = np.random.default_rng(seed)
    width = HEADS * 2 * HD + 2 * KVH * HD
    qkv = orc.f32_to_bf16(rng.standard_normal((rows, width)).astype(np.float32))
    qn = orc.f32_to_bf16(rng.uniform(-0.5, 0.5, HD).astype(np.float32))
    kn = orc.f32_to_bf16(rng.uniform(-0.5, 0.5, HD).astype(np.float32))
    half = ROT // 2
    cos = np.empty((MAXC, half), np.float32)
    sin = np.empty((MAXC, half), np.float32)
    orc.lib.mxo_rope_table(MAXC, ROT, THETA, orc._p(cos), orc._p(sin))
    slot_stride = KVH * MAXC * HD
    # earlier positions of each row's slot hold random keys and values
    kc = orc.f32_to_bf16(rng.standard_normal((rows, KVH, MAXC, HD)).astype(np.float32))
    vc = orc.f32_to_bf16(rng.standard_normal((rows, KVH, MAXC, HD)).astype(np.float32))
    slots = np.arange(rows, dtype=np.int32)
    pos = np.asarray(pos, np.int32)
    q_out = np.empty((rows, HEADS, HD), np.uint16)
    orc.lib.mxo_attn_prep(orc._p(qkv), width, rows, orc._p(slots), orc._p(pos), orc._p(qn),
                          orc._p(kn), EPS, orc._p(cos), orc._p(sin), HEADS, KVH, HD, ROT, MAXC,
                          slot_stride, orc._p(q_out), orc._p(kc), orc._p(vc))
    return qkv, qn, kn, kc, vc, slots, pos, q_out, width, slot_stride


def _inv_freq32(theta, rot):
    """inv_freq[i] = 1 / powf(theta, 2i/rot) in fp32 (src/rope.rs:20-24), with
    the C library's powf."""
    libm = C.CDLL(ctypes.util.find_library("m"))
    libm.powf.restype = C.c_float
    libm.powf.argtypes = [C.c_float, C.c_float]
    half = rot // 2
    return np.array([np.float32(1.0) / np.float32(libm.powf(theta, np.float32(2 * i) / np.float32(rot)))
                     for i in range(half)], np.float32)


def _rope64(x, p):
    """Rotate-half RoPE on the first ROT dims (kernels/text_rope.metal): the
    angle is the fp32 product pos * inv_freq, the rotation in float64."""
    half = ROT // 2
    inv = _inv_freq32(THETA, ROT)
    a = (np.float32(p) * inv).astype(np.float64)
    c, s = np.cos(a), np.sin(a)
    out = x.copy()
    out[..., :half] = x[..., :half] * c - x[..., half:ROT] * s
    out[..., half:ROT] = x[..., half:ROT] * c + x[..., :half] * s
    return out


def test_attn_prep_against_float64_reference(orc):
    """Gated attention input (src/dense.rs:139-215): q and k pass compiled::norm
    with (1 + weight), then rotate-half RoPE over rotary_dim at the row's
    position; v is copied; k and v land in the slot's cache at that position."""
    pos = [0, 5, 517]
    qkv, qn, kn, kc, vc, slots, pos, q_out, width, _ = _prep(orc, 3, pos, 41)
    x = bf(qkv)

    def norm(v, w):
        return v / np.sqrt((v * v).mean(axis=-1, keepdims=True) + EPS) * (1.0 + bf(w))

    for r, p in enumerate(pos):
        q = x[r, :HEADS * 2 * HD].reshape(HEADS, 2, HD)[:, 0]
        k = x[r, HEADS * 2 * HD:HEADS * 2 * HD + KVH * HD].reshape(KVH, HD)
        v = x[r, HEADS * 2 * HD + KVH * HD:].reshape(KVH, HD)
        q_w, k_w = _rope64(norm(q, qn), p), _rope64(norm(k, kn), p)
        assert within(bf(q_out[r]), q_w, rel=1e-2, frac=1e-3)
        assert within(bf(kc[r, :, p]), k_w, rel=1e-2, frac=1e-3)
        assert (vc[r, :, p] == qkv[r, HEADS * 2 * HD + KVH * HD:].reshape(KVH, HD)).all()
        # RoPE preserves every rotated pair's norm and leaves dims >= ROT alone
        nq = norm(q, qn)
        half = ROT // 2
        pair = lambda t: t[..., :half] ** 2 + t[..., half:ROT] ** 2  # noqa: E731
        assert np.allclose(pair(q_w), pair(nq))
        assert within(bf(q_out[r, :, ROT:]), nq[:, ROT:], rel=1e-2, frac=1e-3)
        if p == 0:  # position 0: no rotation
            assert within(bf(q_out[r]), nq, rel=1e-2, frac=1e-3)


def test_attention_against_float64_softmax(orc):
    """Decode attention (src/dense.rs:216-270): softmax(q k^T / sqrt(hd)) v over
    positions 0..pos of the row's slot, query head h on KV head h // (heads /
    kv_heads), output times sigmoid(gate) of the head (the gated attention);
    517 positions cross the oracle's 256-position chunks."""
    qkv, qn, kn, kc, vc, slots, pos, q_out, width, slot_stride = _prep(orc, 3, [0, 5, 517], 42)
    out = np.empty((3, HEADS, HD), np.uint16)
    orc.lib.mxo_attention(orc._p(q_out), orc._p(qkv), width, 3, orc._p(slots), orc._p(pos),
                          orc._p(kc), orc._p(vc), HEADS, KVH, HD, MAXC, slot_stride, orc._p(out))
    x = bf(qkv)
    for r, p in enumerate(pos):
        gate = x[r, :HEADS * 2 * HD].reshape(HEADS, 2, HD)[:, 1]
        for h in range(HEADS):
            kvh = h // (HEADS // KVH)
            k = bf(kc[r, kvh, :p + 1])
            v = bf(vc[r, kvh, :p + 1])
            s = k @ bf(q_out[r, h]) / np.sqrt(HD)
            w = np.exp(s - s.max())
            o = (w / w.sum()) @ v
            want = o * sigmoid(gate[h])
            assert within(bf(out[r, h]), want), (r, h)
            if p == 0:  # one position: the softmax weight is 1, the output is v
                assert within(bf(out[r, h]), v[0] * sigmoid(gate[h]), rel=1e-2, frac=1e-3)
            # the other KV head gives another answer (the head mapping is pinned)
            other = bf(vc[r, 1 - kvh, :p + 1])
            ko = bf(kc[r, 1 - kvh, :p + 1])
            so = ko @ bf(q_out[r, h]) / np.sqrt(HD)
            wo = np.exp(so - so.max())
            assert not within(bf(out[r, h]), ((wo / wo.sum()) @ other) * sigmoid(gate[h]))


def test_rope_angle_is_the_fp32_product(orc):
    """kernels/text_rope.metal computes `float angle = pos*float(inv_freq)`:
    the angle is rounded to fp32 before cos/sin, an error that grows with the
    position (about 2.4e-4 rad at 4k, 1.6e-2 rad at 262k).  The oracle's table
    equals cos/sin of that fp32 angle at positions near 4000 and 200000, and
    differs there from the exact (float64) angle, so a table built from the
    float64 product fails this test."""
    rot, theta = 64, 1e7
    half = rot // 2
    maxc = 200_008
    cos = np.empty((maxc, half), np.float32)
    sin = np.empty((maxc, half), np.float32)
    orc.lib.mxo_rope_table(maxc, rot, theta, orc._p(cos), orc._p(sin))
    inv = _inv_freq32(theta, rot)
    pos = np.array([0, 1, 3999, 4000, 4097, 199_999, 200_003], np.int64)
    a32 = (pos.astype(np.float32)[:, None] * inv[None, :]).astype(np.float64)
    assert (cos[pos] == np.cos(a32).astype(np.float32)).all()
    assert (sin[pos] == np.sin(a32).astype(np.float32)).all()
    a64 = pos.astype(np.float64)[:, None] * inv.astype(np.float64)[None, :]
    far = pos >= 199_999
    assert (sin[pos[far]] != np.sin(a64[far]).astype(np.float32)).any()
    assert np.abs(a32[far] - a64[far]).max() > 1e-3
