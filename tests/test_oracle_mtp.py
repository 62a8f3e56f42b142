"""Pins of the oracle's MTP draft step (Model.mtp_step, the restatement of
Mtp::forward, reference src/mtp.rs:72-127), on the CPU, by what the
mathematics fixes.  The reference holds no MTP fixture, so:

  * closed form: the draft layer's input streams (src/mtp.rs:88-104) against
    a float64 evaluation from the dequantised weights -- e = fc_embedding(
    norm(embedding)) over H, ONE norm of the previous hidden streams over all
    hc*H values, fc_hidden applied to each stream, e added to every stream --
    within the bound of the oracle's bf16 rounding points.  Plausible
    mistakes (a per-stream norm, a dropped +1 of the norm scale, e added to
    one stream only, the two projections swapped, an unnormalised hidden
    input) each break the bound;
  * reduction: a draft layer holding a trunk attention layer's weights, an
    identity fc_embedding, a zero fc_hidden, a zero norm scale and the trunk
    mixer, fed an embedding table of +-1 rows (whose norm is the identity in
    bf16), receives exactly the trunk layer's input streams; it must then
    reproduce the trunk layer's output streams, KV and greedy tokens bit for
    bit at the same positions.  This ties the draft step's positions (RoPE),
    its own KV cache plane and its mixer to the trunk layer, which the
    reference fixture pins through the composition test; drafting one
    position late breaks it.

The engine's draft step is bit-exact with Model.mtp_step (tests/
test_mtp_gpu.py), so these pins carry over to it."""
import numpy as np
import pytest

from mlx_ckpt import engine_tensors, make_fetch, synth_checkpoint
from oracle import oracle as orc
from oracle.model import Model

U = 2.0 ** -8  # bf16 unit roundoff


def _f64(bits16):
    return orc.bf16_to_f32(np.asarray(bits16, np.uint16)).astype(np.float64)


def _dequant64(E, name, n, k, bits):
    """W = s * q + b in float64 (value j of a row at bit j*bits of the row's
    little-endian bitstream)."""
    codes = np.ascontiguousarray(E[name + ".codes"]).reshape(n, k * bits // 32)
    bitsarr = np.unpackbits(codes.view(np.uint8).reshape(n, -1), axis=1, bitorder="little")
    q = (bitsarr.reshape(n, k, bits) * (1 << np.arange(bits))).sum(axis=2).astype(np.float64)
    s = _f64(E[name + ".scales"]).reshape(n, k // 64)
    b = _f64(E[name + ".biases"]).reshape(n, k // 64)
    g = np.arange(k) // 64
    return s[:, g] * q + b[:, g]


def _norm64(x, w, eps):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * (1.0 + w)


@pytest.fixture(scope="module")
def tiny(mx):
    cfg = dict(mx.TINY, mtp=1, max_slots=2, max_context=64)
    T, _ = synth_checkpoint(cfg, 31)
    E = engine_tensors(mx, cfg, T)
    return cfg, E


def _inputs(cfg, rows=3, seed=7):
    rng = np.random.default_rng(seed)
    H, hc = cfg["hidden"], cfg["hc"]
    tokens = [int(t) for t in rng.integers(0, cfg["vocab"], rows)]
    # streams of different scales, so a per-stream norm differs from the global one
    scale = np.repeat([1.0, 2.0, 4.0, 8.0], H)[None, :]
    prev = orc.f32_to_bf16((rng.standard_normal((rows, hc * H)) * scale).astype(np.float32))
    return tokens, prev


def _closed_form(cfg, E, tokens, prev):
    """float64 h, and the elementwise bound of the oracle's bf16 chain."""
    H, hc, eps = cfg["hidden"], cfg["hc"], cfg["rms_eps"]
    rows = len(tokens)
    emb = _dequant64(E, "embed", cfg["vocab"], H, cfg["embed_bits"])[tokens]
    We = _dequant64(E, "mtp.fc_emb", H, H, cfg["bits"])
    Wh = _dequant64(E, "mtp.fc_hidden", H, H, cfg["bits"])
    a = _norm64(emb, _f64(E["mtp.norm_emb"]), eps)
    e = a @ We.T
    hn = _norm64(_f64(prev), _f64(E["mtp.norm_hidden"]), eps).reshape(rows, hc, H)
    f = hn @ Wh.T
    h = e[:, None, :] + f
    # emb, its norm and a: 3 roundings feed e; hn 2 roundings feed f; e, f, h one each
    bound = U * (np.abs(h) + np.abs(e)[:, None, :] + np.abs(f)) \
        + 3 * U * (np.abs(a) @ np.abs(We).T)[:, None, :] + 2 * U * (np.abs(hn) @ np.abs(Wh).T)
    return h.reshape(rows, hc * H), 1.25 * bound.reshape(rows, hc * H) + 1e-30


def test_draft_input_streams_match_the_float64_closed_form(tiny):
    cfg, E = tiny
    model = Model(cfg, make_fetch(E))
    tokens, prev = _inputs(cfg)
    got = _f64(model.mtp_compose(tokens, prev))
    want, bound = _closed_form(cfg, E, tokens, prev)
    err = np.abs(got - want)
    print(f"max err / bound {np.max(err / bound):.3f}; max rel err "
          f"{np.max(err) / np.max(np.abs(want)):.2e}")
    assert (err <= bound).all(), float(np.max(err / bound))
    assert np.max(err / bound) > 0.0  # the bf16 chain does round somewhere


# ---- mistakes planted in the composition (each restated with the oracle's
# primitives, then held to the same closed form) ----------------------------
def _compose(model, tokens, prev, mistake):
    import ctypes as C

    c, m = model.c, model.mtp
    H, hc, eps = model.H, model.hc, c["rms_eps"]
    rows = len(tokens)
    tok = np.ascontiguousarray(tokens, np.uint32)
    emb = np.empty((rows, H), np.uint16)
    orc.lib.mxo_embed(C.byref(model.embed), orc._p(tok), rows, 1, orc._p(emb))
    w_e, w_h = m["norm_emb"], m["norm_hid"]
    if mistake == "no-plus-one":     # scale (w) in place of (w + 1): pass w - 1
        w_e = orc.f32_to_bf16((orc.bf16_to_f32(w_e) - 1).astype(np.float32))
        w_h = orc.f32_to_bf16((orc.bf16_to_f32(w_h) - 1).astype(np.float32))
    a = np.empty_like(emb)
    orc.lib.mxo_hc_norm(orc._p(emb), orc._p(w_e), rows, 1, H, eps, orc._p(a))
    prev = np.ascontiguousarray(prev, np.uint16)
    hn = np.empty_like(prev)
    if mistake == "per-stream-norm":
        orc.lib.mxo_hc_norm(orc._p(prev), orc._p(w_h), rows, hc, H, eps, orc._p(hn))
    elif mistake == "hidden-unnormalised":
        hn = prev.copy()
    else:
        orc.lib.mxo_hc_norm(orc._p(prev), orc._p(w_h), rows, 1, hc * H, eps, orc._p(hn))
    fe, fh = (m["fc_hid"], m["fc_emb"]) if mistake == "swapped-projections" else \
        (m["fc_emb"], m["fc_hid"])
    e = orc.bf16_to_f32(model._qmv(fe, a)).astype(np.float32)
    f = orc.bf16_to_f32(model._qmv(fh, hn.reshape(rows * hc, H))).astype(np.float32)
    f = f.reshape(rows, hc, H)
    if mistake == "one-stream":
        f[:, 0, :] += e
        s = f
    else:
        s = e[:, None, :] + f
    return orc.f32_to_bf16(s.astype(np.float32)).reshape(rows, hc * H)


def test_the_restated_composition_equals_the_oracle(tiny):
    cfg, E = tiny
    model = Model(cfg, make_fetch(E))
    tokens, prev = _inputs(cfg)
    assert (_compose(model, tokens, prev, None) == model.mtp_compose(tokens, prev)).all()


@pytest.mark.parametrize("mistake", ["per-stream-norm", "no-plus-one", "one-stream",
                                     "swapped-projections", "hidden-unnormalised"])
def test_planted_composition_mistakes_break_the_closed_form(tiny, mistake):
    cfg, E = tiny
    model = Model(cfg, make_fetch(E))
    tokens, prev = _inputs(cfg)
    got = _f64(_compose(model, tokens, prev, mistake))
    want, bound = _closed_form(cfg, E, tokens, prev)
    ratio = np.max(np.abs(got - want) / bound)
    print(f"{mistake}: max err / bound {ratio:.1f}")
    assert ratio > 1.0


# ---- reduction to a trunk layer --------------------------------------------
def _pack(values, bits):
    """MLX packing of integer codes [n, k] (value j at bit j*bits)."""
    n, k = values.shape
    b = ((values[:, :, None] >> np.arange(bits)) & 1).astype(np.uint8).reshape(n, k * bits)
    return np.packbits(b, axis=1, bitorder="little").view(np.uint32).reshape(n, k * bits // 32)


def _reduction_model(mx, seed=33):
    cfg = dict(mx.TINY, layers=1, attn_every=1, mtp=1, max_slots=2, max_context=64)
    T, _ = synth_checkpoint(cfg, seed)
    E = engine_tensors(mx, cfg, T)
    H, V, bits = cfg["hidden"], cfg["vocab"], cfg["bits"]
    for k in list(E):
        if k.startswith("layers.0."):
            E["mtp.layer." + k[len("layers.0."):]] = E[k].copy()
        if k.startswith("mixer."):
            E["mtp.mixer." + k[len("mixer."):]] = E[k].copy()
    one, zero = np.uint16(0x3F80), np.uint16(0)
    E["mtp.fc_emb.codes"] = _pack(np.eye(H, dtype=np.int64), bits)         # identity
    E["mtp.fc_emb.scales"] = np.full((H, H // 64), one, np.uint16)
    E["mtp.fc_emb.biases"] = np.full((H, H // 64), zero, np.uint16)
    E["mtp.fc_hidden.codes"] = np.zeros((H, H * bits // 32), np.uint32)   # zero
    E["mtp.fc_hidden.scales"] = np.zeros((H, H // 64), np.uint16)
    E["mtp.fc_hidden.biases"] = np.zeros((H, H // 64), np.uint16)
    E["mtp.norm_emb"] = np.zeros(H, np.uint16)                          # scale 0 + 1
    # embedding rows of +-1: 8-bit codes 0 / 2 with scale 1, bias -1
    signs = np.random.default_rng(seed).integers(0, 2, (V, H)) * 2
    E["embed.codes"] = _pack(signs.astype(np.int64), cfg["embed_bits"])
    E["embed.scales"] = np.full((V, H // 64), one, np.uint16)
    E["embed.biases"] = np.full((V, H // 64), np.uint16(0xBF80), np.uint16)
    return cfg, E


@pytest.mark.parametrize("late", [0, 1], ids=["same-positions", "planted-one-late"])
def test_draft_layer_with_trunk_weights_reproduces_the_trunk_layer(mx, late):
    cfg, E = _reduction_model(mx)
    model = Model(cfg, make_fetch(E))
    tokens = [3, 900, 17, 250, 42, 7]
    rows = len(tokens)
    want_tok = model.block(0, tokens)
    want_h = model.hidden.copy()
    trunk_in = model.layer_in[0].copy()
    prev = orc.f32_to_bf16(np.random.default_rng(1).standard_normal(
        (rows, cfg["hc"] * cfg["hidden"])).astype(np.float32))
    got_tok = model.mtp_step(1, tokens, late, prev)
    # the composed stream is the trunk layer's input, whatever `prev` holds
    assert (model.mtp_input == trunk_in).all()
    same_h = (model.mtp_hidden == want_h).all()
    same_tok = [int(t) for t in got_tok] == [int(t) for t in want_tok]
    # the draft wrote its own KV plane (cache index n_attn) of slot 1; the
    # trunk's plane of slot 0 holds the same keys and values
    kv = model.kv_slot_stride
    c = model.c
    plane = c["kv_heads"] * c["max_context"] * c["head_dim"]
    trunk_k = model.k[0:plane].reshape(c["kv_heads"], c["max_context"], -1)[:, :rows]
    draft_k = model.k[kv + model.n_attn * plane: kv + (model.n_attn + 1) * plane].reshape(
        c["kv_heads"], c["max_context"], -1)[:, late:late + rows]
    same_kv = (trunk_k == draft_k).all()
    if late == 0:
        assert same_h and same_tok and same_kv
    else:
        assert not same_h and not same_kv  # RoPE at the wrong positions
