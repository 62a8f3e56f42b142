"""Checkpoint loading into the engine (mx_engine_load_safetensors): the MLX
tensor names the reference's loaders read (src/weights.rs:22-99,
src/hybrid.rs:56-66, 130-142, 335-352, 529-567, src/mtp.rs:39-70) onto the
engine's fused matrices (the names and shapes of the reference's own fixture
are checked on the CPU, tests/test_loader.py).  Round trip: an engine's
weights written out under MLX names (the fused matrices split back into the
reference's modules) and loaded into an engine with other seeded weights
make every weight buffer equal byte for byte, and the two engines prefill
and decode the same tokens in exact mode; a tensor of a module the engine
does not build, or with other widths, is refused with its name."""
import json
import os
import struct

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
NP_OF = {"U32": np.uint32, "BF16": np.uint16, "F16": np.float16, "F32": np.float32}


def _export(eng, cfg, path):
    """The engine's weights under MLX names, the fused matrices split back."""
    c = cfg
    tensors = {}
    gs = c["group_size"]

    def quant(name, src, n, k, bits, row0, rows):
        words, groups = k * bits // 32, k // gs
        codes = eng.read(src + ".codes", np.uint32, (n, words))
        sc = eng.read(src + ".scales", np.uint16, (n, groups))
        bi = eng.read(src + ".biases", np.uint16, (n, groups))
        tensors[name + ".weight"] = ("U32", codes[row0:row0 + rows])
        tensors[name + ".scales"] = ("BF16", sc[row0:row0 + rows])
        tensors[name + ".biases"] = ("BF16", bi[row0:row0 + rows])

    def bank(name, src, e, n, k, bits):
        words, groups = k * bits // 32, k // gs
        tensors[name + ".weight"] = ("U32", eng.read(src + ".codes", np.uint32, (e, n, words)))
        tensors[name + ".scales"] = ("BF16", eng.read(src + ".scales", np.uint16, (e, n, groups)))
        tensors[name + ".biases"] = ("BF16", eng.read(src + ".biases", np.uint16, (e, n, groups)))

    H, hc, r, b = c["hidden"], c["hc"], c["hc_rank"], c["bits"]

    def hcw(name, src, inject):
        tensors[name + ".hc_norm.weight"] = ("BF16", eng.read(src + ".scale", np.uint16, (hc * H,)))
        n_down = r + (hc if inject else 0)
        quant(name + ".input_mix_weight_down", src + ".down", n_down, hc * H, b, 0, r)
        if inject:
            quant(name + ".block_inject_weight", src + ".down", n_down, hc * H, b, r, hc)
        quant(name + ".input_mix_weight_up", src + ".up", hc * H, r, b, 0, hc * H)

    lm = "language_model."
    quant(lm + "model.embed_tokens", "embed", c["vocab"], H, c["embed_bits"], 0, c["vocab"])
    quant(lm + "lm_head", "head", c["vocab"], H, c["head_bits"], 0, c["vocab"])
    hcw(lm + "model.hyper_connection_mixer", "mixer", False)
    cd = 2 * c["gdn_hk"] * c["gdn_dk"] + c["gdn_hv"] * c["gdn_dv"]
    vd = c["gdn_hv"] * c["gdn_dv"]
    hv = c["gdn_hv"]
    P = cd + vd + 2 * hv
    qr = c["heads"] * 2 * c["head_dim"]
    kv = c["kv_heads"] * c["head_dim"]
    E, I, SI = c["experts"], c["moe_inter"], c["shared_inter"]
    for i in range(c["layers"]):
        p, s = f"{lm}model.layers.{i}", f"layers.{i}"
        hcw(p + ".attn_hyper_connection", s + ".attn_hc", True)
        hcw(p + ".mlp_hyper_connection", s + ".mlp_hc", True)
        if i % c["attn_every"] != c["attn_every"] - 1:
            la = p + ".linear_attn"
            for nm, r0, rows in (("in_proj_qkv", 0, cd), ("in_proj_z", cd, vd),
                                 ("in_proj_a", cd + vd, hv), ("in_proj_b", cd + vd + hv, hv)):
                quant(f"{la}.{nm}", s + ".gdn.in", P, H, b, r0, rows)
            quant(la + ".out_proj", s + ".gdn.out", H, vd, b, 0, H)
            conv = eng.read(s + ".gdn.conv_w", np.float32, (c["conv_k"], cd))
            tensors[la + ".conv1d.weight"] = ("F32", np.ascontiguousarray(conv.T)[:, :, None])
            tensors[la + ".A_log"] = ("F32", eng.read(s + ".gdn.a_log", np.float32, (hv,)))
            tensors[la + ".dt_bias"] = ("BF16", eng.read(s + ".gdn.dt_bias", np.uint16, (hv,)))
            tensors[la + ".norm.weight"] = ("BF16", eng.read(s + ".gdn.norm", np.uint16, (c["gdn_dv"],)))
        else:
            sa = p + ".self_attn"
            Q = qr + 2 * kv
            quant(sa + ".q_proj", s + ".attn.in", Q, H, b, 0, qr)
            quant(sa + ".k_proj", s + ".attn.in", Q, H, b, qr, kv)
            quant(sa + ".v_proj", s + ".attn.in", Q, H, b, qr + kv, kv)
            quant(sa + ".o_proj", s + ".attn.out", H, c["heads"] * c["head_dim"], b, 0, H)
            for nm in ("q_norm", "k_norm"):
                tensors[f"{sa}.{nm}.weight"] = ("BF16", eng.read(f"{s}.attn.{nm}", np.uint16,
                                                                 (c["head_dim"],)))
        mp = p + ".mlp"
        quant(mp + ".gate", s + ".moe.router", E + 1, H, b, 0, E)
        quant(mp + ".shared_expert_gate", s + ".moe.router", E + 1, H, b, E, 1)
        bank(mp + ".switch_mlp.gate_proj", s + ".moe.gate", E, I, H, b)
        bank(mp + ".switch_mlp.up_proj", s + ".moe.up", E, I, H, b)
        bank(mp + ".switch_mlp.down_proj", s + ".moe.down", E, H, I, c["down_bits"])
        quant(mp + ".shared_expert.gate_proj", s + ".moe.shared_gate", SI, H, b, 0, SI)
        quant(mp + ".shared_expert.up_proj", s + ".moe.shared_up", SI, H, b, 0, SI)
        quant(mp + ".shared_expert.down_proj", s + ".moe.shared_down", H, SI, c["down_bits"], 0, H)
    # safetensors: JSON header, then the tensors' bytes in order
    header, blobs, off = {}, [], 0
    for name, (dt, a) in tensors.items():
        a = np.ascontiguousarray(a, NP_OF[dt])
        header[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + a.nbytes]}
        blobs.append(a.tobytes())
        off += a.nbytes
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for blob in blobs:
            f.write(blob)
    return len(tensors)


def test_round_trip_through_an_mlx_checkpoint(mx, tmp_path):
    cfg = dict(mx.TINY)
    a = mx.Engine(dict(cfg, seed=77))
    b = mx.Engine(dict(cfg, seed=1234))
    try:
        path = tmp_path / "model.safetensors"
        n = _export(a, cfg, path)
        assert b.load_safetensors(str(path)) == n
        names = [k for k in a_names(mx, a) if not k.startswith(("cache.", "verify.", "act.", "rope."))]
        assert len(names) > 50
        for nm in names:
            nb = a.tensor_bytes(nm)
            assert (a.read(nm, np.uint8, (nb,)) == b.read(nm, np.uint8, (nb,))).all(), nm
        for e in (a, b):
            e.set_flags(exact=True)
        slots = [0, 1, 2]
        prompts = [[5, 17, 300], [9, 2], [1000, 44, 7, 8]]
        ta = [a.prefill(s, p) for s, p in zip(slots, prompts)]
        tb = [b.prefill(s, p) for s, p in zip(slots, prompts)]
        assert ta == tb
        for _ in range(3):
            ta = a.decode_batch(slots, ta, equal=False)
            tb = b.decode_batch(slots, tb, equal=False)
            assert (ta == tb).all()
        # refusals name the tensor and the difference
        rc = b.load_tensor("language_model.model.layers.0.ple.key_proj.weight",
                           np.zeros((4, 4), np.uint32), raise_on_error=False)
        assert rc == mx.MX_EUNSUPPORTED and b"ple" in mx.lib.mx_last_error()
        wrong = np.zeros((cfg["vocab"], cfg["hidden"] * 4 // 32), np.uint32)  # 4-bit, head is 8
        rc = b.load_tensor("language_model.lm_head.weight", wrong, raise_on_error=False)
        assert rc == mx.MX_EUNSUPPORTED and b"4-bit" in mx.lib.mx_last_error()
    finally:
        a.close()
        b.close()


def a_names(mx, eng):
    """The engine's weight tensor names, from the TINY layout."""
    c = eng.cfg
    names = ["embed", "head"]
    qw = lambda p: [p + ".codes", p + ".scales", p + ".biases"]  # noqa: E731
    out = qw("embed") + qw("head") + ["mixer.scale"] + qw("mixer.down") + qw("mixer.up")
    for i in range(c["layers"]):
        s = f"layers.{i}"
        for h in ("attn_hc", "mlp_hc"):
            out += [f"{s}.{h}.scale"] + qw(f"{s}.{h}.down") + qw(f"{s}.{h}.up")
        if i % c["attn_every"] != c["attn_every"] - 1:
            out += qw(s + ".gdn.in") + qw(s + ".gdn.out") + [s + ".gdn.conv_w", s + ".gdn.a_log",
                                                           s + ".gdn.dt_bias", s + ".gdn.norm"]
        else:
            out += qw(s + ".attn.in") + qw(s + ".attn.out") + [s + ".attn.q_norm", s + ".attn.k_norm"]
        for m in ("router", "gate", "up", "down", "shared_gate", "shared_up", "shared_down"):
            out += qw(f"{s}.moe.{m}")
    return out


def test_mixed_width_checkpoint_runs_bit_exact_with_the_oracle(mx, tmp_path):
    """A synthetic MLX checkpoint whose layers are quantised at their own
    widths (per-module quantization entries, src/weights.rs:70-90): its
    config.json gives the engine's width table (config_from_mlx), the file
    loads into the engine, every engine weight equals the file's mapping
    through mx_checkpoint_target, and the exact engine's speculative
    generation (prefill, verify blocks, the MTP draft layer) and batched
    decode equal the oracle model's on the same tensors bit for bit."""
    from mlx_ckpt import engine_tensors, make_fetch, synth_checkpoint, write_safetensors
    from oracle.model import Model

    base = dict(mx.TINY, mtp=1, vocab=16)
    widths = {0: (8, 6), 1: (5, 4), 2: (6, 8), 3: (5, 5), 4: (8, 4)}  # index 4: the MTP layer
    T, config = synth_checkpoint(base, 21, widths)
    cfg = mx.config_from_mlx(config, max_slots=3, max_context=96, seed=9, mtp=1)
    assert cfg["layer_widths"][:10] == [8, 6, 5, 4, 6, 8, 5, 5, 8, 4]
    path = tmp_path / "mixed.safetensors"
    n = write_safetensors(path, T)
    assert mx.checkpoint_check(cfg, path) == n
    E = engine_tensors(mx, cfg, T)
    eng = mx.Engine(cfg)
    try:
        assert eng.load_safetensors(str(path)) == n
        for name, a in E.items():
            assert (eng.read(name, a.dtype, a.shape) == a).all(), name
        eng.set_flags(exact=True)
        model = Model(cfg, make_fetch(E))
        prompt = [int(t) for t in np.random.default_rng(6).integers(0, 16, 13)]
        toks, st = eng.generate(0, prompt, 12, 3)
        want, wst = model.generate(0, prompt, 12, 3)
        assert [int(t) for t in toks] == want
        assert [int(d) for d in st["drafts"]] == wst["drafts"]
        assert (st["rounds"], st["accepted"]) == (wst["rounds"], wst["accepted"])
        # two more slots decoded together, at their own offsets
        for s, p in ((1, prompt[:5]), (2, prompt[3:12])):
            assert eng.prefill(s, p) == int(model.prefill(s, p))
        t = [int(x) for x in model.decode_rows([1, 2], [3, 7])]
        assert [int(x) for x in eng.decode_batch([1, 2], [3, 7], equal=False)] == t
    finally:
        eng.close()


def test_a_checkpoint_value_that_would_round_is_refused(mx, tmp_path):
    """An fp32 scale that bf16 cannot hold stops the load with its name."""
    from mlx_ckpt import synth_checkpoint, write_safetensors

    T, config = synth_checkpoint(dict(mx.TINY), 5)
    cfg = mx.config_from_mlx(config, max_slots=1, max_context=32)
    name = "language_model.model.layers.1.mlp.switch_mlp.up_proj.scales"
    T[name] = T[name].copy()
    T[name].reshape(-1)[3] += np.float32(1e-5)
    path = tmp_path / "inexact.safetensors"
    write_safetensors(path, T, dtypes={name: "F32"})
    eng = mx.Engine(cfg)
    try:
        with pytest.raises(mx.MxError, match="up_proj.scales: value"):
            eng.load_safetensors(str(path))
    finally:
        eng.close()
