"""The oracle's model composition against the float32 restatement, on the CPU.

oracle/model.py strings the oracle's C primitives together the way the engine
does (bf16 activations, exact-integer projections, fused matrices).  Its
wiring -- which stream feeds which projection, where the injections, gates,
shared expert, caches and the mixer enter -- is checked here against
oracle/hybrid.py, a float32 restatement of the reference's HybridModel and
Mtp (src/hybrid.rs:594-685, src/mtp.rs:72-127) that the reference's own
end-to-end fixture pins (tests/test_hybrid_fixture.py).

Both read ONE synthetic MLX-format checkpoint: the restatement by the MLX
tensor names, the oracle through mx_checkpoint_target -- the mapping
mx_engine_load_tensor applies -- onto the engine's fused matrices, so the
loader's mapping is checked by the same comparison.  The two differ by the
engine's bf16 rounding points (about 2^-9 relative per step), so hidden
streams and logits are compared in relative L2 norm with a bound a few times
the measured drift, and the routed experts must agree.  Mistakes planted in
the oracle's wiring (a dropped injection, a dropped shared expert,
unnormalised routing scores, a recurrent state that is not carried, RoPE
rotating the wrong way) each fail that check.  The draft layer (Mtp) has no
reference fixture: its comparison checks the oracle's draft step against a
second, independent restatement only."""
import numpy as np
import pytest

from oracle import hybrid as hy

TOL = 0.02          # relative L2 bound on hidden streams and logits (drift measured: 0.0086)
PROMPT = [5, 901, 17, 333, 42, 7, 610]
STEPS = 3


def bf16(a):
    a = np.ascontiguousarray(a, np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return u.view(np.float32)


def synth_checkpoint(cfg, seed):
    """(tensors by MLX name, config.json) of a random model of the engine
    configuration cfg, in MLX's affine layout; float values are bf16."""
    rng = np.random.default_rng(seed)
    H, hc, r, gs = cfg["hidden"], cfg["hc"], cfg["hc_rank"], cfg["group_size"]
    T = {}
    quant_over = {}

    def quant(p, n, k, bits, lead=(), gain=1.0, kscale=True):
        T[p + ".weight"] = rng.integers(0, 2**32, size=lead + (n, k * bits // 32),
                                        dtype=np.uint64).astype(np.uint32)
        s = gain * np.sqrt(12.0) / ((np.sqrt(k) if kscale else 1.0) * 2**bits)
        sc = bf16(s * rng.uniform(0.75, 1.25, size=lead + (n, k // gs)))
        T[p + ".scales"] = sc
        T[p + ".biases"] = bf16(-sc * (2**bits - 1) / 2 + sc * rng.normal(0, 0.1, size=sc.shape))
        if bits != cfg["bits"]:
            quant_over[p] = {"bits": bits, "group_size": gs}

    def vec(p, shape, mean, std):
        T[p] = bf16(mean + std * rng.normal(size=shape))

    def hcw(p, layer_bits, inject):
        vec(p + ".hc_norm.weight", (hc * H,), 0.0, 0.1)
        quant(p + ".input_mix_weight_down", r, hc * H, layer_bits, gain=2.0)
        quant(p + ".input_mix_weight_up", hc * H, r, layer_bits)
        if inject:
            quant(p + ".block_inject_weight", hc, hc * H, layer_bits, gain=2.0)

    def moe(p, bits, dbits):
        E, I, SI = cfg["experts"], cfg["moe_inter"], cfg["shared_inter"]
        quant(p + ".gate", E, H, bits, gain=3.0)
        quant(p + ".shared_expert_gate", 1, H, bits)
        quant(p + ".switch_mlp.gate_proj", I, H, bits, lead=(E,))
        quant(p + ".switch_mlp.up_proj", I, H, bits, lead=(E,))
        quant(p + ".switch_mlp.down_proj", H, I, dbits, lead=(E,))
        quant(p + ".shared_expert.gate_proj", SI, H, bits)
        quant(p + ".shared_expert.up_proj", SI, H, bits)
        quant(p + ".shared_expert.down_proj", H, SI, dbits)

    def attn(p, bits):
        hd = cfg["head_dim"]
        quant(p + ".q_proj", cfg["heads"] * 2 * hd, H, bits)
        quant(p + ".k_proj", cfg["kv_heads"] * hd, H, bits)
        quant(p + ".v_proj", cfg["kv_heads"] * hd, H, bits)
        quant(p + ".o_proj", H, cfg["heads"] * hd, bits)
        vec(p + ".q_norm.weight", (hd,), 0.0, 0.1)
        vec(p + ".k_norm.weight", (hd,), 0.0, 0.1)

    bits, dbits = cfg["bits"], cfg["down_bits"]
    lm = "language_model.model."
    quant("language_model.model.embed_tokens", cfg["vocab"], H, cfg["embed_bits"], kscale=False)
    quant("language_model.lm_head", cfg["vocab"], H, cfg["head_bits"])
    hcw(lm + "hyper_connection_mixer", bits, False)
    hk, hv, dk, dv = cfg["gdn_hk"], cfg["gdn_hv"], cfg["gdn_dk"], cfg["gdn_dv"]
    types = []
    for i in range(cfg["layers"]):
        p = f"{lm}layers.{i}"
        full = i % cfg["attn_every"] == cfg["attn_every"] - 1
        types.append("full_attention" if full else "linear_attention")
        hcw(p + ".attn_hyper_connection", bits, True)
        hcw(p + ".mlp_hyper_connection", bits, True)
        if full:
            attn(p + ".self_attn", bits)
        else:
            g = p + ".linear_attn"
            cd = 2 * hk * dk + hv * dv
            quant(g + ".in_proj_qkv", cd, H, bits)
            quant(g + ".in_proj_z", hv * dv, H, bits)
            quant(g + ".in_proj_a", hv, H, bits)
            quant(g + ".in_proj_b", hv, H, bits)
            quant(g + ".out_proj", H, hv * dv, bits)
            T[g + ".conv1d.weight"] = bf16(rng.normal(0, 0.5, size=(cd, cfg["conv_k"], 1)))
            T[g + ".A_log"] = rng.uniform(-1.0, 1.0, size=(hv,)).astype(np.float32)
            T[g + ".dt_bias"] = bf16(rng.uniform(0.0, 1.0, size=(hv,)))
            vec(g + ".norm.weight", (dv,), 1.0, 0.1)
        moe(p + ".mlp", bits, dbits)
    if cfg.get("mtp"):
        p = "mtp.layers.0"
        hcw(p + ".attn_hyper_connection", bits, True)
        hcw(p + ".mlp_hyper_connection", bits, True)
        attn(p + ".self_attn", bits)
        moe(p + ".mlp", bits, dbits)
        vec("mtp.pre_fc_norm_embedding.weight", (H,), 0.0, 0.1)
        vec("mtp.pre_fc_norm_hidden.weight", (hc * H,), 0.0, 0.1)
        quant("mtp.fc_embedding", H, H, bits)
        quant("mtp.fc_hidden", H, H, bits)
        hcw("mtp.hyper_connection_mixer", bits, False)
    text = dict(hidden_size=H, num_hidden_layers=cfg["layers"], hc_count=hc, hc_lowrank=r,
                num_attention_heads=cfg["heads"], num_key_value_heads=cfg["kv_heads"],
                head_dim=cfg["head_dim"], linear_num_key_heads=hk, linear_num_value_heads=hv,
                linear_key_head_dim=dk, linear_value_head_dim=dv,
                linear_conv_kernel_dim=cfg["conv_k"], num_experts=cfg["experts"],
                num_experts_per_tok=cfg["top_k"], moe_intermediate_size=cfg["moe_inter"],
                shared_expert_intermediate_size=cfg["shared_inter"], rms_norm_eps=cfg["rms_eps"],
                vocab_size=cfg["vocab"], layer_types=types, ngram_size=3, eos_token_id=cfg["vocab"] - 1,
                rope_parameters=dict(rope_theta=cfg["rope_theta"],
                                     partial_rotary_factor=cfg["rotary_dim"] / cfg["head_dim"]))
    config = {"text_config": text,
              "quantization": dict(bits=bits, group_size=gs, mode="affine", **quant_over)}
    return T, config


def engine_tensors(mx, cfg, T):
    """The engine's tensors (oracle fetch names) assembled from the MLX ones by
    mx_checkpoint_target."""
    out = {}
    gs = cfg["group_size"]
    u16 = lambda a: (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)
    for name, a in T.items():
        rc, tensor, t = mx.checkpoint_target(cfg, name)
        assert rc == 0, (name, rc)
        kind = t["kind"]
        if kind == 0:                                   # quantised rows
            a2 = a.reshape(-1, a.shape[-1])
            assert a2.shape[0] == t["rows"], (name, a2.shape, t)
            part = t["part"]
            suffix = (".codes", ".scales", ".biases")[part]
            width = t["k"] * t["bits"] // 32 if part == 0 else t["k"] // gs
            dt = np.uint32 if part == 0 else np.uint16
            buf = out.setdefault(tensor + suffix, np.zeros((t["n"], width), dt))
            assert a2.shape[1] == width, (name, a2.shape, width)
            buf[t["row0"]:t["row0"] + t["rows"]] = a2 if part == 0 else u16(a2)
        elif kind == 1:                                 # bf16 vector
            assert a.size == t["count"], name
            out[tensor] = u16(a.reshape(-1))
        elif kind == 2:                                 # fp32 vector
            out[tensor] = np.ascontiguousarray(a, np.float32).reshape(-1)
        else:                                           # conv [C, K, 1] -> [K][C]
            out[tensor] = np.ascontiguousarray(a[:, :, 0].T, np.float32)
    return out


def make_fetch(E):
    def fetch(name, dtype, shape):
        a = E[name]
        assert a.dtype == np.dtype(dtype) and a.size == int(np.prod(shape)), (name, a.shape, shape)
        return np.ascontiguousarray(a.reshape(shape))
    return fetch


@pytest.fixture(scope="module")
def setup(mx):
    cfg = dict(mx.TINY, mtp=1, max_slots=1, max_context=64)
    T, config = synth_checkpoint(cfg, seed=11)
    E = engine_tensors(mx, cfg, T)
    return cfg, T, config, E


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def run_pair(cfg, T, config, E, plant=None):
    """Prefill PROMPT, then STEPS greedy decode steps (tokens chosen by the
    restatement, fed to both).  Returns the worst relative differences of
    (hidden streams, logits) and whether every routing agreed."""
    from oracle import oracle as orc
    from oracle.model import Model

    ref = hy.HybridModel(hy.Weights(T, config))
    model = Model(cfg, make_fetch(E))
    if plant:
        plant(model)
    worst_h = worst_l = 0.0
    routes_equal = True
    toks = list(PROMPT)
    for step in range(STEPS + 1):
        feed = list(toks) if step == 0 else toks[-1:]
        lr, hr = ref.forward(feed)
        nxt = model.block(0, feed) if step == 0 else model.decode_rows([0], feed)
        ho = orc.bf16_to_f32(model.hidden).reshape(hr.shape)
        lo = orc.bf16_to_f32(model._qmv(model.head, model.last_mixed))
        worst_h = max(worst_h, _rel(ho, hr))
        worst_l = max(worst_l, _rel(lo, lr))
        for ids_o, ids_r in zip(model.last_ids, ref.routes):
            routes_equal &= all(set(a.tolist()) == set(b.tolist()) for a, b in zip(ids_o, ids_r))
        toks.append(int(np.argmax(lr[-1])))
        assert len(nxt) == len(feed)
    return worst_h, worst_l, routes_equal


def test_oracle_model_matches_the_restatement(setup):
    cfg, T, config, E = setup
    h, l, routes = run_pair(cfg, T, config, E)
    print(f"hidden rel {h:.4g} logits rel {l:.4g}")
    assert routes, "routed experts differ"
    assert h <= TOL and l <= TOL, (h, l)


def test_oracle_draft_layer_matches_the_restatement(setup):
    """Mtp::forward (src/mtp.rs:72-127) in the oracle (Model.mtp_step) against
    the restatement's Mtp, on the target's hidden streams after the prompt."""
    from oracle import oracle as orc
    from oracle.model import Model

    cfg, T, config, E = setup
    W = hy.Weights(T, config)
    ref = hy.HybridModel(W)
    mtp = hy.Mtp(W, ref)
    model = Model(cfg, make_fetch(E))
    _, hr = ref.forward(PROMPT)
    model.block(0, PROMPT)
    prev = model.hidden.copy()
    nxt = PROMPT[1:] + [3]
    d = model.mtp_step(0, nxt, 0, prev)
    mixed_r, h_r = mtp.forward(ref.embed(nxt), orc.bf16_to_f32(prev).reshape(hr.shape), 0)
    lr = hy.lin(mixed_r, ref.head)
    lo = orc.bf16_to_f32(model._qmv(model.head, model.last_mixed))
    ho = orc.bf16_to_f32(model.mtp_hidden).reshape(h_r.shape)
    print(f"draft hidden rel {_rel(ho, h_r):.4g} logits rel {_rel(lo, lr):.4g}")
    assert _rel(ho, h_r) <= TOL and _rel(lo, lr) <= TOL, (_rel(ho, h_r), _rel(lo, lr))
    assert len(d) == len(nxt)


# ---- planted mistakes (in the oracle, on the CPU) --------------------------
def _no_inject(model):
    f = model._hc_forward

    def g(w, h, rows):
        mixed, inj = f(w, h, rows)
        return mixed, np.full_like(inj, 0x3F80)      # bf16 1.0 in place of the gate
    model._hc_forward = g


def _no_shared(model):
    import oracle.model as om
    real = om.orc.moe_route

    def route(logits, shared, k):
        ids, scores, factor = real(logits, shared, k)
        return ids, scores, np.zeros_like(factor)
    om.orc = _Shim(om.orc, moe_route=route)


def _raw_scores(model):
    import oracle.model as om
    real = om.orc.moe_route

    def route(logits, shared, k):
        ids, scores, factor = real(logits, shared, k)
        f = om.orc.bf16_to_f32(scores) * 0.5          # scores no longer sum to one
        return ids, om.orc.f32_to_bf16(f.astype(np.float32)), factor
    om.orc = _Shim(om.orc, moe_route=route)


def _state_dropped(model):
    f = model.decode_rows

    def g(slots, tokens):
        model.state[...] = 0                           # recurrent state not carried
        return f(slots, tokens)
    model.decode_rows = g


def _rope_backwards(model):
    model.sin = np.ascontiguousarray(-model.sin)       # rotation in the wrong sense


class _Shim:
    def __init__(self, base, **over):
        self._base, self._over = base, over

    def __getattr__(self, k):
        return self._over.get(k, getattr(self._base, k))


@pytest.mark.parametrize("plant", [_no_inject, _no_shared, _raw_scores, _state_dropped,
                                   _rope_backwards],
                         ids=["no-inject", "no-shared-expert", "raw-scores", "state-dropped",
                              "rope-backwards"])
def test_planted_wiring_mistakes_fail_the_bound(setup, plant):
    import oracle.model as om
    cfg, T, config, E = setup
    saved = om.orc
    try:
        h, l, routes = run_pair(cfg, T, config, E, plant)
    finally:
        om.orc = saved
    print(f"{plant.__name__}: hidden rel {h:.4g} logits rel {l:.4g} routes equal {routes}")
    assert (not routes) or max(h, l) > TOL, (h, l, routes)
