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

from mlx_ckpt import engine_tensors, make_fetch, synth_checkpoint  # noqa: F401
from oracle import hybrid as hy

TOL = 0.02          # relative L2 bound on hidden streams and logits (drift measured: 0.0086)
PROMPT = [5, 901, 17, 333, 42, 7, 610]
STEPS = 3


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
