"""Parity of the decode engine at config 3's geometry (the size bench.py
times): hidden 2048, 512 experts top-10 with a 512-wide shared expert,
hyper-connections hc 4 / rank 256, GDN 16 key / 32 value heads of 128,
attention 16 q / 2 KV heads of 256, vocabulary 151936 -- the first four
layers of the stack ([G, G, G, A]) so that the CPU oracle model keeps up.

Exact mode, bit for bit against the oracle model (tokens, hidden streams,
routing, logits, GDN state, conv windows, KV):
  * ragged prefill of 8 slots, then batch-8 steps with every row at its own
    offset, and an equal-offset step through mx_engine_decode_batch_outputs
    (logits and hidden as HybridModel::decode_batch returns them,
    src/batching.rs:34-170) -- batch-parity.rs:126-171;
  * a 4-token verify block committed with keep 4, 1 and 0, each followed by a
    decode step, on the base widths and on config 4's mixed per-layer widths
    (verify-parity.rs:90-195, rollback-parity.rs, hybrid.rs:699-759).

Fast mode (the bf16 matrix-core path, not the benched one), teacher-forced:
every layer takes the oracle's input streams for that layer
(mx_engine_decode_forced), so each layer's error is its own, not the drift
of the layers before it.  Fast mode is not bit-exact: its matrix cores sum
bf16 products in an order that no IEEE evaluation reproduces, and where a
layer's output cancels (|w| near 0 next to inputs near 70) no elementwise
bound of the form 2e-2 |w| + 1e-2 holds -- the test prints that ratio (it
reaches about 55) and the exact mode above is the path that meets the north
star's bar.  What fast mode does keep, and the test asserts at this size:
  * routing equal to the oracle's except where the experts that differ have
    oracle router logits within one bf16 ulp of the oracle's 10th (a tie
    that a last-bit change in the logits may resolve either way);
  * every layer's output streams within 3e-2 relative L2 per row;
  * the greedy token equal to the oracle's unless the oracle's logits of the
    two tokens are within one bf16 ulp of each other;
  * the fp32 GDN state within 5e-2 relative (Frobenius) per (slot, layer):
    the state integrates the fast projections' k, v, beta and decay.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LAYERS = 4
PROMPTS = [3, 2, 9, 2, 5, 1, 4, 2]  # ragged prompt lengths of slots 0..7


def _bf(a):
    return (np.asarray(a, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _make(mx, **over):
    from oracle.model import Model

    cfg = dict(mx.CONFIG3, layers=LAYERS, max_context=96, **over)
    eng = mx.Engine(cfg)
    eng.set_flags(exact=True)
    model = Model(cfg, lambda name, dtype, shape: eng.read(name, dtype, shape))
    return eng, model


@pytest.fixture(scope="module")
def c3(mx):
    eng, model = _make(mx)
    yield eng, model
    eng.close()


def _kv_view(model, a):
    c = model.c
    return a.reshape(c["max_slots"], model.n_kv, c["kv_heads"], c["max_context"], c["head_dim"])


def _assert_caches_equal(eng, model, slots):
    c = model.c
    st = eng.read("cache.gdn_state", np.float32, model.state.shape)
    cv = eng.read("cache.conv_state", np.uint16, model.conv.shape)
    k = _kv_view(model, eng.read("cache.k", np.uint16, model.k.shape))
    v = _kv_view(model, eng.read("cache.v", np.uint16, model.v.shape))
    mk, mv = _kv_view(model, model.k), _kv_view(model, model.v)
    for s in slots:
        assert eng.offset(s) == model.offsets[s], s
        g = slice(s * model.n_gdn, (s + 1) * model.n_gdn)
        assert (st[g] == model.state[g]).all(), ("gdn state", s)
        assert (cv[g] == model.conv[g]).all(), ("conv window", s)
        off = model.offsets[s]
        assert (k[s, :, :, :off] == mk[s, :, :, :off]).all(), ("keys", s)
        assert (v[s, :, :, :off] == mv[s, :, :, :off]).all(), ("values", s)


def _clone(eng, model, src, dst):
    eng.clone(src, dst)
    n, kv = model.n_gdn, model.kv_slot_stride
    model.state[dst * n:(dst + 1) * n] = model.state[src * n:(src + 1) * n]
    model.conv[dst * n:(dst + 1) * n] = model.conv[src * n:(src + 1) * n]
    model.k[dst * kv:(dst + 1) * kv] = model.k[src * kv:(src + 1) * kv]
    model.v[dst * kv:(dst + 1) * kv] = model.v[src * kv:(src + 1) * kv]
    model.offsets[dst] = model.offsets[src]


def _hidden(eng, model, rows):
    return eng.read("hidden", np.uint16, (rows, model.c["hc"] * model.c["hidden"]))


def test_ragged_prefill_bit_exact(c3):
    eng, model = c3
    rng = np.random.default_rng(31)
    nxt = []
    for s, n in enumerate(PROMPTS):
        prompt = [int(t) for t in rng.integers(0, model.c["vocab"], n)]
        got = eng.prefill(s, prompt)
        want = model.prefill(s, prompt)
        print(f"prefill slot {s} ({n} tokens): engine {got} oracle {want}", flush=True)
        assert got == want, s
        assert (_hidden(eng, model, (n - 1) % 8 + 1) == model.hidden).all(), s
        nxt.append(got)
    _assert_caches_equal(eng, model, range(8))
    c3[1].next_tokens = nxt


def test_batch8_rows_at_own_offsets_bit_exact(c3):
    eng, model = c3
    slots = list(range(8))
    toks = list(model.next_tokens)
    for step in range(2):
        got = eng.decode_batch(slots, toks, equal=False)
        want = model.decode_rows(slots, toks)
        print(f"batch-8 step {step}: engine {list(got)} oracle {list(want)}", flush=True)
        assert (got == want).all(), step
        assert (_hidden(eng, model, 8) == model.hidden).all(), step
        ids = eng.read("act.ids", np.uint32, (8, model.c["top_k"]))
        assert (ids == model.last_ids[-1]).all(), step
        toks = [int(t) for t in want]
    _assert_caches_equal(eng, model, slots)
    model.next_tokens = toks


def test_equal_offset_batch_returns_logits_and_hidden(c3):
    """Slots 1, 3, 7 hold 2-token prompts, so they share an offset: one
    equal-offset step through mx_engine_decode_batch_outputs returns the
    oracle's greedy tokens, its bf16 logits (whose argmax the tokens are) and
    its final hidden streams; a ragged group is rejected."""
    eng, model = c3
    from oracle import oracle as orc

    slots = [1, 3, 7]
    assert len({eng.offset(s) for s in slots}) == 1
    toks = [model.next_tokens[s] for s in slots]
    got, logits, hidden = eng.decode_batch_outputs(slots, toks)
    want = model.decode_rows(slots, toks)
    assert (got == want).all()
    assert (hidden == model.hidden).all()
    want_logits = model._qmv(model.head, model.last_mixed)
    assert (logits == want_logits).all()
    assert (orc.argmax_bf16(logits) == got).all()
    for i, s in enumerate(slots):
        model.next_tokens[s] = int(got[i])
    with pytest.raises(Exception):
        eng.decode_batch_outputs([0, 2], [1, 2])  # offsets 5 and 11 differ


def _verify_commit_sequence(eng, model, slot, blocks):
    for keep, block in blocks:
        got = eng.verify(slot, block)
        want = model.verify(slot, block)
        assert (got == want).all(), keep
        assert (_hidden(eng, model, len(block)) == model.hidden).all(), keep
        eng.commit(slot, keep)
        model.commit(slot, keep)
        _assert_caches_equal(eng, model, [slot])
        tok = int(got[max(keep - 1, 0)])
        a = eng.decode_batch([slot], [tok])
        b = model.decode_rows([slot], [tok])
        assert a[0] == b[0], keep
        assert (_hidden(eng, model, 1) == model.hidden).all(), keep
        _assert_caches_equal(eng, model, [slot])


def test_verify_commit_rollback_bit_exact(c3):
    eng, model = c3
    _verify_commit_sequence(eng, model, 2, [(4, [11, 22, 33, 44]), (1, [5, 6, 7, 8]),
                                            (0, [9, 10, 11, 12])])


def test_verify_commit_rollback_mixed_widths_bit_exact(mx):
    """Config 4's per-layer widths ({4, 5, 6, 8} drawn by seed for the
    projections and the expert down banks) through prefill, verify and commit."""
    eng, model = _make(mx, mixed_bits=1, seed=60)
    try:
        widths = [model.layer_bits(i) for i in range(LAYERS)]
        print("layer widths", widths, flush=True)
        assert len({w for pair in widths for w in pair}) >= 3
        prompt = [7, 1234, 99, 150000, 3]
        assert eng.prefill(0, prompt) == model.prefill(0, prompt)
        _assert_caches_equal(eng, model, [0])
        _verify_commit_sequence(eng, model, 0, [(4, [1, 2, 3, 4]), (1, [40, 50, 60, 70]),
                                                (0, [8, 9, 10, 11])])
    finally:
        eng.close()


def _ulp_bf16(v):
    return 2.0 ** (np.floor(np.log2(np.abs(v))) - 7)


def test_fast_mode_teacher_forced_per_layer(c3):
    """Matrix-core mode, each layer on the oracle's input streams (the caches
    the exact tests above left equal to the oracle's): routing, per-layer
    relative L2, greedy tokens and GDN state against the bounds above; the
    elementwise ratio is reported only."""
    eng, model = c3
    slots = list(range(8))
    toks = list(model.next_tokens)
    eng.set_flags(exact=False)
    worst = {"elementwise": 0.0, "rel_l2": 0.0, "gap": 0.0, "token_gap": 0.0, "state": 0.0}
    flips = 0
    try:
        for step in range(2):
            want = model.decode_rows(slots, toks)
            h_in = np.stack(model.layer_in)
            got, h_out, ids = eng.decode_forced(slots, toks, h_in)
            for i in range(LAYERS):
                w = _bf(model.layer_in[i + 1])
                g = _bf(h_out[i])
                lg = _bf(model.last_router[i])
                ratios, rels = [], []
                for r in range(8):
                    mine, theirs = set(ids[i, r].tolist()), set(model.last_ids[i][r].tolist())
                    if mine != theirs:
                        flips += 1
                        tenth = model.last_ids[i][r][0]
                        diff = sorted(mine ^ theirs)
                        gap = np.abs(lg[r][diff] - lg[r][tenth]) / _ulp_bf16(lg[r][tenth])
                        print(f"step {step} layer {i} row {r}: routing differs in {diff}, "
                              f"router-logit gaps to the 10th {gap.tolist()} bf16 ulp", flush=True)
                        worst["gap"] = max(worst["gap"], float(gap.max()))
                        continue
                    err = np.abs(g[r] - w[r])
                    ratios.append(float((err / (2e-2 * np.abs(w[r]) + 1e-2)).max()))
                    rels.append(float(np.linalg.norm(g[r] - w[r]) / np.linalg.norm(w[r])))
                if ratios:
                    print(f"step {step} layer {i}: relative L2 up to {max(rels):.2e}, "
                          f"elementwise error / (2e-2|w| + 1e-2) up to {max(ratios):.1f}",
                          flush=True)
                    worst["elementwise"] = max(worst["elementwise"], max(ratios))
                    worst["rel_l2"] = max(worst["rel_l2"], max(rels))
            lg = _bf(model._qmv(model.head, model.last_mixed))
            for r in range(8):
                if got[r] != want[r]:
                    a, b = lg[r][got[r]], lg[r][want[r]]
                    gap = abs(a - b) / _ulp_bf16(max(abs(a), abs(b)))
                    print(f"step {step} row {r}: token {got[r]} vs {want[r]} "
                          f"(oracle logits {a} vs {b}, {gap} bf16 ulp apart)", flush=True)
                    worst["token_gap"] = max(worst["token_gap"], float(gap))
            n = 8 * model.n_gdn
            st = eng.read("cache.gdn_state", np.float32, model.state.shape)[:n].astype(np.float64)
            ref = model.state[:n].astype(np.float64)
            rel = max(float(np.linalg.norm(a - b) / np.linalg.norm(b)) for a, b in zip(st, ref))
            print(f"step {step}: GDN state relative Frobenius error up to {rel:.2e}, "
                  f"max abs error {np.abs(st - ref).max():.3e}", flush=True)
            worst["state"] = max(worst["state"], rel)
            toks = [int(t) for t in want]
    finally:
        eng.set_flags(exact=True)
    print("worst", worst, "routing flips", flips, flush=True)
    assert worst["gap"] <= 1.0
    assert worst["rel_l2"] <= 3e-2
    assert worst["token_gap"] <= 1.0
    assert worst["state"] <= 5e-2
