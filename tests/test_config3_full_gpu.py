"""The whole config-3 model (48 layers [G, G, G, A] x 12, hidden 2048, 512
experts top-10, vocabulary 151936) in both modes -- the exact fixed-order
kernels and the benched matrix-core kernels:
  * batch invariance (reference batch-parity.rs:126-171, error 0): eight
    rows decoded together at their own offsets give, row for row, the tokens
    and hidden streams of the same rows decoded one at a time from copies of
    their caches;
  * verify invariance with rollback (verify-parity.rs:90-195,
    rollback-parity.rs; config 4): at a context of 4093 positions with
    config 4's mixed per-layer widths, a 4-token verify block committed with
    keep k leaves the GDN state, conv windows and KV of k sequential decode
    steps, bit for bit, its per-position argmax equals those steps' tokens,
    and the next step agrees.
Contexts are synthetic (mx_engine_fill_slot: random KV, state and conv
window), which the decode arithmetic cannot tell from a prefill."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CONTEXTS = [1581, 900, 543, 678, 47, 868, 1478, 406]  # bench.py's ragged prompt lengths


@pytest.fixture(scope="module")
def full(mx):
    cfg = dict(mx.CONFIG3, max_slots=16, max_context=2100)
    eng = mx.Engine(cfg)
    yield eng, cfg
    eng.close()


@pytest.mark.parametrize("exact", [True, False])
def test_batch8_equals_singleton_rows(full, exact):
    eng, cfg = full
    eng.set_flags(exact=exact)
    HS = cfg["hc"] * cfg["hidden"]
    for s, n in enumerate(CONTEXTS):
        eng.fill_slot(s, n, seed=500 + s)
        eng.clone(s, s + 8)
    toks = [int(t) for t in np.random.default_rng(5).integers(0, cfg["vocab"], 8)]
    for step in range(2):
        got = eng.decode_batch(list(range(8)), toks, equal=False)
        hid = eng.read("hidden", np.uint16, (8, HS))
        for r in range(8):
            one = eng.decode_batch([r + 8], [toks[r]])
            h1 = eng.read("hidden", np.uint16, (1, HS))
            assert one[0] == got[r], (exact, step, r)
            assert (h1[0] == hid[r]).all(), (exact, step, r)
        print(f"exact={exact} step {step}: tokens {list(got)}", flush=True)
        toks = [int(t) for t in got]
    eng.set_flags(exact=True)


def _slot_caches(eng, cfg, n_gdn, n_attn, slot, upto):
    """(GDN state, conv window, keys and values of positions < upto) of a slot."""
    sp = cfg["gdn_hv"] * cfg["gdn_dk"] * cfg["gdn_dv"]
    cd = 2 * cfg["gdn_hk"] * cfg["gdn_dk"] + cfg["gdn_hv"] * cfg["gdn_dv"]
    cp = (cfg["conv_k"] - 1) * cd
    S = slot + 1
    st = eng.read("cache.gdn_state", np.float32, (S, n_gdn * sp))[slot]
    cv = eng.read("cache.conv_state", np.uint16, (S, n_gdn * cp))[slot]
    plane = (n_attn, cfg["kv_heads"], cfg["max_context"], cfg["head_dim"])
    k = eng.read("cache.k", np.uint16, (S,) + plane)[slot][:, :, :upto]
    v = eng.read("cache.v", np.uint16, (S,) + plane)[slot][:, :, :upto]
    return st, cv, k, v


@pytest.mark.parametrize("exact", [True, False])
def test_verify_commit_equals_sequential_steps_mixed_widths(mx, exact):
    cfg = dict(mx.CONFIG3, mixed_bits=1, seed=60, max_slots=4, max_context=4104)
    eng = mx.Engine(cfg)
    try:
        eng.set_flags(exact=exact)
        n_gdn = sum(1 for i in range(cfg["layers"]) if i % 4 != 3)
        n_attn = cfg["layers"] - n_gdn
        HS = cfg["hc"] * cfg["hidden"]
        eng.fill_slot(0, 4093, seed=77)
        block = [int(t) for t in np.random.default_rng(9).integers(0, cfg["vocab"], 4)]
        for keep in (4, 2, 1, 0):
            eng.clone(0, 1)
            eng.clone(0, 2)
            pred = eng.verify(1, block)
            eng.commit(1, keep)
            seq = [int(eng.decode_batch([2], [block[i]])[0]) for i in range(keep)]
            assert [int(p) for p in pred[:keep]] == seq, (exact, keep)
            assert eng.offset(1) == eng.offset(2) == 4093 + keep
            a = _slot_caches(eng, cfg, n_gdn, n_attn, 1, 4093 + keep)
            b = _slot_caches(eng, cfg, n_gdn, n_attn, 2, 4093 + keep)
            for name, x, y in zip(("state", "conv", "keys", "values"), a, b):
                assert (x == y).all(), (exact, keep, name)
            t = 17 + keep
            n1 = eng.decode_batch([1], [t])
            h1 = eng.read("hidden", np.uint16, (1, HS))
            n2 = eng.decode_batch([2], [t])
            h2 = eng.read("hidden", np.uint16, (1, HS))
            assert n1[0] == n2[0] and (h1 == h2).all(), (exact, keep)
            print(f"exact={exact} keep {keep}: verify argmax {list(pred)}, next {n1[0]}",
                  flush=True)
    finally:
        eng.close()
