"""The MTP draft layer and speculative generation (config 4's draft model and
acceptance loop: Mtp::forward, src/mtp.rs:72-127; generate_prepared,
src/speculative.rs:225-483) on the tiny model with mtp = 1, at config 3's
geometry (four layers, mixed widths, a 16-token vocabulary slice: bit-exact
with the oracle, drafts accepted) and over the whole 48-layer config-4 model
(lossless against plain greedy decoding).  The oracle's draft step itself is
pinned on the CPU by a float64 closed form and a reduction to a trunk layer
(tests/test_oracle_mtp.py).

Exact mode: the tokens, every round's draft tokens and the acceptance counts
are bit-exact with the CPU oracle model running the same loop, and
speculation is lossless (the tokens equal plain greedy decoding's).  With a
16-token vocabulary the draft layer's guesses are accepted now and then, so
the accept / commit / resynchronise paths with accepted > 0 run too.
Fast mode: the loop runs end to end on the matrix-core kernels; a fast verify
block gives every position the bits of a one-token fast decode step, so the
fast loop's tokens are checked against plain fast greedy decoding token for
token (test_fast_speculation_is_lossless)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


# (vocab, mixed widths, depth, seed): seed 60 draws every width in both roles;
# with 16 tokens, seed 6 (prompt drawn from the same seed) accepts 5-6 drafts
# in 9-10 rounds at depths 2, 3 and 7
@pytest.mark.parametrize("vocab,mixed,depth,seed", [(1024, 0, 3, 77), (1024, 1, 1, 60),
                                                    (16, 0, 3, 6), (16, 0, 7, 6), (16, 0, 2, 6),
                                                    (16, 1, 3, 60)])
def test_exact_speculation_matches_oracle_and_plain_greedy(mx, vocab, mixed, depth, seed):
    from oracle.model import Model

    cfg = dict(mx.TINY, mtp=1, vocab=vocab, mixed_bits=mixed, seed=seed)
    eng = mx.Engine(cfg)
    try:
        eng.set_flags(exact=True)
        model = Model(cfg, lambda name, dtype, shape: eng.read(name, dtype, shape))
        prompt = [int(t) for t in np.random.default_rng(seed).integers(0, vocab, 19)]
        toks, st = eng.generate(1, prompt, 16, depth)
        want, wst = model.generate(1, prompt, 16, depth)
        assert [int(t) for t in toks] == want
        assert [int(d) for d in st["drafts"]] == wst["drafts"]
        assert (st["rounds"], st["drafted"], st["accepted"]) == \
            (wst["rounds"], wst["drafted"], wst["accepted"])
        plain, pst = eng.generate(2, prompt, 16, 0)
        assert [int(t) for t in plain] == [int(t) for t in toks]
        assert pst["rounds"] == 0
        if seed == 6:
            assert st["accepted"] > 0, st  # the accept path ran
    finally:
        eng.close()


def test_generate_rejects_bad_requests(mx):
    cfg = dict(mx.TINY, mtp=0)
    eng = mx.Engine(cfg)
    try:
        with pytest.raises(Exception):
            eng.generate(0, [1, 2, 3], 4, 3)  # no draft layer
        eng.generate(0, [1, 2, 3], 2, 0)
        with pytest.raises(Exception):
            eng.generate(0, [1, 2, 3], 2, 0)  # the slot is no longer empty
    finally:
        eng.close()


MID = dict(hidden=512, layers=4, attn_every=4, vocab=4096, hc=4, hc_rank=256, gdn_hk=2, gdn_hv=4,
           gdn_dk=128, gdn_dv=128, conv_k=4, heads=4, kv_heads=1, head_dim=128, rotary_dim=32,
           rope_theta=1e7, rms_eps=1e-6, experts=64, top_k=4, moe_inter=512, shared_inter=512,
           bits=4, down_bits=5, embed_bits=8, head_bits=8, group_size=64, mixed_bits=0,
           max_slots=4, max_context=128, max_verify=8, seed=4242, mtp=1)


@pytest.mark.parametrize("vocab,depth", [(4096, 3), (16, 1), (16, 3), (16, 7)])
def test_fast_speculation_is_lossless(mx, vocab, depth):
    """Fast mode (matrix-core projections, fast GDN step): speculative
    generation gives plain greedy decoding's tokens.  A verify block's tokens
    take the arithmetic of one-token decode steps in every layer, so greedy
    acceptance loses nothing; with a 16-token vocabulary drafts are accepted
    and the commit / rollback paths run."""
    eng = mx.Engine(dict(MID, vocab=vocab))
    try:
        eng.set_flags(exact=False)
        prompt = [int(t) for t in np.random.default_rng(3).integers(0, vocab, 21)]
        toks, st = eng.generate(0, prompt, 24, depth)
        assert len(toks) == 24 and all(0 <= int(t) < vocab for t in toks)
        assert st["rounds"] >= 1 and st["drafted"] == len(st["drafts"])
        assert 0 <= st["accepted"] <= st["drafted"]
        plain, _ = eng.generate(1, prompt, 24, 0)
        assert [int(t) for t in plain] == [int(t) for t in toks]
        if vocab == 16:
            assert st["accepted"] > 0, st
    finally:
        eng.close()


def test_verify_profile_and_draft_bytes(mx):
    """The measurement hooks of the config-4 bench line: a profiled verify
    block predicts what an unprofiled one does, a one-token profiled verify
    counts the bytes of a one-row profiled decode step on the same state and
    routing (weights, routed experts, embedding row, state read + one state
    write, KV), and a draft step's bytes grow by one KV position per
    position."""
    cfg = dict(mx.TINY, mtp=1, seed=5)
    eng = mx.Engine(cfg)
    try:
        eng.set_flags(exact=True)
        prompt = [int(t) for t in np.random.default_rng(5).integers(0, cfg["vocab"], 21)]
        nxt = eng.prefill(0, prompt)
        eng.clone(0, 1)
        eng.clone(0, 2)
        block = [nxt, 3, 7, 11]
        want = eng.verify(0, block)
        eng.commit(0, 2)
        got, prof = eng.profile_verify(1, block)
        eng.commit(1, 2)
        assert [int(t) for t in got] == [int(t) for t in want]
        assert prof["layers"] == cfg["layers"] and prof["step_bytes"] > 0
        assert prof["distinct_experts"] <= cfg["layers"] * min(len(block) * cfg["top_k"],
                                                              cfg["experts"])
        assert eng.offset(0) == eng.offset(1) == len(prompt) + 2
        # one token: the verify block's bytes equal a decode step's
        _, one = eng.profile_verify(2, [nxt])
        eng.commit(2, 1)
        eng.reset(2)
        nxt2 = eng.prefill(2, prompt)
        assert nxt2 == nxt
        _, step = eng.profile_step([2], [nxt])
        assert step["distinct_experts"] == one["distinct_experts"]
        assert step["step_bytes"] == pytest.approx(one["step_bytes"], rel=1e-12)
        # draft steps: the KV term grows by kv_heads * head_dim * 2 tensors * 2 B
        # per position
        d0, d1 = eng.draft_bytes(100), eng.draft_bytes(150)
        assert d1 - d0 == pytest.approx(50 * cfg["kv_heads"] * cfg["head_dim"] * 4, rel=1e-12)
        assert 0 < d0 < prof["step_bytes"]
    finally:
        eng.close()


def test_exact_speculation_at_config3_geometry_matches_oracle(mx):
    """Config 4 at config 3's geometry (hidden 2048, 512 experts top-10,
    hc 4 / rank 256, GDN 16/32 heads, attention 16/2 heads of 256) with the
    mixed per-layer widths and the MTP draft layer, four layers and a
    16-token vocabulary slice so that drafts are accepted now and then: the
    exact engine's speculative generation (prompt prefill with the drafter's
    prefill, drafts, 4-token verify blocks, greedy acceptance, commit,
    resynchronisation) equals the oracle model's bit for bit -- tokens, every
    draft, rounds and accepted counts -- and plain greedy decoding's tokens."""
    from oracle.model import Model

    cfg = dict(mx.CONFIG3, layers=4, vocab=16, mtp=1, mixed_bits=1, max_slots=3, max_context=96)
    eng = mx.Engine(cfg)
    try:
        eng.set_flags(exact=True)
        chosen = None
        for seed in range(12):  # the engine alone finds a prompt with accepted drafts
            prompt = [int(t) for t in np.random.default_rng(100 + seed).integers(0, 16, 17)]
            eng.reset(0)
            toks, st = eng.generate(0, prompt, 24, 3)
            if st["accepted"] > 0:
                chosen = (prompt, toks, st)
                break
        assert chosen is not None, "no accepted draft in 12 prompts"
        prompt, toks, st = chosen
        print(f"prompt seed {100 + seed}: rounds {st['rounds']}, accepted "
              f"{st['accepted']}/{st['drafted']}", flush=True)
        model = Model(cfg, lambda name, dtype, shape: eng.read(name, dtype, shape))
        want, wst = model.generate(0, prompt, 24, 3)
        assert [int(t) for t in toks] == want
        assert [int(d) for d in st["drafts"]] == wst["drafts"]
        assert (st["rounds"], st["drafted"], st["accepted"]) == \
            (wst["rounds"], wst["drafted"], wst["accepted"])
        plain, pst = eng.generate(1, prompt, 24, 0)
        assert [int(t) for t in plain] == [int(t) for t in toks] and pst["rounds"] == 0
    finally:
        eng.close()


def test_exact_speculation_over_all_48_layers_is_lossless(mx):
    """The whole config-4 model (48 mixed-width layers, vocabulary 151936,
    the MTP draft layer): speculative generation of 40 tokens in depth-3
    rounds gives plain greedy decoding's tokens, over at least 8 rounds."""
    cfg = dict(mx.CONFIG3, mtp=1, mixed_bits=1, max_slots=2, max_context=160)
    eng = mx.Engine(cfg)
    try:
        eng.set_flags(exact=True)
        prompt = [int(t) for t in np.random.default_rng(44).integers(0, cfg["vocab"], 41)]
        toks, st = eng.generate(0, prompt, 40, 3)
        plain, _ = eng.generate(1, prompt, 40, 0)
        print(f"48 layers: rounds {st['rounds']}, accepted {st['accepted']}/{st['drafted']}",
              flush=True)
        assert len(toks) == 40 and st["rounds"] >= 8
        assert [int(t) for t in toks] == [int(t) for t in plain]
    finally:
        eng.close()
