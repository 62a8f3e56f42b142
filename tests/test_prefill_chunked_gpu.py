"""Chunked prefill (mx_engine_prefill_chunked: 512-token chunks whose
projections and experts run as 16-row matrix-core tiles) against the
block prefill (mx_engine_prefill, eight tokens per step).

A chunk of at most eight tokens takes the same kernels as a matrix-core block
step, so it must agree with one bit for bit.  Longer chunks change only the
fp32 summation order of the projections (16-row tiles instead of the
eight-row kernels), so the caches and the next step's hidden state agree with
the block prefill within the north star's tolerance; a wiring mistake (a row
or route served by the wrong tile, a misplaced chunk boundary) moves them by
O(1)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def bf(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


@pytest.fixture(scope="module")
def tiny(mx):
    cfg = dict(mx.TINY)
    eng = mx.Engine(cfg)
    yield eng, cfg
    eng.close()


def dims(cfg):
    n_attn = cfg["layers"] // cfg["attn_every"]
    n_gdn = cfg["layers"] - n_attn
    cd = 2 * cfg["gdn_hk"] * cfg["gdn_dk"] + cfg["gdn_hv"] * cfg["gdn_dv"]
    sp = cfg["gdn_hv"] * cfg["gdn_dk"] * cfg["gdn_dv"]
    return n_gdn, n_attn, cd, sp


def caches(eng, cfg, slot, length):
    """The slot's GDN states, conv windows and its first `length` K / V rows."""
    n_gdn, n_attn, cd, sp = dims(cfg)
    S = cfg["max_slots"]
    st = eng.read("cache.gdn_state", np.float32, (S, n_gdn, sp))[slot].astype(np.float64)
    cv = bf(eng.read("cache.conv_state", np.uint16, (S, n_gdn, cfg["conv_k"] - 1, cd))[slot])
    shape = (S, n_attn, cfg["kv_heads"], cfg["max_context"], cfg["head_dim"])
    k = bf(eng.read("cache.k", np.uint16, shape)[slot, :, :, :length])
    v = bf(eng.read("cache.v", np.uint16, shape)[slot, :, :, :length])
    return st, cv, k, v


def rel(a, b):
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def prefill(eng, slot, prompt, exact, chunked):
    eng.reset(slot)
    eng.set_flags(exact=exact)
    return eng.prefill(slot, prompt, chunked=chunked)


@pytest.mark.parametrize("n", [1, 5, 8])
def test_short_chunk_equals_matrix_core_block(tiny, n):
    eng, cfg = tiny
    prompt = np.random.default_rng(n).integers(0, cfg["vocab"], n)
    a = prefill(eng, 0, prompt, exact=False, chunked=False)
    b = prefill(eng, 1, prompt, exact=False, chunked=True)
    assert a == b
    assert eng.offset(0) == eng.offset(1) == n
    for x, y in zip(caches(eng, cfg, 0, n), caches(eng, cfg, 1, n)):
        assert np.array_equal(x, y)


@pytest.mark.parametrize("n", [560, 128, 9])
def test_chunked_prefill_within_tolerance_of_block_prefill(tiny, n):
    """n = 560: a full chunk and one of 48 tokens; 128: one partial chunk;
    9: the smallest chunk beyond the eight-row kernels."""
    eng, cfg = tiny
    prompt = np.random.default_rng(100 + n).integers(0, cfg["vocab"], n)
    ex = prefill(eng, 0, prompt, exact=True, chunked=False)
    fa = prefill(eng, 1, prompt, exact=False, chunked=False)
    ch = prefill(eng, 2, prompt, exact=False, chunked=True)
    assert eng.offset(2) == n
    exact, fast, got = (caches(eng, cfg, s, n) for s in (0, 1, 2))
    # the block prefill on the matrix cores sets the scale of summation-order
    # differences: the chunked one is as close to the exact prefill as it is
    base = [rel(f, e) for f, e in zip(fast, exact)]
    for name, want in (("exact", exact), ("fast blocks", fast)):
        errs = [rel(g, w) for g, w in zip(got, want)]
        print(f"n={n} chunked vs {name}: state {errs[0]:.2e} conv {errs[1]:.2e} "
              f"k {errs[2]:.2e} v {errs[3]:.2e} (fast blocks vs exact: "
              f"{' '.join(f'{b:.2e}' for b in base)})", flush=True)
        # (a small floor: the conv window is the last three tokens' inputs, a
        # sample small enough to agree by chance in one comparison)
        assert all(e <= 2.0 * b + 1e-2 for e, b in zip(errs, base)), (errs, base)
        assert max(errs) <= 5e-2, errs
    # the next step from each slot (same token, matrix-core mode): hidden
    # states within the north star's elementwise bf16 tolerance
    eng.set_flags(exact=False)
    tok = int(prompt[-1])
    eng.decode_batch([0, 1, 2], [tok, tok, tok], equal=False)
    hid = bf(eng.read("hidden", np.uint16, (3, cfg["hc"] * cfg["hidden"])))
    for r in (0, 1):
        err = np.abs(hid[2] - hid[r])
        bound = 1e-2 * np.abs(hid[r]).max() + 2e-2 * np.abs(hid[r])
        print(f"n={n} hidden vs slot {r}: max err {err.max():.3e}, worst ratio "
              f"{(err / bound).max():.3f}", flush=True)
        assert np.all(err <= bound)
    print(f"n={n} next tokens: exact {ex}, fast blocks {fa}, chunked {ch}", flush=True)


def test_chunked_prefill_then_exact_decode_and_rejections(mx, tiny):
    """Decode after a chunked prefill continues from the chunked caches at the
    right offset; a prompt past the slot's context is refused before any
    launch (the slot stays usable)."""
    eng, cfg = tiny
    prompt = np.random.default_rng(7).integers(0, cfg["vocab"], 150)
    prefill(eng, 3, prompt, exact=True, chunked=True)
    eng.set_flags(exact=True)
    eng.decode_batch([3], [int(prompt[-1])])
    assert eng.offset(3) == 151
    too_long = np.zeros(cfg["max_context"] - 151 + 1, np.uint32)
    with pytest.raises(mx.MxError):
        eng.prefill(3, too_long, chunked=True)
    assert eng.offset(3) == 151
    assert eng.slot_failed(3) == 0


def test_generate_with_chunked_prompt_and_drafter_pass(mx):
    """mx_engine_generate with flag bit 10: the prompt is prefilled in chunks
    and the draft layer's prompt pass runs chunk by chunk.  Speculation stays
    lossless (depth 3 gives plain greedy decoding's tokens from the same
    chunked prompt, drafts accepted now and then with a 16-token vocabulary),
    and the draft layer's KV rows over the prompt agree with the block
    prefill's within the block prefill's own tolerance."""
    cfg = dict(mx.TINY, mtp=1, vocab=16, seed=6)
    eng = mx.Engine(cfg)
    try:
        prompt = [int(t) for t in np.random.default_rng(6).integers(0, 16, 560)]
        out = {}
        for chunked in (False, True):
            for depth in (0, 3):
                eng.reset(0)
                eng.set_flags(exact=True, chunked_generate=chunked)
                toks, st = eng.generate(0, prompt, 16, depth)
                out[chunked, depth] = (toks, st)
            # the draft layer's K / V plane (after the model's attention layers)
            n_gdn, n_attn, _, _ = dims(cfg)
            shape = (cfg["max_slots"], n_attn + 1, cfg["kv_heads"], cfg["max_context"],
                     cfg["head_dim"])
            out[chunked, "kv"] = [bf(eng.read(name, np.uint16, shape)[0, n_attn, :, :560])
                                  for name in ("cache.k", "cache.v")]
        for chunked in (False, True):
            assert np.array_equal(out[chunked, 0][0], out[chunked, 3][0]), chunked
        print(f"chunked prompt: {out[True, 3][1]}; blocks: {out[False, 3][1]}", flush=True)
        for g, w in zip(out[True, "kv"], out[False, "kv"]):
            assert rel(g, w) <= 5e-2, rel(g, w)
    finally:
        eng.close()


def test_chunked_prefill_refuses_unsupported_models_before_any_launch(mx):
    """A model the chunk kernels do not cover (1024 experts: the chunk's expert
    lists hold at most 1023) is refused with MX_EUNSUPPORTED before any
    launch: the slot is not marked failed, its offset does not move, and the
    block prefill still serves it."""
    cfg = dict(mx.TINY, experts=1024, max_slots=2)
    eng = mx.Engine(cfg)
    try:
        prompt = np.random.default_rng(3).integers(0, cfg["vocab"], 40)
        with pytest.raises(mx.MxError) as exc:
            eng.prefill(0, prompt, chunked=True)
        assert exc.value.code == mx.MX_EUNSUPPORTED
        assert eng.offset(0) == 0 and eng.slot_failed(0) == 0
        eng.prefill(0, prompt)
        assert eng.offset(0) == 40
    finally:
        eng.close()


def test_chunked_prefill_continues_an_existing_context(tiny):
    """A chunked prefill after 100 positions of block prefill (a prefix reused,
    then the rest of the prompt): the chunk reads the slot's cached conv
    window, GDN state and K/V, and its queries attend to the earlier
    positions.  The caches agree with a whole-prompt block prefill as closely
    as the matrix-core block prefill does."""
    eng, cfg = tiny
    prompt = np.random.default_rng(41).integers(0, cfg["vocab"], 400)
    prefill(eng, 0, prompt, exact=True, chunked=False)
    prefill(eng, 1, prompt, exact=False, chunked=False)
    prefill(eng, 2, prompt[:100], exact=True, chunked=False)
    eng.set_flags(exact=False)
    eng.prefill(2, prompt[100:], chunked=True)
    assert eng.offset(2) == 400
    exact, fast, got = (caches(eng, cfg, s, 400) for s in (0, 1, 2))
    base = [rel(f, e) for f, e in zip(fast, exact)]
    errs = [rel(g, e) for g, e in zip(got, exact)]
    print(f"continued chunk vs exact: {errs}; fast blocks vs exact: {base}", flush=True)
    assert all(e <= 2.0 * b + 1e-2 for e, b in zip(errs, base)), (errs, base)
