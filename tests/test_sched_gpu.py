"""The scheduler over the real decode engine (exact mode, tiny model): every
job's tokens equal the tokens of that job decoded alone through the engine,
with equal-offset groups of up to 4 rows, prefix-cache hits served by a slot
copy, and a stop token ending a row (the reference's cooperative server loop,
src/bin/server/batch.rs:240-349, with its batch-parity property)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def alone(eng, slot, prompt, max_tokens, stop=()):
    eng.reset(slot)
    t = eng.prefill(slot, prompt)
    out = []
    while True:
        if t in stop:
            return out
        out.append(int(t))
        if len(out) == max_tokens:
            return out
        t = int(eng.decode_batch([slot], [t])[0])


def test_scheduler_matches_solo_decode(mx):
    cfg = dict(mx.TINY, max_slots=12)  # 4 rows + prefix entries + one solo slot
    eng = mx.Engine(cfg)
    try:
        eng.set_flags(exact=True)
        rng = np.random.default_rng(11)
        prompts = [list(rng.integers(0, cfg["vocab"], int(n))) for n in (3, 9, 5, 9, 12, 3)]
        prompts.append(list(prompts[1]))  # identical prompt: a prefix-cache hit
        maxes = [6, 4, 8, 5, 3, 7, 4]
        solo_slot = cfg["max_slots"] - 1
        want = [alone(eng, solo_slot, p, m) for p, m in zip(prompts, maxes)]
        # a stop token taken from job 2's own output ends it early
        stop = (want[2][3],)
        want = [alone(eng, solo_slot, p, m, stop) for p, m in zip(prompts, maxes)]
        sc = mx.Scheduler(4, cfg["max_slots"] - 1, cfg["max_context"], prefix_entries=8,
                          prefix_tokens=200, stop=stop, engine=eng)
        for j, (p, m) in enumerate(zip(prompts, maxes)):
            sc.submit(j, p, m)
        got = {j: [] for j in range(len(prompts))}
        ends, hits, groups = {}, {}, []
        for _ in range(200):
            if not sc.pending():
                break
            ev, rows = sc.step()
            groups.append(rows)
            for job, tok, kind, detail in ev:
                if kind == mx.SCHED_TOKEN:
                    if not got[job]:
                        hits[job] = detail
                    got[job].append(int(tok))
                else:
                    ends[job] = kind
        sc.close()
        assert sc.h is None
        for j in range(len(prompts)):
            assert got[j] == want[j], (j, got[j], want[j])
        assert ends[2] == mx.SCHED_STOP
        assert hits[6] == 1 and hits[1] == 0
        assert max(groups) > 1 and max(groups) <= 4
    finally:
        eng.close()
