"""The equal-offset scheduler (mx_sched_*) on the CPU, over a mock model
whose greedy token is a hash of the slot's whole token history: the policy of
the reference's cooperative server loop (src/bin/server/batch.rs:240-349) and
prefix cache (src/speculative.rs:70-117), checked through properties that do
not restate the loop:
  * every job's tokens equal its greedy generation run alone;
  * every decode groups rows at one offset, at most batch_size of them, and a
    row at the smallest offset is never left out while others decode;
  * an identical prompt hits the cache (no prefill) and LRU / token-budget
    eviction drop the least recently used prompts;
  * stop tokens end a row unemitted, max_tokens ends it, over-long prompts are
    rejected, cancelled jobs never run."""
import numpy as np
import pytest

V = 997


def f(hist):
    h = 1469598103
    for t in hist:
        h = (h * 1099511 + int(t) + 7) % 2147483647
    return h % V


class Mock:
    def __init__(self, slots):
        self.hist = {s: [] for s in range(slots)}
        self.prefills, self.groups, self.clones = [], [], []

    def prefill(self, slot, toks):
        self.hist[slot] = list(toks)
        self.prefills.append(tuple(toks))
        return f(self.hist[slot])

    def decode(self, slots, toks):
        offs = {len(self.hist[s]) for s in slots}
        assert len(offs) == 1, "rows at different offsets decoded together"
        self.groups.append((tuple(slots), offs.pop()))
        out = []
        for s, t in zip(slots, toks):
            self.hist[s].append(int(t))
            out.append(f(self.hist[s]))
        return out

    def clone(self, src, dst):
        self.clones.append((src, dst))
        self.hist[dst] = list(self.hist[src])


def solo(prompt, max_tokens, stop=()):
    hist, out = list(prompt), []
    while True:
        t = f(hist)
        if t in stop:
            return out, "stop"
        out.append(t)
        if len(out) == max_tokens:
            return out, "length"
        hist.append(t)


def run(mx, jobs, batch=4, slots=12, max_context=64, stop=(), entries=4, budget=200,
        arrivals=None, cancel=()):
    m = Mock(slots)
    sc = mx.Scheduler(batch, slots, max_context, entries, budget, stop, prefill=m.prefill,
                      decode=m.decode, clone=m.clone)
    arrivals = arrivals or {0: list(jobs)}
    toks = {j: [] for j in jobs}
    end = {}
    first_hit = {}
    step = 0
    while step in arrivals or sc.pending() or any(k > step for k in arrivals):
        for j in arrivals.get(step, []):
            sc.submit(j, jobs[j][0], jobs[j][1])
        for j in cancel if step == 0 else ():
            assert sc.cancel(j)
        ev, rows = sc.step()
        assert rows <= batch
        for job, tok, kind, detail in ev:
            if kind == mx.SCHED_TOKEN:
                if not toks[job]:
                    first_hit[job] = detail
                toks[job].append(tok)
            else:
                assert job not in end
                end[job] = (kind, tok, detail)
        step += 1
        assert step < 10000
    sc.close()
    return m, toks, end, first_hit


def test_jobs_match_solo_generation_and_group_by_offset(mx):
    rng = np.random.default_rng(1)
    jobs = {j: (list(rng.integers(0, V, int(rng.integers(1, 20)))), int(rng.integers(1, 12)))
            for j in range(9)}
    m, toks, end, _ = run(mx, jobs, batch=4)
    for j, (p, mt) in jobs.items():
        want, why = solo(p, mt)
        assert toks[j] == want, j
        assert end[j][0] == mx.SCHED_LENGTH
    assert max(len(g[0]) for g in m.groups) <= 4
    assert any(len(g[0]) > 1 for g in m.groups)  # rows did catch up and share steps


def test_smallest_offset_first(mx):
    # three rows with prompt lengths 3, 5, 9: the shortest decodes alone until it
    # reaches 5, then the two share steps until 9, then all three
    jobs = {0: ([1, 2, 3], 10), 1: ([4, 5, 6, 7, 8], 10), 2: (list(range(9)), 10)}
    m, toks, end, _ = run(mx, jobs, batch=4)
    offsets = [o for _, o in m.groups]
    sizes = [len(s) for s, _ in m.groups]
    assert offsets[:2] == [3, 4] and sizes[:2] == [1, 1]
    assert offsets[2:6] == [5, 6, 7, 8] and sizes[2:6] == [2, 2, 2, 2]
    assert sizes[6] == 3 and offsets[6] == 9
    assert offsets == sorted(offsets)


def test_prefix_cache_hits_and_lru(mx):
    A, B, Cp = [5] * 6, [6] * 7, [7] * 8
    jobs = {0: (A, 2), 1: (B, 2), 2: (Cp, 2), 3: (A, 2), 4: (Cp, 2)}
    # entries = 2: A, B cached, then C evicts A; A misses again, C hits
    m, toks, end, hit = run(mx, jobs, batch=1, slots=4, entries=2, budget=100,
                            arrivals={0: [0], 5: [1], 10: [2], 15: [3], 20: [4]})
    assert m.prefills.count(tuple(A)) == 2 and m.prefills.count(tuple(Cp)) == 1
    assert hit == {0: 0, 1: 0, 2: 0, 3: 0, 4: 1}
    for j, (p, mt) in jobs.items():
        assert toks[j] == solo(p, mt)[0]
    # a token budget smaller than the prompt: never cached
    m, toks, end, hit = run(mx, {0: (A, 2), 1: (A, 2)}, batch=1, slots=4, entries=2, budget=5,
                            arrivals={0: [0], 5: [1]})
    assert m.prefills.count(tuple(A)) == 2 and hit[1] == 0


def test_stop_length_reject_cancel(mx):
    p = [3, 1, 4, 1, 5]
    gen, _ = solo(p, 50)
    stop = (gen[3],)
    jobs = {0: (p, 50), 1: (p, 2), 2: (list(range(60)), 10), 3: ([9, 9], 5), 4: ([], 3)}
    m, toks, end, _ = run(mx, jobs, batch=2, stop=stop, entries=0, cancel=[3])
    want, why = solo(p, 50, stop)
    assert toks[0] == want and why == "stop" and end[0][:2] == (mx.SCHED_STOP, stop[0])
    assert stop[0] not in toks[0]
    assert toks[1] == solo(p, 2, stop)[0] and end[1][0] == mx.SCHED_LENGTH
    assert end[2][0] == mx.SCHED_ERROR and toks[2] == []  # 60 + 10 > max_context 64
    assert end[4][0] == mx.SCHED_ERROR  # empty prompt
    assert 3 not in end and toks[3] == []  # cancelled while queued


def test_decode_failure_reports_error(mx):
    def bad_decode(slots, toks):
        raise RuntimeError("device lost")

    m = Mock(4)
    sc = mx.Scheduler(2, 4, 64, prefill=m.prefill, decode=bad_decode, clone=m.clone)
    sc.submit(7, [1, 2, 3], 5)
    ev, _ = sc.step()
    kinds = [e[2] for e in ev if e[0] == 7]
    assert kinds[0] == mx.SCHED_TOKEN and kinds[-1] == mx.SCHED_ERROR
    assert sc.pending() == 0
    sc.close()
