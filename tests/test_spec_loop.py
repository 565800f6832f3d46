"""The speculative loop on the device (hearth_gpu_spec_greedy, hearth_gpu_spec_sample), on the CPU.

- The device drafter's formulation (k_loop_draft: the largest end e among those with the
  most trailing tokens equal to the sequence's suffix, capped at ngram_n) proposes what
  the reference's NgramIndex proposes (generate.py:150-186), on every sequence over small
  alphabets, at every length, n-gram order and draft length.
- generate() on an engine that runs batches of steps (LoopToy.spec_greedy restates the
  loop: fixed-width steps with padding rows that the acceptance cannot walk into, the
  stop and length rules per token, the position it leaves) yields what the host loop
  yields: the same tokens, Token fields, GenStats counts and KV, with stops, budgets and
  capacities that end a batch in its middle.
"""
from __future__ import annotations

import itertools

import numpy as np
import pytest

import oracle_py as O
from hearth_amd.engine import chain_uniforms
from hearth_amd.generate import NgramIndex, Sampler, generate, generate_ids
from test_generate import PROMPTS, REPEAT, ToyEngine


def scan_propose(seq, max_n, k):
    """k_loop_draft's proposal: for each end e in [1, len - 1], m(e) = the number of
    tokens before e that equal the sequence's last tokens (at most max_n); the largest e
    of the largest m(e) > 0 gives seq[e : e + k]."""
    n = len(seq)
    best = (0, 0)
    for e in range(1, n):
        m = 0
        while m < max_n and m < e and seq[e - 1 - m] == seq[n - 1 - m]:
            m += 1
        if m and (m, e) > best:
            best = (m, e)
    if not best[0] or k <= 0:
        return []
    return list(seq[best[1]:best[1] + k])


def test_scan_proposes_what_the_index_proposes():
    rng = np.random.default_rng(5)
    checked = nonempty = 0
    for alpha in (1, 2, 3, 5):
        for _ in range(60):
            seq = [int(t) for t in rng.integers(0, alpha, int(rng.integers(1, 40)))]
            for max_n in (1, 2, 3, 5):
                idx = NgramIndex(max_n)
                for i, t in enumerate(seq):
                    idx.append(t)
                    for k in (0, 1, 4, 9):
                        want = idx.propose(k)
                        assert scan_propose(seq[:i + 1], max_n, k) == want, (seq[:i + 1], max_n, k)
                        checked += 1
                        nonempty += bool(want)
    # exhaustive over short binary and ternary sequences
    for alpha, length in ((2, 10), (3, 7)):
        for seq in itertools.product(range(alpha), repeat=length):
            for max_n in (1, 3):
                assert scan_propose(seq, max_n, 3) == NgramIndex(max_n, seq).propose(3), (seq, max_n)
    assert checked > 10000 and nonempty > checked // 3


class LoopToy(ToyEngine):
    """ToyEngine with the device loop: spec_greedy restates hearth_gpu_spec_greedy."""
    spec_loop_ok = True

    def __init__(self, *a, **kw):
        super().__init__(*a, **kw)
        self.batches = 0
        self.padded_rows = 0

    def spec_greedy(self, seq, new_tokens, max_new, draft_len, ngram_n, stop_ids=(), max_steps=64):
        def accept(rows, cmp, nd, hist):
            T = len(cmp)
            return O.accept_tree(rows, np.asarray(cmp, np.int32), np.arange(-1, T - 1), mode=0)

        return self._steps(seq, new_tokens, max_new, draft_len, ngram_n, stop_ids, max_steps, accept)

    def _steps(self, seq, new_tokens, max_new, draft_len, ngram_n, stop_ids, max_steps, accept):
        seq = [int(t) for t in seq]
        assert self.pos == len(seq) - 1 and 0 <= new_tokens < max_new
        T = draft_len + 1
        steps_fit = min(max_steps, (self.kv_capacity - self.pos) // T)
        if steps_fit < 1:
            return None
        self.batches += 1
        stops = {int(s) for s in stop_ids}
        hist, nw, finish, stop_id, steps = list(seq), new_tokens, None, 0, []
        for _ in range(steps_fit):
            nmax = min(T - 1, max_new - nw - 1)
            draft = scan_propose(hist, ngram_n, nmax) if draft_len and ngram_n else []
            nd, last = len(draft), hist[-1]
            self.padded_rows += T - 1 - nd
            rows_tokens = [last] + draft + [last] * (T - 1 - nd)      # padding: a valid id for the forward
            cmp = [last] + draft + [-1] * (T - 1 - nd)                 # padding: no argmax equals -1
            pos0 = self.pos
            rows = self.eval(rows_tokens, all_logits=True)
            rc, path, fin = accept(rows, cmp, nd, hist)
            if rc != 0:
                del self.kv[pos0:]
                finish = "bad_logits"
                break
            assert path == list(range(len(path))) and len(path) <= nd + 1
            del self.kv[pos0 + len(path):]
            nacc, handled = len(path) - 1, []
            for j in range(nacc + 1):
                tok = draft[j] if j < nacc else fin
                handled.append(tok)
                if tok in stops:
                    finish, stop_id = "stop", tok
                    break
                hist.append(tok)
                nw += 1
                if nw >= max_new:
                    finish = "length"
                    break
            steps.append((nd, nacc, handled))
            if finish:
                del self.kv[len(hist):]
                break
        return {"steps": steps, "finish": finish, "stop_id": stop_id, "pos": self.pos}


    def spec_sample(self, seq, new_tokens, max_new, draft_len, ngram_n, sampler, rng, stop_ids=(), max_steps=64):
        """hearth_gpu_spec_sample restated: the same steps with the sampled walk over each
        step's live rows (penalty context = the committed sequence), the step's uniforms
        taken in order from a window of the run's stream, rng advanced by those used."""
        draws = sampler.temperature > 0.0
        saved = rng.bit_generator.state if draws else None
        stream = rng.random(max_steps * (draft_len + 1)) if draws else None
        used = 0

        def accept(rows, cmp, nd, hist):
            nonlocal used
            s = O.sampler(sampler.temperature, sampler.top_k, sampler.top_p, sampler.min_p,
                          sampler.repetition_penalty, context=hist)
            u = chain_uniforms(stream[used:used + nd + 1], nd) if draws else np.zeros(2 * (nd + 1))
            rc, path, fin = O.accept_tree_s(rows[:nd + 1], np.asarray(cmp[:nd + 1], np.int32), np.arange(-1, nd), s, u=u)
            if rc == 0 and draws:
                nacc = len(path) - 1
                used += nacc + 1 + (nacc < nd)
            return rc, path, fin

        try:
            res = self._steps(seq, new_tokens, max_new, draft_len, ngram_n, stop_ids, max_steps, accept)
        finally:
            if draws:
                rng.bit_generator.state = saved
        if draws and used:
            rng.random(used)
        if res is not None:
            res["used"] = used
        return res


def _run(make, prompt, n, stops, spec, k, ng, loop, sampler=None):
    e = make()
    gen = generate(e, prompt, n, sampler or Sampler.greedy(), stops, spec, k, ng, device_loop=loop)
    toks = []
    try:
        while True:
            toks.append(next(gen))
    except StopIteration as done:
        st = done.value
    return e, [(t.id, t.step, t.drafted, t.accepted) for t in toks], st


def _counts(st):
    return (st.new_tokens, st.decode_tokens, st.forwards, st.draft_steps, st.drafted, st.accepted, st.finish_reason,
            st.stop_id)


@pytest.mark.parametrize("kw", [dict(follow=2.5), dict(follow=4.0, pos_amp=0.3), dict(history_amp=1.0, follow=1.0)])
def test_device_batches_equal_host_steps(kw):
    drafted = batches = padded = 0
    for seed in range(4):
        for prompt in PROMPTS + [REPEAT]:
            for spec, k, ng in (("ngram", 4, 3), ("ngram", 1, 1), ("ngram", 8, 2), ("none", 4, 3), ("ngram", 0, 3)):
                ref_e, ref, ref_st = _run(lambda: ToyEngine(seed=seed, **kw), prompt, 40, (), spec, k, ng, False)
                e, got, st = _run(lambda: LoopToy(seed=seed, **kw), prompt, 40, (), spec, k, ng, True)
                assert got == ref, (seed, prompt, spec, k, ng)
                assert _counts(st) == _counts(ref_st)
                assert e.kv == ref_e.kv
                drafted += st.drafted
                batches += e.batches
                padded += e.padded_rows
    assert drafted > 0 and batches > 0 and padded > 0


def test_stops_budgets_and_capacity_inside_a_batch():
    cut = 0
    for seed in range(10):
        mk = dict(seed=seed, follow=3.0)
        ref_ids, _ = generate_ids(ToyEngine(**mk), REPEAT, 60)
        for stop_at in (0, 3, 7, 20):
            stops = [ref_ids[min(stop_at, len(ref_ids) - 1)], 999]
            for n in (1, 2, 5, 13, 60):
                for cap in (512, 40, 23):
                    a_e, a, a_st = _run(lambda: ToyEngine(max_seq=cap, **mk), REPEAT, n, stops, "ngram", 6, 3, False)
                    b_e, b, b_st = _run(lambda: LoopToy(max_seq=cap, **mk), REPEAT, n, stops, "ngram", 6, 3, True)
                    assert a == b, (seed, stop_at, n, cap)
                    assert _counts(a_st) == _counts(b_st) and a_e.kv == b_e.kv
                    cut += b_st.finish_reason == "stop" and b_e.batches > 0
    assert cut > 0


def test_closing_inside_a_batch_leaves_a_prefix():
    inside = 0
    for k in range(1, 40):
        e = LoopToy(seed=3, follow=4.0)
        gen = generate(e, REPEAT, 60, Sampler.greedy(), speculative="ngram", draft_len=6, device_loop=True)
        got = [next(gen).id for _ in range(k)]
        inside += e.pos > len(REPEAT) + k
        gen.close()
        seq = REPEAT + got
        assert len(seq) - 1 <= e.pos <= len(seq) and e.kv == seq[:e.pos]
    assert inside > 0


@pytest.mark.parametrize("kw", [dict(follow=2.5), dict(follow=1.0, history_amp=1.0)])
def test_sampled_device_batches_equal_host_steps(kw):
    """Sampled and penalised runs: the device batches yield the host steps' tokens, Token
    fields and counts, keep the same KV, and leave the sampler's generator in the same
    state (the window of uniforms is rewound to what the steps used)."""
    drafted = batches = draws = 0
    settings = (dict(temperature=0.8, top_p=0.95), dict(temperature=1.3, top_k=5),
                dict(temperature=0.7, repetition_penalty=1.3), dict(temperature=0.0, repetition_penalty=1.2),
                dict(temperature=1.0, min_p=0.1))
    for seed in range(3):
        for prompt in (PROMPTS[0], PROMPTS[3], REPEAT):
            for st_kw in settings:
                for spec, k, ng in (("ngram", 4, 3), ("ngram", 8, 2), ("none", 4, 3)):
                    s_ref = Sampler(seed=100 + seed, **st_kw)
                    s_dev = Sampler(seed=100 + seed, **st_kw)
                    ref_e, ref, ref_st = _run(lambda: ToyEngine(seed=seed, **kw), prompt, 30, (), spec, k, ng, False,
                                              s_ref)
                    e, got, st = _run(lambda: LoopToy(seed=seed, **kw), prompt, 30, (), spec, k, ng, True, s_dev)
                    assert got == ref, (seed, prompt, st_kw, spec, k, ng)
                    assert _counts(st) == _counts(ref_st)
                    assert e.kv == ref_e.kv
                    assert s_dev.rng.random() == s_ref.rng.random(), "generator states differ"
                    drafted += st.drafted
                    batches += e.batches
                    draws += st_kw["temperature"] > 0
    assert drafted > 0 and batches > 0 and draws > 0


def test_loop_selection():
    e = LoopToy(seed=1, follow=2.0)
    pen = Sampler(temperature=0.0, repetition_penalty=1.2)
    # with drafts, any sampler takes the device loop by default and on request, and host
    # steps when asked; too many stop ids, or drafts wider than the loop's rows, never do
    for s in (pen, Sampler(temperature=0.7, seed=1), Sampler.greedy()):
        generate_ids(e, REPEAT, 8, s, (), "ngram", 4, 3)
        assert e.batches > 0
        e.batches = 0
        generate_ids(e, REPEAT, 8, s, (), "ngram", 4, 3, device_loop=True)
        assert e.batches > 0
        e.batches = 0
    for stops, k in ((list(range(100, 165)), 4), ((), 128)):
        generate_ids(e, REPEAT, 8, Sampler.greedy(), stops, "ngram", k, 3)
        assert e.batches == 0
        with pytest.raises(ValueError):
            generate_ids(e, REPEAT, 8, Sampler.greedy(), stops, "ngram", k, 3, device_loop=True)
    with pytest.raises(ValueError):
        generate_ids(ToyEngine(), REPEAT, 8, Sampler.greedy(), (), "ngram", 4, 3, device_loop=True)
    generate_ids(e, REPEAT, 8, Sampler.greedy(), (), "ngram", 4, 3, device_loop=False)
    assert e.batches == 0
    # None: the device loop for runs with and without drafts (greedy, penalised or sampled)
    e.batches = 0
    generate_ids(e, REPEAT, 8, Sampler.greedy(), (), "ngram", 4, 3)
    assert e.batches > 0
    for s in (Sampler.greedy(), pen, Sampler(temperature=0.9, seed=2)):
        e.batches = 0
        generate_ids(e, REPEAT, 8, s, (), "none", 4, 3)
        assert e.batches > 0
    generate_ids(e, REPEAT, 8, Sampler.greedy(), (), "ngram", 4, 3, device_loop=True)
    assert e.batches > 1
