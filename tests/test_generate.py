"""hearth_amd.generate on the CPU, through a deterministic stand-in engine.

ToyEngine computes each position's logits as a function of the tokens so far and does
the verify entry points' acceptance with the CPU restatement (which
tests/test_sampling_oracle.py pins to the reference's Sampler / accept_point_mass /
verify-step vectors). What these tests pin, after the reference's own generate()
tests (tests/py/test_runtime.py:780-996, restated here):

- greedy speculative output equals plain greedy output, token for token, over seeds,
  prompts, draft lengths, n-gram orders, stop tokens, the repetition penalty (whose
  context grows inside a draft) and the KV capacity;
- sampled speculative output has the plain output's distribution (chi-square against
  the exact enumeration, with a negative control that accepts every draft);
- a sampled verify step consumes the reference's uniforms in the reference's order:
  the reference's recorded chain steps (tests/golden/sampling_ref.npz) are reproduced;
- the engine holds a prefix of prompt + yielded tokens whenever the generator is
  suspended or closed, and the Token / GenStats fields add up.
"""
from __future__ import annotations

import zlib

import numpy as np
import pytest

import oracle_py as O
from golden_io import GOLDEN
from hearth_amd.generate import (GenStats, NgramIndex, Sampler, _device_verify, check_speculative, common_prefix,
                                 generate, generate_ids, kv_capacity, sync_prefix)

_CACHE: dict = {}


class ToyEngine:
    """Stand-in engine: the logits after prefix P mix a bigram table (seeded on the last
    two tokens), a position term, a pull towards the token that followed the latest
    earlier occurrence of P[-1] (repetitive text, so n-gram drafts get accepted) and a
    term seeded on all of P (aperiodic text). A forced stop token from position
    `stop_at` on. verify_greedy / verify_sample evaluate the chain, accept with the
    CPU restatement and keep the accepted path, as the engine does on the GPU."""

    def __init__(self, vocab=32, seed=0, max_seq=512, pos_amp=0.0, follow=0.0, history_amp=0.0, stop=None,
                 stop_at=None):
        self.cfg = (vocab, seed, pos_amp, follow, history_amp, stop, stop_at)
        self.vocab_size, self.kv_capacity = vocab, max_seq
        self.kv: list[int] = []
        self.calls = 0
        self.accept = O.accept_tree_s

    def _logits(self, P) -> np.ndarray:
        key = (self.cfg, tuple(P))
        row = _CACHE.get(key)
        if row is not None:
            return row
        V, seed, pos_amp, follow, history_amp, stop, stop_at = self.cfg
        x = np.random.default_rng([seed, P[-1], P[-2] if len(P) > 1 else V]).normal(0, 1, V)
        if pos_amp:
            x += pos_amp * np.random.default_rng([seed, 1 << 20, len(P)]).normal(0, 1, V)
        if follow:
            for j in range(len(P) - 2, -1, -1):
                if P[j] == P[-1]:
                    x[P[j + 1]] += follow
                    break
        if history_amp:
            x += history_amp * np.random.default_rng([seed, zlib.crc32(np.asarray(P, np.int64).tobytes())]).normal(0, 1, V)
        if stop is not None and stop_at is not None and len(P) >= stop_at:
            x[stop] = 50.0
        row = x.astype(np.float32)
        _CACHE[key] = row
        return row

    @property
    def pos(self) -> int:
        return len(self.kv)

    def reset(self) -> None:
        self.kv = []

    def rewind(self, pos: int) -> None:
        if not 0 <= pos <= len(self.kv):
            raise ValueError(f"rewind position {pos} outside [0, {len(self.kv)}]")
        del self.kv[pos:]

    def eval(self, tokens, all_logits=False):
        toks = [int(t) for t in np.asarray(tokens).reshape(-1)]
        if not toks:
            raise ValueError("eval needs at least one token")
        if len(self.kv) + len(toks) > self.kv_capacity:
            raise RuntimeError("KV capacity exceeded")
        self.calls += 1
        rows = []
        for t in toks:
            self.kv.append(t)
            rows.append(self._logits(self.kv))
        return np.stack(rows) if all_logits else rows[-1]

    def _verify(self, tokens, parent, s, u):
        pos0 = self.pos
        rows = self.eval(tokens, all_logits=True)
        n = len(tokens)
        par = np.arange(-1, n - 1) if parent is None else np.asarray(parent)
        rc, path, fin = self.accept(rows, np.asarray(tokens, np.int32), par, s, u=u)
        assert rc == 0
        self.kv[pos0:] = [int(tokens[i]) for i in path]
        return path, fin, rows

    def verify_greedy(self, tokens, parent=None, want_logits=False):
        return self._verify(tokens, parent, O.sampler(0.0), None)

    def verify_sample(self, tokens, parent=None, sampler=None, q=None, u=None, want_logits=False):
        assert q is None
        s = sampler
        ctx = getattr(s, "_ctx", ())
        return self._verify(tokens, parent, O.sampler(s.temperature, s.top_k, s.top_p, s.min_p, s.repetition_penalty,
                                                      context=ctx), u)


PROMPTS = [[1, 2, 3, 1, 2, 3, 1, 2], [5], [7, 7, 7, 7], [3, 9, 4, 3, 9, 4, 3, 9, 4, 3, 9], [0, 1, 2, 3, 4, 5, 6, 7]]
REPEAT = [10, 11, 12, 13, 10, 11, 12, 13, 10, 11]


@pytest.mark.parametrize("kw", [dict(follow=2.5), dict(follow=2.5, pos_amp=0.5), dict(history_amp=1.0, follow=1.0)])
def test_greedy_speculative_equals_plain(kw):
    drafted = accepted = 0
    for seed in range(8):
        for prompt in PROMPTS:
            for draft_len, n in ((4, 3), (1, 1), (8, 2)):
                plain, s1 = generate_ids(ToyEngine(seed=seed, **kw), prompt, 40, Sampler.greedy())
                e = ToyEngine(seed=seed, **kw)
                spec, s2 = generate_ids(e, prompt, 40, Sampler.greedy(), (), "ngram", draft_len, n)
                assert spec == plain, (seed, prompt, draft_len, n)
                assert s1.finish_reason == s2.finish_reason == "length"
                seq = prompt + spec
                assert e.kv == seq[:e.pos] and e.pos == len(seq) - 1
                drafted += s2.drafted
                accepted += s2.accepted
    assert drafted > 0 and accepted > 0


def test_speculation_cuts_forwards_on_repetitive_text():
    plain, s1 = generate_ids(ToyEngine(seed=3, follow=4.0), REPEAT, 100, Sampler.greedy())
    spec, s2 = generate_ids(ToyEngine(seed=3, follow=4.0), REPEAT, 100, Sampler.greedy(), (), "ngram", 6)
    assert spec == plain
    assert s2.acceptance_rate > 0.3 and s2.forwards < s1.forwards / 2 and s2.tokens_per_forward > 2.0
    assert s1.tokens_per_forward == 1.0


def test_stop_penalty_and_capacity_match_plain():
    for seed in range(8):
        prompt = [5, 6, 7, 8, 5, 6, 7]
        ref, _ = generate_ids(ToyEngine(seed=seed, follow=2.0), prompt, 30)
        stop = [ref[min(6, len(ref) - 1)]]
        a, sa = generate_ids(ToyEngine(seed=seed, follow=2.0), prompt, 30, Sampler.greedy(), stop)
        b, sb = generate_ids(ToyEngine(seed=seed, follow=2.0), prompt, 30, Sampler.greedy(), stop, "ngram", 5, 3)
        assert a == b and sa.finish_reason == sb.finish_reason == "stop" and sa.stop_id == sb.stop_id == stop[0]
        assert stop[0] not in a
        pen = dict(temperature=0.0, repetition_penalty=1.3)
        a, _ = generate_ids(ToyEngine(seed=seed, follow=2.0), prompt, 40, Sampler(**pen))
        b, _ = generate_ids(ToyEngine(seed=seed, follow=2.0), prompt, 40, Sampler(**pen), (), "ngram", 4, 3)
        assert a == b
        a, sa = generate_ids(ToyEngine(seed=seed, follow=2.0, max_seq=20), prompt, 100)
        e = ToyEngine(seed=seed, follow=2.0, max_seq=20)
        b, sb = generate_ids(e, prompt, 100, Sampler.greedy(), (), "ngram", 6, 3)
        assert a == b and len(a) == 20 - len(prompt) + 1 and sa.finish_reason == sb.finish_reason == "length"
        assert e.pos <= 20


def test_penalty_context_inside_a_draft():
    """Small vocabulary and short prompts: accepted drafts are long next to the
    context, so the penalty context of rows inside the draft decides the output."""
    accepted = 0
    for seed in range(12):
        for penalty in (1.5, 2.5, 4.0):
            for prompt in ([2, 0, 3, 0, 2], [1, 2, 3, 1, 2], [7, 7]):
                kw = dict(vocab=12, seed=seed, follow=3.0)
                s = dict(temperature=0.0, repetition_penalty=penalty)
                a, _ = generate_ids(ToyEngine(**kw), prompt, 24, Sampler(**s))
                b, st = generate_ids(ToyEngine(**kw), prompt, 24, Sampler(**s), (), "ngram", 4, 1)
                assert a == b, (seed, penalty, prompt)
                accepted += st.accepted
    assert accepted > 0


def test_closing_mid_burst_leaves_a_prefix():
    inside = 0
    for k in range(1, 40):
        e = ToyEngine(seed=3, follow=4.0)
        gen = generate(e, REPEAT, 60, Sampler.greedy(), speculative="ngram", draft_len=6)
        got = [next(gen).id for _ in range(k)]
        inside += e.pos > len(REPEAT) + k
        gen.close()
        seq = REPEAT + got
        assert len(seq) - 1 <= e.pos <= len(seq) and e.kv == seq[:e.pos]
    assert inside > 0


def test_token_fields_and_stats_add_up():
    toks = list(generate(ToyEngine(seed=3, follow=4.0), REPEAT, 60, Sampler.greedy(), speculative="ngram",
                         draft_len=6))
    st = toks[-1].stats
    by_step: dict = {}
    for t in toks:
        by_step.setdefault(t.step, []).append(t)
    assert [(t.drafted, t.accepted) for t in by_step[0]] == [(0, 0)]
    for ts in by_step.values():
        d, a = ts[0].drafted, ts[0].accepted
        assert all((t.drafted, t.accepted) == (d, a) for t in ts) and 0 <= a <= d and len(ts) <= a + 1
    assert st.drafted == sum(ts[0].drafted for ts in by_step.values())
    assert st.accepted == sum(ts[0].accepted for ts in by_step.values())
    assert st.draft_steps == sum(1 for ts in by_step.values() if ts[0].drafted) > 0
    assert st.forwards == max(by_step) and st.decode_tokens == st.new_tokens - 1 == 59
    assert 0 < st.decode_tok_s and 0 < st.prefill_tok_s
    d = st.as_dict()
    assert d["accepted"] == st.accepted and d["acceptance_rate"] == st.acceptance_rate
    plain = list(generate(ToyEngine(seed=3), REPEAT, 20))
    assert [(t.step, t.drafted, t.accepted) for t in plain] == [(i, 0, 0) for i in range(20)]
    assert plain[-1].stats.forwards == 19 and plain[-1].stats.draft_steps == 0


def test_edge_cases_and_argument_checks():
    e = ToyEngine()
    out, st = generate_ids(e, [1, 2], 0)
    assert out == [] and st.finish_reason == "length"
    for args, kw in ((([], 4), {}), (([1], -1), {}), (([1], 4), dict(speculative="medusa")),
                     (([1], 4), dict(speculative="ngram", ngram_n=0))):
        with pytest.raises(ValueError):
            generate_ids(e, *args, **kw)
    with pytest.raises(ValueError):
        generate_ids(ToyEngine(max_seq=4), [1, 2, 3, 4, 5], 4)
    out, st = generate_ids(ToyEngine(stop=3, stop_at=4), [1, 2], 10, None, [3])
    assert st.finish_reason == "stop" and st.stop_id == 3 and 3 not in out and len(out) == 2
    assert check_speculative("none", 4, 3) == "none" and check_speculative(None, 0, 1) == "none"
    assert check_speculative(True, np.int64(4), 3) == "ngram"
    for bad in (("medusa", 4, 3), ("ngram", -1, 3), ("ngram", 4, 0), ("ngram", 2.5, 3), ("ngram", 4, True)):
        with pytest.raises(ValueError):
            check_speculative(*bad)
    for bad in (dict(temperature=-1), dict(top_k=-1), dict(top_p=0.0), dict(min_p=1.5),
                dict(repetition_penalty=0.0), dict(temperature=float("nan"))):
        with pytest.raises(ValueError):
            Sampler(**bad)


def test_prefix_reuse():
    e = ToyEngine()
    a, b = [1, 2, 3, 4, 5, 6], [1, 2, 9, 9]
    e.eval(a)
    out, st = generate_ids(e, b, 0, held=a)
    assert out == [] and st.reused_tokens == 2 and e.kv == [1, 2] and e.calls == 1
    out, st = generate_ids(e, [1, 2], 0, held=None)
    assert e.pos == 0 and st.reused_tokens == 0
    # a reused prefix gives the output of a cold start
    cold, _ = generate_ids(ToyEngine(seed=2, follow=2.0), [4, 5, 6, 4, 5], 12)
    e = ToyEngine(seed=2, follow=2.0)
    e.eval([4, 5, 6, 9])
    warm, st = generate_ids(e, [4, 5, 6, 4, 5], 12, held=[4, 5, 6, 9], speculative="ngram")
    assert warm == cold and st.reused_tokens == 3 and st.prompt_tokens == 5
    assert common_prefix([1, 2, 3], [1, 2, 4, 5]) == 2 and common_prefix([], [1]) == 0
    assert kv_capacity(ToyEngine(max_seq=33)) == 33
    e = ToyEngine()
    e.eval([1, 2, 3])
    assert sync_prefix(e, [1, 2, 3], [1, 2, 3]) == 2 and e.pos == 2     # one token left to evaluate


def test_ngram_index_proposals():
    ix = NgramIndex(3, [1, 2, 3, 4, 1, 2, 3])
    assert ix.propose(3) == [4, 1, 2]          # "1 2 3" followed by 4 1 2
    ix.append(9)
    assert ix.propose(2) == []                 # 9 never seen before
    ix = NgramIndex(2, [5, 6, 5, 7, 5])
    assert ix.propose(4) == [7, 5]             # latest earlier occurrence of "5" wins
    ix = NgramIndex(3, [1, 2, 1, 3, 1, 4, 2, 1])
    assert ix.propose(1) == [3]                # "2 1" (longest match) beats the later "1"
    assert NgramIndex(2).propose(3) == [] and ix.propose(0) == []
    with pytest.raises(ValueError):
        NgramIndex(0)


class _Stream:
    """A generator stand-in whose random() draws come from a recorded stream."""

    class _Bits:
        def __init__(self, outer):
            self.outer = outer

        @property
        def state(self):
            return self.outer.used

        @state.setter
        def state(self, v):
            self.outer.used = v

    def __init__(self, values):
        self.values = np.asarray(values, dtype=np.float64)
        self.used = 0
        self.bit_generator = _Stream._Bits(self)

    def random(self, n=None):
        m = 1 if n is None else n
        out = np.concatenate([self.values[self.used:self.used + m], np.full(max(0, self.used + m - self.values.size), 0.5)])
        self.used += m
        return out[0] if n is None else out


class _RowsEngine(ToyEngine):
    """Serves recorded logits rows for one verify call."""

    def __init__(self, rows, n_ctx):
        super().__init__(vocab=rows.shape[1], max_seq=n_ctx + rows.shape[0] + 1)
        self.rows = rows
        self.kv = [0] * (n_ctx - 1)

    def eval(self, tokens, all_logits=False):
        n = len(tokens)
        self.kv += [int(t) for t in tokens]
        return self.rows[:n] if all_logits else self.rows[n - 1]


def test_sampled_step_reproduces_reference_steps():
    fix = np.load(GOLDEN / "sampling_ref.npz")
    C = fix["chains"]
    for j in range(len(C)):
        rows, draft, seq = fix[f"s{j}_rows"], fix[f"s{j}_draft"], fix[f"s{j}_seq"]
        T, top_k, top_p, min_p, rp = (float(v) for v in C[j][:5])
        smp = Sampler(temperature=T, top_k=int(top_k), top_p=top_p, min_p=min_p, repetition_penalty=rp)
        stream = fix[f"s{j}_stream"]
        smp.rng = _Stream(stream)
        e = _RowsEngine(rows, len(seq))
        n_acc, final = _device_verify(e, [int(t) for t in seq], [int(d) for d in draft], smp)
        want_acc, want_final, used = int(C[j][5]), int(C[j][6]), int(C[j][7])
        assert (n_acc, final) == (want_acc, want_final), j
        assert smp.rng.used == used, j
        assert e.pos == len(seq) + n_acc


def _plain_distribution(make, prompt, n_new, kw):
    """The exact distribution of n_new plain-sampled tokens, by enumeration."""
    dist: dict = {}

    def rec(seq, prob):
        if len(seq) - len(prompt) == n_new:
            dist[tuple(seq[len(prompt):])] = prob
            return
        lg = make()._logits(seq)
        rc, p = O.probs_s(lg, O.sampler(**kw))
        assert rc == 0
        for t in np.flatnonzero(p):
            rec(seq + [int(t)], prob * p[t])

    rec(list(prompt), 1.0)
    return dist


@pytest.mark.parametrize("broken", [False, True])
def test_sampled_speculation_keeps_the_distribution(broken):
    """Speculative sampling must leave the distribution of the generated text that of
    plain sampling. The exact plain distribution of 3 new tokens (vocabulary 4) comes
    from enumerating every continuation; n speculative runs give an empirical one. Their
    total-variation distance is a sum of |binomial deviations|, whose mean is at most
    0.5 * sum_i sqrt(p_i (1 - p_i) / n); the test allows twice that mean plus a floor. A
    drafter whose drafts are always accepted (the negative control) shifts mass towards
    the n-gram continuations and must fail the same bound."""
    def make():
        e = ToyEngine(vocab=4, seed=5, follow=1.0, pos_amp=0.5)
        if broken:
            e.accept = lambda rows, toks, par, s, u=None: (0, list(range(len(toks))),
                                                           O.accept_tree_s(rows, toks, par, s, u=u)[2])
        return e

    prompt = [0, 1, 2, 3, 0, 1, 2, 3, 0, 1]
    exact = _plain_distribution(make, prompt, 3, dict(temperature=1.0))
    n = 4000
    seen: dict = {}
    drafted = 0
    for seed in range(n):
        out, st = generate_ids(make(), prompt, 3, Sampler(seed=seed, temperature=1.0), (), "ngram", 2, 2)
        seen[tuple(out)] = seen.get(tuple(out), 0) + 1
        drafted += st.drafted
    assert drafted > 0
    support = set(exact) | set(seen)
    tv = 0.5 * sum(abs(seen.get(k, 0) / n - exact.get(k, 0.0)) for k in support)
    mean_bound = 0.5 * sum(np.sqrt(p * (1 - p) / n) for p in exact.values())
    limit = 2.0 * mean_bound + 0.005
    assert (tv > limit) if broken else (tv < limit), (tv, limit)


def test_sampled_generation_is_reproducible_and_consistent():
    kw = dict(vocab=16, seed=7, follow=2.0)
    for s in (dict(temperature=0.8, top_p=0.95), dict(temperature=1.0, top_k=5, repetition_penalty=1.2)):
        a, sa = generate_ids(ToyEngine(**kw), REPEAT, 30, Sampler(seed=11, **s), (), "ngram", 4)
        e = ToyEngine(**kw)
        b, sb = generate_ids(e, REPEAT, 30, Sampler(seed=11, **s), (), "ngram", 4)
        assert a == b and sa.accepted == sb.accepted and len(a) == 30
        seq = REPEAT + b
        assert e.kv == seq[:e.pos] and e.pos == len(seq) - 1
        assert isinstance(sa, GenStats) and sa.drafted > 0


def test_cli_rejects_bad_arguments_before_opening(capsys):
    from hearth_amd.cli import build_parser, main
    assert main(["run", "missing.hearth", "--ids", "1,x"]) == 2
    assert main(["run", "missing.hearth", "--ids", "1,2", "--top-p", "0"]) == 2
    assert main(["run", "missing.hearth", "--ids", "1", "--speculative", "ngram", "--draft-len", "-1"]) == 2
    assert main(["bench", "missing.hearth", "--speculative", "ngram"]) == 2      # needs --ids greedy
    err = capsys.readouterr().err
    assert err.count("hearth_amd: error:") == 4
    a = build_parser().parse_args(["bench", "m.hearth", "--ids", "greedy", "--speculative", "ngram", "--draft-len", "8"])
    assert (a.speculative, a.draft_len, a.ngram_n, a.prompt_tokens, a.gen_tokens) == ("ngram", 8, 3, 128, 64)
