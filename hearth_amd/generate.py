"""Generation with lossless prompt-lookup speculative decoding, verified on the GPU.

The same interface and emitted tokens as the reference's python/hearth/generate.py:
`generate()` (generate.py:292-400) yields `Token`s with running `GenStats`
(generate.py:189-225), drafts come from an n-gram lookup over the context itself
(`NgramIndex`, generate.py:150-186) and `Sampler` carries the reference's settings
(generate.py:31-126).

The difference is where a verify step runs. The reference evaluates [last] + draft
with all logits, walks the draft in numpy and rewinds the KV cache
(generate.py:365-392). Here one engine call does all three on the device:
`verify_greedy` (argmax compare) or `verify_sample` (exact speculative sampling with a
point-mass proposal, fed the uniforms the reference would draw from the sampler's
generator) evaluates the chain, accepts on the GPU and commits the accepted prefix, so
no [k+1][V] logits block crosses PCIe. Greedy output is token-for-token the output of
plain greedy decoding because batched evaluation is bit-identical to sequential
evaluation; sampled output has the plain output's distribution, and with a fixed seed
it is the sample the reference's own speculative loop draws on the same logits.

`engine` is anything with `pos`, `reset()`, `rewind(pos)`, `eval(tokens)`,
`verify_greedy(tokens)` and `verify_sample(tokens, parent, sampler, u=...)`
(hearth_amd.engine.Engine, or a test double).
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Iterator, NamedTuple, Sequence

import numpy as np

from . import engine as _eng

__all__ = ["Sampler", "GenStats", "Token", "generate", "generate_ids", "NgramIndex", "common_prefix", "sync_prefix",
           "kv_capacity", "check_speculative", "SPECULATIVE_MODES"]

SPECULATIVE_MODES = ("none", "ngram")


@dataclass
class Sampler:
    """Sampling settings, applied in the reference's order (generate.py:31-36):
    repetition penalty, temperature, top-k, top-p, min-p. temperature 0 is greedy
    (argmax, first index wins ties). `rng` is the generator the sampled verify steps
    draw their uniforms from (seeded by `seed`).

    probs / argmax / sample evaluate one logits row on the GPU (hearth_gpu_probs,
    hearth_gpu_accept_sample) with the reference's numerics (generate.py:69-126)."""
    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 1.0
    min_p: float = 0.0
    repetition_penalty: float = 1.0
    seed: int | None = None
    rng: np.random.Generator = field(init=False, repr=False, compare=False)

    def __post_init__(self):
        # the reference's argument checks and messages (generate.py:44-55)
        if not np.isfinite(self.temperature) or self.temperature < 0:
            raise ValueError(f"temperature must be >= 0, got {self.temperature}")
        if self.top_k < 0:
            raise ValueError(f"top_k must be >= 0, got {self.top_k}")
        if not 0.0 < self.top_p <= 1.0:
            raise ValueError(f"top_p must be in (0, 1], got {self.top_p}")
        if not 0.0 <= self.min_p <= 1.0:
            raise ValueError(f"min_p must be in [0, 1], got {self.min_p}")
        if not np.isfinite(self.repetition_penalty) or self.repetition_penalty <= 0:
            raise ValueError(f"repetition_penalty must be > 0, got {self.repetition_penalty}")
        self.rng = np.random.default_rng(self.seed)

    @classmethod
    def greedy(cls) -> "Sampler":
        return cls(temperature=0.0)

    @property
    def is_greedy(self) -> bool:
        return self.temperature == 0.0

    @property
    def uses_context(self) -> bool:
        return self.repetition_penalty != 1.0

    def device(self, context=None, *, greedy: bool = False) -> _eng.HearthSampler:
        """The hearth_sampler of these settings; `context` (the ids the penalty applies
        to) is only passed when the penalty is on. greedy=True keeps the penalty and
        sets temperature 0 (the reference's argmax of penalised logits)."""
        ctx = context if self.uses_context and context is not None and len(context) else None
        return _eng.make_sampler(0.0 if greedy else self.temperature, self.top_k, self.top_p, self.min_p,
                                 self.repetition_penalty, ctx)

    @staticmethod
    def _row(logits) -> np.ndarray:
        return np.ascontiguousarray(logits, dtype=np.float32).reshape(1, -1)

    def probs(self, logits, context=None) -> np.ndarray:
        """The final sampling distribution of one logits row (float64, one-hot when
        greedy). NaN or +inf logits, or all -inf, raise ValueError."""
        rc, p = _eng.gpu_probs(self._row(logits), sampler=self.device(context))
        if rc < 0:
            raise ValueError("logits contain NaN or +inf, or are all -inf")
        return p[0]

    def argmax(self, logits, context=None) -> int:
        rc, _, fin = _eng.accept_sample(self._row(logits), [0], None, self.device(context, greedy=True))
        if rc < 0:
            raise ValueError("logits contain NaN or +inf, or are all -inf")
        return fin

    def sample(self, logits, context=None) -> int:
        """argmax when greedy, else one inverse-CDF draw (one uniform from rng)."""
        if self.is_greedy:
            return self.argmax(logits, context)
        rc, _, fin = _eng.accept_sample(self._row(logits), [0], None, self.device(context),
                                        u=np.array([0.0, self.rng.random()]))
        if rc < 0:
            raise ValueError("logits contain NaN or +inf, or are all -inf")
        return fin


class NgramIndex:
    """Prompt-lookup index over a growing token sequence (generate.py:150-186).

    For each n-gram of length 1..max_n it keeps the latest start position that is
    followed by at least one token, so the current suffix never matches itself, and
    `propose(k)` returns up to k tokens that followed the latest earlier occurrence of
    the longest matching suffix. Keys of different lengths are distinct tuples, so one
    dictionary holds every n."""

    def __init__(self, max_n: int, tokens: Sequence[int] = ()):
        if max_n < 1:
            raise ValueError("ngram_n must be >= 1")
        self.max_n = max_n
        self.seq: list[int] = []
        self._last: dict[tuple, int] = {}
        for t in tokens:
            self.append(t)

    def append(self, tok: int) -> None:
        s = self.seq
        s.append(int(tok))
        end = len(s) - 1                 # the n-grams ending just before the new token gained a follower
        for n in range(1, min(self.max_n, end) + 1):
            self._last[tuple(s[end - n:end])] = end - n

    def propose(self, k: int) -> list[int]:
        s = self.seq
        if k <= 0:
            return []
        for n in range(min(self.max_n, len(s)), 0, -1):
            start = self._last.get(tuple(s[-n:]))
            if start is not None:
                return s[start + n:start + n + k]
        return []


@dataclass
class GenStats:
    """Running totals of one generation (generate.py:189-225, same fields)."""
    prompt_tokens: int = 0
    reused_tokens: int = 0         # prompt tokens whose KV the engine already held
    new_tokens: int = 0            # tokens yielded (a stop token is not)
    decode_tokens: int = 0         # tokens produced by decode forwards, a final stop token included
    forwards: int = 0              # decode forwards (verify steps), prefill excluded
    draft_steps: int = 0           # forwards that verified a non-empty draft
    drafted: int = 0
    accepted: int = 0
    prefill_s: float = 0.0
    decode_s: float = 0.0
    finish_reason: str | None = None   # "stop" or "length"
    stop_id: int | None = None

    @property
    def acceptance_rate(self) -> float:
        return self.accepted / self.drafted if self.drafted else 0.0

    @property
    def tokens_per_forward(self) -> float:
        return self.decode_tokens / self.forwards if self.forwards else 0.0

    @property
    def prefill_tok_s(self) -> float:
        n = self.prompt_tokens - self.reused_tokens
        return n / self.prefill_s if self.prefill_s > 0 else 0.0

    @property
    def decode_tok_s(self) -> float:
        return self.decode_tokens / self.decode_s if self.decode_s > 0 else 0.0

    def as_dict(self) -> dict:
        d = dict(self.__dict__)
        d.update(acceptance_rate=self.acceptance_rate, tokens_per_forward=self.tokens_per_forward,
                 prefill_tok_s=self.prefill_tok_s, decode_tok_s=self.decode_tok_s)
        return d


class Token(NamedTuple):
    id: int
    step: int          # forward that produced it (0 = prefill)
    drafted: int       # draft length verified in that forward
    accepted: int      # draft tokens accepted in that forward
    stats: GenStats    # running totals (one object for the whole generation)


def kv_capacity(engine) -> int:
    cap = getattr(engine, "kv_capacity", None)
    if cap is None:
        info = getattr(engine, "info", None) or {}
        cap = int(info.get("max_seq", 0)) or (1 << 30)
    return int(cap)


def common_prefix(a: Sequence[int], b: Sequence[int]) -> int:
    n = min(len(a), len(b))
    if n == 0:
        return 0
    ne = np.flatnonzero(np.asarray(a[:n], dtype=np.int64) != np.asarray(b[:n], dtype=np.int64))
    return int(ne[0]) if ne.size else n


def sync_prefix(engine, held: Sequence[int] | None, prompt: Sequence[int]) -> int:
    """Rewinds the engine to the longest prefix of `prompt` whose KV it holds and
    returns its length (generate.py:250-266). `held` lists the tokens behind the
    engine's KV (None: unknown, so reset). At least one prompt token is left to
    evaluate, since the first generated token needs its logits."""
    if held is None:
        engine.reset()
        return 0
    pos = engine.pos
    if pos > len(held):
        engine.reset()
        return 0
    k = min(common_prefix(held[:pos], prompt), len(prompt) - 1, pos)
    if k < pos:
        engine.rewind(k)
    return k


def _mode(speculative) -> str:
    if speculative in (None, False, "none", "off", ""):
        return "none"
    if speculative in (True, "ngram", "prompt", "prompt_lookup"):
        return "ngram"
    raise ValueError(f"speculative must be one of {SPECULATIVE_MODES}, got {speculative!r}")


def check_speculative(speculative, draft_len: int, ngram_n: int) -> str:
    """Validates the speculative settings (front ends reject a bad configuration at
    start-up) and returns the normalised mode."""
    mode = _mode(speculative)
    for name, v, lo in (("draft_len", draft_len, 0), ("ngram_n", ngram_n, 1)):
        if isinstance(v, bool) or not isinstance(v, (int, np.integer)):
            raise ValueError(f"{name} must be an integer, got {v!r}")
        if v < lo:
            raise ValueError(f"{name} must be >= {lo}, got {v}")
    return mode


def _chain_step(engine, seq: list[int], draft: list[int], sampler: Sampler) -> tuple[int, int]:
    """One verify forward of [seq[-1]] + draft on the device; the engine then holds
    seq plus the accepted drafts. Returns (accepted drafts, next token).

    The penalty context of row i is seq + draft[:i] (generate.py:372-375): the
    sampler's context is seq and the device appends the path tokens. A sampled step
    takes the reference's uniforms in the reference's order (one per tried draft, a
    second one at a rejection, one for the final draw when every draft holds;
    generate.py:137-147,385) and leaves rng advanced by exactly that many."""
    toks = [seq[-1]] + draft
    k = len(draft)
    if sampler.is_greedy:
        if sampler.uses_context:
            path, fin, _ = engine.verify_sample(toks, None, sampler.device(seq, greedy=True), u=np.zeros(2 * (k + 1)))
        else:
            path, fin, _ = engine.verify_greedy(toks)
        return len(path) - 1, int(fin)
    rng = sampler.rng
    state = rng.bit_generator.state
    stream = rng.random(k + 1)
    path, fin, _ = engine.verify_sample(toks, None, sampler.device(seq), u=_eng.chain_uniforms(stream, k))
    n_acc = len(path) - 1
    rng.bit_generator.state = state
    rng.random(n_acc + (1 if n_acc < k else 0) + 1)
    return n_acc, int(fin)


def generate(engine, prompt_ids: Sequence[int], max_new_tokens: int = 256, sampler: Sampler | None = None,
             stop_ids: Sequence[int] = (), speculative: str = "none", draft_len: int = 4, ngram_n: int = 3,
             *, held: Sequence[int] | None = None) -> Iterator[Token]:
    """Yields the generated tokens one at a time (a stop token is not yielded) and
    returns the GenStats (StopIteration.value).

    held: the tokens whose KV the engine holds (prefix reuse); None resets the engine.
    Once a token has been yielded or the generator has returned (max_new_tokens == 0
    included), and from then on even if it is closed or interrupted, the engine holds a
    prefix of prompt + yielded tokens of length engine.pos (all but the last token
    after a normal finish). If it raises before that, the KV content is unspecified.
    """
    sampler = sampler if sampler is not None else Sampler.greedy()
    mode = check_speculative(speculative, draft_len, ngram_n)
    if max_new_tokens < 0:
        raise ValueError("max_new_tokens must be >= 0")
    prompt = [int(t) for t in prompt_ids]
    if not prompt:
        raise ValueError("prompt_ids must not be empty")
    cap = kv_capacity(engine)
    if len(prompt) > cap:
        raise ValueError(f"prompt has {len(prompt)} tokens but the KV cache holds {cap}")
    stop = frozenset(int(s) for s in stop_ids)
    st = GenStats(prompt_tokens=len(prompt))
    if max_new_tokens == 0:
        # nothing is evaluated, but the engine still ends up holding a prefix of this
        # prompt, which callers that track the KV rely on
        st.reused_tokens = sync_prefix(engine, held, prompt)
        st.finish_reason = "length"
        return st

    seq = list(prompt)
    index = NgramIndex(ngram_n, seq) if mode == "ngram" else None
    try:
        k = sync_prefix(engine, held, prompt)
        st.reused_tokens = k
        t0 = time.perf_counter()
        if len(prompt) - k > 1:
            engine.eval(prompt[k:-1])
        _, first = _chain_step(engine, seq, [], sampler)
        st.prefill_s = time.perf_counter() - t0
        new, step, drafted, n_acc = [first], 0, 0, 0

        while True:
            for tok in new:
                if step > 0:
                    st.decode_tokens += 1
                if tok in stop:
                    st.finish_reason, st.stop_id = "stop", tok
                    return st
                seq.append(tok)
                if index is not None:
                    index.append(tok)
                st.new_tokens += 1
                yield Token(tok, step, drafted, n_acc, st)
                if st.new_tokens >= max_new_tokens:
                    st.finish_reason = "length"
                    return st

            base = engine.pos                      # holds seq[:-1]; seq[-1] is fed next
            if base != len(seq) - 1:
                raise RuntimeError(f"engine position {base} out of sync with sequence length {len(seq)}")
            if base + 1 > cap:
                st.finish_reason = "length"
                return st
            room = min(draft_len, max_new_tokens - st.new_tokens - 1, cap - base - 1)
            draft = index.propose(room) if index is not None and room > 0 else []
            t0 = time.perf_counter()
            step += 1
            st.forwards += 1
            n_acc, final = _chain_step(engine, seq, draft, sampler)
            new = draft[:n_acc] + [final]
            drafted = len(draft)
            if draft:
                st.draft_steps += 1
                st.drafted += drafted
                st.accepted += n_acc
            st.decode_s += time.perf_counter() - t0
    finally:
        # the post-condition holds even when the generator is closed inside a burst of
        # accepted drafts (the device committed them before they were yielded)
        try:
            if engine.pos > len(seq):
                engine.rewind(len(seq))
        except Exception:
            pass


def generate_ids(engine, prompt_ids, max_new_tokens=256, sampler=None, stop_ids=(), speculative="none",
                 draft_len=4, ngram_n=3, *, held=None) -> tuple[list[int], GenStats]:
    """All tokens of generate() and its GenStats."""
    gen = generate(engine, prompt_ids, max_new_tokens, sampler, stop_ids, speculative, draft_len, ngram_n, held=held)
    out = []
    while True:
        try:
            out.append(next(gen).id)
        except StopIteration as e:
            return out, e.value
