"""Generation on the MI355X verify engine: prompt-lookup speculative decoding in which a
decode step is one device call.

Public surface: the names, fields, argument checks and messages of the reference's
python/hearth/generate.py (Sampler 31-126, NgramIndex 150-186, GenStats / Token 189-225,
sync_prefix 250-266, generate 292-400), so front ends written against it run unchanged.

How a generation runs here. A `_Run` owns the committed token sequence, the drafter (an
NgramIndex over that sequence, or none) and the running GenStats. A host step
(`_Run.advance()` without the device loop) is one decode forward: it asks the drafter for
up to `room` tokens and hands [last] + draft to the engine's verify call, which evaluates
the chain, accepts on the GPU (argmax comparison, or exact speculative sampling of a
point-mass proposal fed the uniforms the reference would draw) and commits the accepted
prefix in the KV cache. Only the accepted path and the next token come back to the host;
no logits block crosses PCIe. Greedy runs without a repetition penalty can go further:
the engine's device loop (Engine.spec_greedy) drafts from the sequence it keeps in HBM
and applies the stop and length rules itself, so a batch of steps runs with no host
round trip between them, and only the committed tokens and per-step counts come back
(`device_loop`: by default whenever the engine can run it).
`generate()` applies the stop and length rules to the tokens each forward commits (for a
device batch, the same cut the device made).

Greedy output equals plain greedy decoding token for token (batched evaluation is
bit-identical to sequential evaluation); sampled output has the plain output's
distribution, and for a given seed it is the sample the reference's own speculative loop
draws from the same logits.

`engine` is anything with `pos`, `reset()`, `rewind(pos)`, `eval(tokens)`,
`verify_greedy(tokens)` and `verify_sample(tokens, parent, sampler, u=...)`, and
optionally `spec_loop_ok` and `spec_greedy(...)` (hearth_amd.engine.Engine, or a test
double).
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
_MODE_ALIASES = {None: "none", False: "none", "none": "none", "off": "none", "": "none",
                 True: "ngram", "ngram": "ngram", "prompt": "ngram", "prompt_lookup": "ngram"}

_BAD_LOGITS = "logits contain NaN or +inf, or are all -inf"


# ---------------------------------------------------------------- sampling settings

def _finite_nonneg(v) -> bool:
    return bool(np.isfinite(v)) and v >= 0


# (field, predicate, message) in the order the reference checks them (generate.py:44-55)
_SAMPLER_RULES = (
    ("temperature", _finite_nonneg, "temperature must be >= 0, got {}"),
    ("top_k", lambda v: v >= 0, "top_k must be >= 0, got {}"),
    ("top_p", lambda v: 0.0 < v <= 1.0, "top_p must be in (0, 1], got {}"),
    ("min_p", lambda v: 0.0 <= v <= 1.0, "min_p must be in [0, 1], got {}"),
    ("repetition_penalty", lambda v: bool(np.isfinite(v)) and v > 0, "repetition_penalty must be > 0, got {}"),
)


@dataclass
class Sampler:
    """Sampling settings, applied in the order repetition penalty, temperature, top-k,
    top-p, min-p; temperature 0 is greedy (argmax, first index wins ties). Draws come
    from `rng`, a generator seeded by `seed`. probs / argmax / sample evaluate one logits
    row on the GPU (hearth_gpu_probs, hearth_gpu_accept_sample), in float64 with the
    reference's operation order."""
    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 1.0
    min_p: float = 0.0
    repetition_penalty: float = 1.0
    seed: int | None = None
    rng: np.random.Generator = field(init=False, repr=False, compare=False)

    def __post_init__(self):
        for name, ok, msg in _SAMPLER_RULES:
            v = getattr(self, name)
            if not ok(v):
                raise ValueError(msg.format(v))
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
        """These settings as a hearth_sampler. The penalty context travels only when the
        penalty is on; greedy=True keeps the penalty and sets temperature 0 (the argmax
        of the penalised logits)."""
        ctx = None
        if self.uses_context and context is not None and len(context):
            ctx = context
        return _eng.make_sampler(0.0 if greedy else self.temperature, self.top_k, self.top_p, self.min_p,
                                 self.repetition_penalty, ctx)

    def probs(self, logits, context=None) -> np.ndarray:
        """The final distribution of one logits row (float64; one-hot when greedy)."""
        rc, p = _eng.gpu_probs(_one_row(logits), sampler=self.device(context))
        _raise_on_bad(rc)
        return p[0]

    def argmax(self, logits, context=None) -> int:
        rc, _, tok = _eng.accept_sample(_one_row(logits), [0], None, self.device(context, greedy=True))
        _raise_on_bad(rc)
        return tok

    def sample(self, logits, context=None) -> int:
        """The argmax when greedy, else one inverse-CDF draw (one uniform from rng)."""
        if self.is_greedy:
            return self.argmax(logits, context)
        u = np.array([0.0, self.rng.random()])
        rc, _, tok = _eng.accept_sample(_one_row(logits), [0], None, self.device(context), u=u)
        _raise_on_bad(rc)
        return tok


def _one_row(logits) -> np.ndarray:
    return np.ascontiguousarray(logits, dtype=np.float32).reshape(1, -1)


def _raise_on_bad(rc: int) -> None:
    if rc < 0:
        raise ValueError(_BAD_LOGITS)


# ---------------------------------------------------------------- drafting

class NgramIndex:
    """Prompt-lookup index over a growing token sequence (the reference's drafter,
    generate.py:150-186).

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


# ---------------------------------------------------------------- statistics

def _ratio(num: float, den: float) -> float:
    return num / den if den else 0.0


@dataclass
class GenStats:
    """Running totals of one generation (the reference's fields, generate.py:189-225)."""
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

    acceptance_rate = property(lambda self: _ratio(self.accepted, self.drafted))
    tokens_per_forward = property(lambda self: _ratio(self.decode_tokens, self.forwards))
    prefill_tok_s = property(lambda self: _ratio(self.prompt_tokens - self.reused_tokens, self.prefill_s))
    decode_tok_s = property(lambda self: _ratio(self.decode_tokens, self.decode_s))

    def as_dict(self) -> dict:
        out = dict(self.__dict__)
        for name in ("acceptance_rate", "tokens_per_forward", "prefill_tok_s", "decode_tok_s"):
            out[name] = getattr(self, name)
        return out


class Token(NamedTuple):
    id: int
    step: int          # forward that produced it (0 = prefill)
    drafted: int       # draft length verified in that forward
    accepted: int      # draft tokens accepted in that forward
    stats: GenStats    # running totals (one object for the whole generation)


# ---------------------------------------------------------------- KV bookkeeping

def _max_batch(engine) -> int:
    """Rows one forward may evaluate (the engine's max_batch option; 0 means 512, api.c:178-179)."""
    opts = getattr(engine, "options", None) or {}
    return int(opts.get("max_batch", 0) or 512)


def kv_capacity(engine) -> int:
    """Positions the engine's KV cache holds (kv_capacity, else the model's max_seq)."""
    cap = getattr(engine, "kv_capacity", None)
    if cap is not None:
        return int(cap)
    info = getattr(engine, "info", None) or {}
    return int(info.get("max_seq", 0)) or (1 << 30)


def common_prefix(a: Sequence[int], b: Sequence[int]) -> int:
    """Length of the longest common prefix of two token sequences."""
    n = min(len(a), len(b))
    for i, (x, y) in enumerate(zip(a[:n], b[:n])):
        if int(x) != int(y):
            return i
    return n


def sync_prefix(engine, held: Sequence[int] | None, prompt: Sequence[int]) -> int:
    """Rewinds the engine to the longest prefix of `prompt` whose KV it holds and
    returns that length. `held` lists the tokens behind the engine's KV (None: unknown,
    so the engine is reset). The last prompt token is always left to evaluate: the first
    generated token needs its logits."""
    if held is None or engine.pos > len(held):
        engine.reset()
        return 0
    pos = engine.pos
    keep = min(common_prefix(held[:pos], prompt), len(prompt) - 1, pos)
    if keep < pos:
        engine.rewind(keep)
    return keep


def check_speculative(speculative, draft_len: int, ngram_n: int) -> str:
    """Validates the speculative settings (front ends reject a bad configuration at
    start-up) and returns the normalised mode ("none" or "ngram")."""
    try:
        mode = _MODE_ALIASES[speculative]
    except (KeyError, TypeError):
        raise ValueError(f"speculative must be one of {SPECULATIVE_MODES}, got {speculative!r}") from None
    for name, v, lo in (("draft_len", draft_len, 0), ("ngram_n", ngram_n, 1)):
        if isinstance(v, bool) or not isinstance(v, (int, np.integer)):
            raise ValueError(f"{name} must be an integer, got {v!r}")
        if v < lo:
            raise ValueError(f"{name} must be >= {lo}, got {v}")
    return mode


# ---------------------------------------------------------------- one generation

def _device_verify(engine, context: list[int], draft: list[int], sampler: Sampler) -> tuple[int, int]:
    """One verify forward of [context[-1]] + draft; afterwards the engine holds context
    plus the accepted drafts. Returns (accepted drafts, next token).

    The penalty context of draft row i is context + draft[:i] (generate.py:372-375): the
    device sampler gets `context` and appends the path tokens itself. A sampled step uses
    the reference's uniforms in the reference's order (one per tried draft, a second at a
    rejection, one for the final draw when every draft holds; generate.py:137-147,385)
    and leaves rng advanced by exactly the number it used."""
    toks = [context[-1], *draft]
    k = len(draft)
    if sampler.is_greedy and not sampler.uses_context:
        path, tok, _ = engine.verify_greedy(toks)
        return len(path) - 1, int(tok)
    if sampler.is_greedy:   # argmax of penalised logits: the sampled walk at temperature 0
        path, tok, _ = engine.verify_sample(toks, None, sampler.device(context, greedy=True), u=np.zeros(2 * (k + 1)))
        return len(path) - 1, int(tok)
    rng = sampler.rng
    saved = rng.bit_generator.state
    u = _eng.chain_uniforms(rng.random(k + 1), k)
    path, tok, _ = engine.verify_sample(toks, None, sampler.device(context), u=u)
    accepted = len(path) - 1
    used = accepted + 1 + (accepted < k)
    rng.bit_generator.state = saved
    rng.random(used)
    return accepted, int(tok)


class _Run:
    """The state of one generation: the committed sequence, the drafter, the limits and
    the statistics. After prefill() and every advance(), `steps` holds the forwards that
    call ran, in order, as (drafted, accepted, tokens committed by the forward), and the
    engine holds all of the committed tokens but the last.

    With `loop` set (a greedy run without a repetition penalty, on an engine that offers
    it: `spec_loop_ok`), the run advances by batches of steps run on the device
    (Engine.spec_greedy: drafting, verify, acceptance and the stop and length rules
    without a host round trip per step); the host steps take over near the end of the KV
    cache, where a step's draft must be shorter than the draft length."""

    def __init__(self, engine, prompt: list[int], sampler: Sampler, drafter: NgramIndex | None, draft_len: int,
                 max_new: int, cap: int, stats: GenStats, stops: frozenset, device_loop: bool):
        self.engine, self.sampler, self.drafter = engine, sampler, drafter
        self.draft_len, self.max_new, self.cap, self.stats = draft_len, max_new, cap, stats
        self.seq = list(prompt)
        self.steps: list[tuple[int, int, list[int]]] = []
        self.decoding = False     # steps come from decode forwards (not the prefill)
        self.step = 0
        self.drafted = self.accepted = 0
        self.stops = sorted(stops)
        self.loop = device_loop
        self.batch = 4            # device steps per call, doubling up to 64
        self.bad = False          # the device batch ended at a step with a rejected logits row

    def prefill(self, held) -> None:
        st, prompt = self.stats, self.seq
        st.reused_tokens = sync_prefix(self.engine, held, prompt)
        t0 = time.perf_counter()
        if len(prompt) - st.reused_tokens > 1:
            self.engine.eval(prompt[st.reused_tokens:-1])
        _, first = _device_verify(self.engine, self.seq, [], self.sampler)
        st.prefill_s = time.perf_counter() - t0
        self.steps = [(0, 0, [first])]

    def begin(self, drafted: int, accepted: int) -> None:
        """Counts one decode forward before its tokens are handled."""
        st = self.stats
        self.step += 1
        st.forwards += 1
        self.drafted, self.accepted = drafted, accepted
        if drafted:
            st.draft_steps += 1
            st.drafted += drafted
            st.accepted += accepted

    def commit(self, tok: int) -> None:
        self.seq.append(tok)
        if self.drafter is not None:
            self.drafter.append(tok)

    def base(self) -> int:
        """The engine's position, which must hold all of seq but its last token."""
        pos = self.engine.pos
        if pos != len(self.seq) - 1:
            raise RuntimeError(f"engine position {pos} out of sync with sequence length {len(self.seq)}")
        return pos

    def advance(self, base: int) -> None:
        """The next decode forwards from position base: a batch on the device, or one
        host step. A host step's draft may hold up to the draft length, what the token
        budget leaves after the forward's own token, and the KV positions left."""
        st = self.stats
        if self.bad:
            raise ValueError(_BAD_LOGITS)
        self.decoding = True
        t0 = time.perf_counter()
        if self.loop:
            k = self.draft_len if self.drafter is not None else 0
            ng = self.drafter.max_n if self.drafter is not None else 0
            steps = min(self.batch, self.max_new - st.new_tokens)
            smp = self.sampler
            if smp.is_greedy and not smp.uses_context:
                res = self.engine.spec_greedy(self.seq, st.new_tokens, self.max_new, k, ng, self.stops, max_steps=steps)
            else:
                # sampled acceptance on the device; the penalty context is the committed
                # sequence there, so the sampler travels without one
                res = self.engine.spec_sample(self.seq, st.new_tokens, self.max_new, k, ng,
                                              smp.device(None, greedy=smp.is_greedy),
                                              None if smp.is_greedy else smp.rng, self.stops, max_steps=steps)
            if res is not None:
                self.batch = min(2 * self.batch, 64)
                self.steps = res["steps"]
                self.bad = res["finish"] == "bad_logits"
                st.decode_s += time.perf_counter() - t0
                if self.bad and not self.steps:
                    raise ValueError(_BAD_LOGITS)
                return
        n = min(self.draft_len, self.max_new - st.new_tokens - 1, self.cap - base - 1)
        draft = self.drafter.propose(n) if self.drafter is not None and n > 0 else []
        accepted, final = _device_verify(self.engine, self.seq, draft, self.sampler)
        self.steps = [(len(draft), accepted, draft[:accepted] + [final])]
        st.decode_s += time.perf_counter() - t0

    def release(self) -> None:
        """Cuts the KV back to the yielded tokens (a forward commits its accepted drafts
        before they are yielded, and the caller may stop in between)."""
        try:
            if self.engine.pos > len(self.seq):
                self.engine.rewind(len(self.seq))
        except Exception:
            pass


def _use_device_loop(engine, sampler: Sampler, stops: frozenset, device_loop: bool | None, drafts: bool,
                     draft_len: int = 0) -> bool:
    """None picks the device loop whenever the engine can run it, with or without drafts
    (its padding rows past a short draft cost no work in the forward, and the tokens are
    the host steps' tokens); False forces host steps, True the loop."""
    able = len(stops) <= _eng.SPEC_STOPS_MAX and draft_len + 1 <= _eng.SPEC_ROWS_MAX
    if device_loop is False or not able:
        if device_loop:
            raise ValueError(f"the device loop runs at most {_eng.SPEC_STOPS_MAX} stop ids and drafts of at most "
                             f"{_eng.SPEC_ROWS_MAX - 1} tokens")
        return False
    if drafts and draft_len + 1 > _max_batch(engine):
        if device_loop:
            raise ValueError(f"the device loop evaluates draft_len + 1 = {draft_len + 1} rows per step, more than "
                             f"the engine's max_batch {_max_batch(engine)}")
        return False
    ok = bool(getattr(engine, "spec_loop_ok", False))
    if device_loop and not ok:
        raise ValueError("this engine cannot run the device loop (expert streaming, route replay, a routing trace "
                         "or profiling is on)")
    return ok


def generate(engine, prompt_ids: Sequence[int], max_new_tokens: int = 256, sampler: Sampler | None = None,
             stop_ids: Sequence[int] = (), speculative: str = "none", draft_len: int = 4, ngram_n: int = 3,
             *, held: Sequence[int] | None = None, device_loop: bool | None = None) -> Iterator[Token]:
    """Yields the generated tokens one at a time (a stop token is not yielded) and
    returns the GenStats (StopIteration.value).

    held: the tokens whose KV the engine holds (prefix reuse); None resets the engine.
    device_loop: True runs the generation in batches of steps on the device (drafting and
    acceptance included, greedy or sampled: the sampler's generator is advanced by exactly
    the uniforms the host steps would draw), False always steps from the host, None picks
    the device loop for runs without drafts when the engine offers it. The tokens, the
    statistics and the generator's state afterwards are the same either way.
    Once a token has been yielded or the generator has returned (max_new_tokens == 0
    included), and from then on even if it is closed or interrupted, the engine holds a
    prefix of prompt + yielded tokens of length engine.pos (all but the last token
    after a normal finish). If it raises before that, the KV content is unspecified."""
    sampler = Sampler.greedy() if sampler is None else sampler
    mode = check_speculative(speculative, draft_len, ngram_n)
    if max_new_tokens < 0:
        raise ValueError("max_new_tokens must be >= 0")
    prompt = [int(t) for t in prompt_ids]
    if not prompt:
        raise ValueError("prompt_ids must not be empty")
    cap = kv_capacity(engine)
    if len(prompt) > cap:
        raise ValueError(f"prompt has {len(prompt)} tokens but the KV cache holds {cap}")
    stops = frozenset(int(s) for s in stop_ids)
    st = GenStats(prompt_tokens=len(prompt))
    if max_new_tokens == 0:
        # nothing is evaluated, but the engine still ends up holding a prefix of this
        # prompt, which callers that track the KV rely on
        st.reused_tokens = sync_prefix(engine, held, prompt)
        st.finish_reason = "length"
        return st

    run = _Run(engine, prompt, sampler, NgramIndex(ngram_n, prompt) if mode == "ngram" else None, draft_len,
               max_new_tokens, cap, st, stops,
               _use_device_loop(engine, sampler, stops, device_loop, mode == "ngram" and draft_len > 0,
                                draft_len if mode == "ngram" else 0))
    try:
        run.prefill(held)
        while True:
            for drafted, accepted, toks in run.steps:
                if run.decoding:
                    run.begin(drafted, accepted)
                for tok in toks:
                    st.decode_tokens += run.step > 0
                    if tok in stops:
                        st.finish_reason, st.stop_id = "stop", tok
                        return st
                    run.commit(tok)
                    st.new_tokens += 1
                    yield Token(tok, run.step, run.drafted, run.accepted, st)
                    if st.new_tokens >= max_new_tokens:
                        st.finish_reason = "length"
                        return st
            base = run.base()
            if base + 1 > cap:
                st.finish_reason = "length"
                return st
            run.advance(base)
    finally:
        run.release()


def generate_ids(engine, prompt_ids, max_new_tokens=256, sampler=None, stop_ids=(), speculative="none",
                 draft_len=4, ngram_n=3, *, held=None, device_loop=None) -> tuple[list[int], GenStats]:
    """All tokens of generate() and its GenStats."""
    ids: list[int] = []
    gen = generate(engine, prompt_ids, max_new_tokens, sampler, stop_ids, speculative, draft_len, ngram_n, held=held,
                   device_loop=device_loop)
    try:
        while True:
            ids.append(next(gen).id)
    except StopIteration as done:
        return ids, done.value
