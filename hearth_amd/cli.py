"""`python -m hearth_amd <command>`: the verify engine's command line.

Commands: `info` (a container's engine info), `run` (generate from token ids, with
sampling and prompt-lookup speculative decoding verified on the GPU) and `bench`
(prefill and decode speed). Flag names, defaults and the JSON keys of `bench` are the
reference's (python/hearth/cli.py: engine options 27-53, sampling 56-73, bench 408-474
and 705-717), so scripts written against `hearth bench` read this output unchanged;
`bench --speculative ngram` adds a `verify` block (forwards, drafted, accepted,
acceptance rate, tokens per forward). Text front ends (tokenizer, chat template, HTTP
server) are not part of this package.
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from .engine import Engine, HearthError
from .generate import Sampler, check_speculative, generate


class CLIError(Exception):
    """A user-facing error: printed without a traceback, exit status 2."""


# ---------------------------------------------------------------- engine options

# (flag, Engine keyword, argparse settings). One table drives both the parser and the
# Engine call. --buffered is stored inverted (direct_io) and --mirror appends.
_ENGINE_FLAGS = (
    ("--cache-gb", "cache_gb", dict(type=float, default=8.0, help="budget for routed experts in GiB (default 8)")),
    ("--threads", "threads", dict(type=int, default=0, help="host threads (0 = default)")),
    ("--io-threads", "io_threads", dict(type=int, default=0, help="expert reader threads (0 = default)")),
    ("--buffered", "direct_io", dict(action="store_true", help="use the OS page cache instead of direct I/O")),
    ("--policy", "policy", dict(choices=["lru", "lfu"], default="lfu", help="expert cache eviction policy")),
    ("--prefetch", "prefetch", dict(choices=["off", "next", "shared"], default="shared", help="next-layer prefetch mode")),
    ("--prefetch-extra", "prefetch_extra", dict(type=int, default=0, help="predict top_k + N experts for the next layer")),
    ("--usage-in", "usage_in", dict(metavar="PATH", help="heat profile to seed the cache")),
    ("--usage-out", "usage_out", dict(metavar="PATH", help="write the heat profile here on close")),
    ("--pin-fraction", "pin_fraction", dict(type=float, default=0.0, help="fraction of cache slots pinned at open")),
    ("--warm-start", "warm_start", dict(action="store_true", help="fill the cache with the hottest experts at open")),
    ("--max-seq", "max_seq", dict(type=int, default=0, help="KV capacity in tokens (0 = min(model, 4096))")),
    ("--max-batch", "max_batch", dict(type=int, default=0, help="max tokens per forward chunk (0 = default)")),
    ("--isa", "isa", dict(choices=["auto", "scalar", "avx2", "avx512"], default="auto")),
    ("--mirror", "mirrors", dict(action="append", default=[], metavar="PATH", help="byte-identical model copy")),
    ("-v", "verbose", dict(action="count", default=0, help="engine log level", dest="verbose")),
)


def add_engine_args(p: argparse.ArgumentParser) -> None:
    g = p.add_argument_group("engine")
    for flag, _, kw in _ENGINE_FLAGS:
        names = [flag, "--verbose"] if flag == "-v" else [flag]
        g.add_argument(*names, **kw)


def engine_kwargs(args) -> dict:
    """Engine keyword arguments of parsed engine flags."""
    out = {}
    for flag, key, kw in _ENGINE_FLAGS:
        v = getattr(args, kw.get("dest", flag.lstrip("-").replace("-", "_")))
        if key == "direct_io":
            v = not v
        elif key == "mirrors":
            v = list(v)
        out[key] = v
    return out


# ---------------------------------------------------------------- sampling options

def add_spec_args(g) -> None:
    g.add_argument("--speculative", choices=["none", "ngram"], default="none",
                   help="prompt-lookup speculative decoding, verified on the GPU (lossless)")
    g.add_argument("--draft-len", type=int, default=4, help="max draft tokens per forward (default 4)")
    g.add_argument("--ngram-n", type=int, default=3, help="longest n-gram matched for drafting (default 3)")


def add_sampling_args(p: argparse.ArgumentParser, temperature: float, max_tokens: int) -> None:
    g = p.add_argument_group("sampling")
    g.add_argument("-n", "--max-tokens", type=int, default=max_tokens, help=f"tokens to generate (default {max_tokens})")
    g.add_argument("--temperature", type=float, default=temperature, help=f"0 = greedy (default {temperature})")
    for flag, typ, default in (("--top-k", int, 0), ("--top-p", float, 1.0), ("--min-p", float, 0.0),
                               ("--repetition-penalty", float, 1.0)):
        g.add_argument(flag, type=typ, default=default)
    g.add_argument("--seed", type=int, default=None)
    add_spec_args(g)


def _sampler_of(args) -> Sampler:
    try:
        return Sampler(temperature=args.temperature, top_k=args.top_k, top_p=args.top_p, min_p=args.min_p,
                       repetition_penalty=args.repetition_penalty, seed=args.seed)
    except ValueError as e:
        raise CLIError(str(e)) from None


# ---------------------------------------------------------------- info

def cmd_info(args) -> int:
    with Engine(args.model, **engine_kwargs(args)) as eng:
        info = {**eng.info, "kv_capacity": eng.kv_capacity}
    if args.json:
        print(json.dumps(info, indent=1, default=str))
    else:
        fields = ("arch", "n_layers", "d_model", "vocab_size", "n_experts", "top_k", "cache_slots", "kv_capacity")
        shown = " ".join(f"{k}={info[k]}" for k in fields)
        print(f"{Path(args.model).name}: {shown} params={info['params_total'] / 1e9:.2f}B "
              f"({info['params_active'] / 1e9:.2f}B active)")
    return 0


# ---------------------------------------------------------------- run

def _parse_ids(s: str) -> list[int]:
    parts = s.replace(",", " ").split()
    if not all(p.lstrip("+-").isdigit() for p in parts):
        raise CLIError(f"--ids must be integers separated by commas, got {s!r}")
    if not parts:
        raise CLIError("--ids is empty")
    return [int(p) for p in parts]


def cmd_run(args) -> int:
    mode = check_speculative(args.speculative, args.draft_len, args.ngram_n)
    sampler = _sampler_of(args)
    prompt = _parse_ids(args.ids)
    printing = not args.quiet and not args.json_out
    out: list[int] = []
    stats = None
    with Engine(args.model, **engine_kwargs(args)) as eng:
        if not all(0 <= t < eng.vocab_size for t in prompt):
            raise CLIError(f"prompt ids must be in [0, {eng.vocab_size})")
        stops = () if args.ignore_eos else tuple(eng.info["eos_ids"])
        for tok in generate(eng, prompt, args.max_tokens, sampler, stops, mode, args.draft_len, args.ngram_n):
            out.append(tok.id)
            stats = tok.stats
            if printing:
                print(tok.id, end=" ", flush=True)
    if printing:
        print()
    if args.json_out:
        doc = {"prompt_ids": prompt, "output_ids": out, "stats": stats.as_dict() if stats else {}}
        Path(args.json_out).write_text(json.dumps(doc, indent=1))
    if stats is not None and not args.quiet:
        print(f"[{stats.new_tokens} tokens, {stats.decode_tok_s:.1f} tok/s decode, {stats.forwards} forwards, "
              f"acceptance {stats.acceptance_rate:.1%}]", file=sys.stderr)
    return 0


# ---------------------------------------------------------------- bench

def bench_ids(kind: str, n: int, vocab: int, seed: int, offset: int = 0) -> list[int]:
    """The ids `bench` feeds (the reference's recipe, cli.py:400-404): seeded random ids,
    or the fixed sequence (i + offset) * 7919 + 13 mod vocab."""
    if kind == "random":
        return np.random.default_rng((seed, offset)).integers(0, vocab, size=n).tolist()
    i = np.arange(offset, offset + n, dtype=np.int64)
    return ((i * 7919 + 13) % vocab).tolist()


@dataclass
class _Timed:
    """Seconds and engine statistics of one measured phase."""
    seconds: float = 0.0
    stats: dict | None = None


def _timed(eng, fn) -> tuple[_Timed, object]:
    eng.reset_stats()
    t0 = time.perf_counter()
    value = fn()
    ph = _Timed(time.perf_counter() - t0)
    ph.stats = eng.stats()
    return ph, value


def _decode_plain(eng, args, V, first_logits) -> None:
    """gen_tokens single-token forwards: fed ids, or the argmax of the previous logits
    (--ids greedy, starting from the prompt's last logits)."""
    greedy = args.ids == "greedy"
    fed = bench_ids("fixed" if greedy else args.ids, args.gen_tokens, V, args.seed, offset=args.prompt_tokens)
    nxt = int(np.argmax(first_logits)) if greedy and first_logits is not None else None
    for i in range(args.gen_tokens):
        lg = eng.eval([nxt if nxt is not None else fed[i]])
        if greedy:
            nxt = int(np.argmax(lg))


def _decode_spec(eng, args, ctx, mode) -> dict:
    """gen_tokens greedy tokens by speculative decoding from the prefilled context (the
    engine holds ctx; generate() re-feeds its last token). Returns the verify block."""
    toks = list(generate(eng, ctx, args.gen_tokens, Sampler.greedy(), (), mode, args.draft_len, args.ngram_n,
                         held=ctx))
    if not toks:
        return {}
    st = toks[-1].stats
    return dict(speculative=mode, draft_len=args.draft_len, ngram_n=args.ngram_n, forwards=st.forwards,
                draft_steps=st.draft_steps, drafted=st.drafted, accepted=st.accepted,
                acceptance_rate=st.acceptance_rate, tokens_per_forward=st.tokens_per_forward)


def _rate(n: int, s: float) -> float:
    return n / s if s > 0 and n else 0.0


def cmd_bench(args) -> int:
    mode = check_speculative(args.speculative, args.draft_len, args.ngram_n)
    if mode != "none" and args.ids != "greedy":
        raise CLIError("--speculative needs --ids greedy (drafts are checked against the model's own continuation)")
    if mode != "none" and args.prompt_tokens < 1:
        raise CLIError("--speculative needs --prompt-tokens >= 1")
    feed = "fixed" if args.ids == "greedy" else args.ids
    with Engine(args.model, **engine_kwargs(args)) as eng:
        info, V = eng.info, eng.vocab_size
        total = args.warmup + args.prompt_tokens + args.gen_tokens
        if total > eng.kv_capacity:
            raise CLIError(f"warmup + prompt + gen = {total} tokens exceeds the KV capacity {eng.kv_capacity}; "
                           f"raise --max-seq or lower the token counts")
        if args.route_replay:
            eng.route_replay(args.route_replay)
        if args.trace:
            eng.trace_start(args.trace)
        ctx = bench_ids(feed, args.warmup, V, args.seed, offset=10_000_000) if args.warmup else []
        if ctx:
            eng.eval(ctx)
        prompt = bench_ids(feed, args.prompt_tokens, V, args.seed)
        ctx = ctx + prompt
        pre, logits = _timed(eng, lambda: eng.eval(prompt) if prompt else None)
        if mode == "none":
            dec, verify = _timed(eng, lambda: _decode_plain(eng, args, V, logits))[0], None
        else:
            dec, verify = _timed(eng, lambda: _decode_spec(eng, args, ctx, mode))
        if args.trace:
            eng.trace_stop()

    res = {
        "model": str(args.model), "arch": info.get("arch"), "params_total": info.get("params_total"),
        "params_active": info.get("params_active"), "isa": info.get("isa_name", "gfx950"),
        "threads": info.get("n_threads"), "io_threads": info.get("n_io_threads"), "cache_slots": info.get("cache_slots"),
        "options": engine_kwargs(args), "ids": args.ids, "route_replay": args.route_replay,
        "prefill_tokens": args.prompt_tokens, "prefill_s": pre.seconds,
        "prefill_tok_s": _rate(args.prompt_tokens, pre.seconds),
        "decode_tokens": args.gen_tokens, "decode_s": dec.seconds, "decode_tok_s": _rate(args.gen_tokens, dec.seconds),
        "prefill_stats": pre.stats, "decode_stats": dec.stats,
    }
    if verify is not None:
        res["verify"] = verify
    if args.json:
        print(json.dumps(res, indent=1, default=str))
    else:
        _print_bench(res, args)
    return 0


def _print_bench(res: dict, args) -> None:
    tag = " (routing replayed from trace: synthetic workload)" if args.route_replay else ""
    print(f"hearth_amd bench: {Path(args.model).name}  arch={res['arch']}  cache_slots={res['cache_slots']}{tag}")
    sp, sd = res["prefill_stats"], res["decode_stats"]
    if args.prompt_tokens:
        print(f"  prefill  {args.prompt_tokens:6d} tok  {res['prefill_s']:8.3f} s  {res['prefill_tok_s']:9.2f} tok/s  "
              f"hit {sp['hit_rate']:.1%}")
    if args.gen_tokens:
        print(f"  decode   {args.gen_tokens:6d} tok  {res['decode_s']:8.3f} s  {res['decode_tok_s']:9.2f} tok/s  "
              f"hit {sd['hit_rate']:.1%}  prefetch used {sd['prefetch_used']}/{sd['prefetch_issued']}")
        v = res.get("verify")
        if v:
            print(f"  verify   {v['forwards']} forwards, {v['accepted']}/{v['drafted']} drafts accepted "
                  f"({v['acceptance_rate']:.1%}), {v['tokens_per_forward']:.2f} tokens per forward")


# ---------------------------------------------------------------- parser

def build_parser() -> argparse.ArgumentParser:
    p = argparse.ArgumentParser(prog="hearth_amd", description="Speculative verification of MoE models on an MI355X.")
    sub = p.add_subparsers(dest="cmd", metavar="<command>")
    sub.required = True

    def command(name, fn, help_text):
        s = sub.add_parser(name, help=help_text)
        s.add_argument("model")
        s.set_defaults(fn=fn)
        return s

    s = command("info", cmd_info, "open a model container and print its engine info")
    s.add_argument("--json", action="store_true")
    add_engine_args(s)

    s = command("run", cmd_run, "generate from prompt token ids")
    s.add_argument("--ids", required=True, help="prompt as token ids, e.g. '1,17,42'")
    s.add_argument("--ignore-eos", action="store_true", help="do not stop at end-of-sequence tokens")
    s.add_argument("--json-out", metavar="PATH", help="write prompt/output ids and stats as JSON")
    s.add_argument("-q", "--quiet", action="store_true", help="no token or stats output")
    add_sampling_args(s, temperature=0.0, max_tokens=128)
    add_engine_args(s)

    s = command("bench", cmd_bench, "measure prefill/decode speed and speculative verification")
    s.add_argument("--prompt-tokens", type=int, default=128)
    s.add_argument("--gen-tokens", type=int, default=64)
    s.add_argument("--ids", choices=["random", "fixed", "greedy"], default="random",
                   help="token ids fed: seeded random, a fixed sequence, or greedy argmax feedback")
    s.add_argument("--seed", type=int, default=0)
    s.add_argument("--warmup", type=int, default=0, help="tokens evaluated before measuring")
    s.add_argument("--trace", metavar="OUT", help="record the routing trace")
    s.add_argument("--route-replay", metavar="TRACE", help="replay routing from a trace (synthetic containers)")
    s.add_argument("--json", action="store_true")
    add_spec_args(s.add_argument_group("speculative decoding (decode phase, with --ids greedy)"))
    add_engine_args(s)
    return p


def main(argv=None) -> int:
    args = build_parser().parse_args(argv)
    try:
        return args.fn(args)
    except (CLIError, HearthError, ValueError) as e:
        print(f"hearth_amd: error: {e}", file=sys.stderr)
        return 2
