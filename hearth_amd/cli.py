"""`python -m hearth_amd <command>`: the verify engine's command line.

`bench` keeps the JSON keys of the reference's `hearth bench` (python/hearth/cli.py:
408-474, arguments at cli.py:705-717 and the engine options of cli.py:27-53) and adds
the verify-step fields of a speculative decode (`--speculative ngram`): forwards,
drafted, accepted, acceptance rate and tokens per forward. `run` generates from token
ids (`--ids 1,17,42`) with the sampling and speculative options of cli.py:56-73;
`info` prints a container's engine info. Text front ends (tokenizer, chat template,
HTTP server) are not part of this package.
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

import numpy as np

from .engine import Engine, HearthError
from .generate import Sampler, check_speculative, generate


class CLIError(Exception):
    """A user-facing error: printed without a traceback, exit status 2."""


def add_engine_args(p: argparse.ArgumentParser) -> None:
    g = p.add_argument_group("engine")
    g.add_argument("--cache-gb", type=float, default=8.0, help="budget for routed experts in GiB (default 8)")
    g.add_argument("--threads", type=int, default=0, help="host threads (0 = default)")
    g.add_argument("--io-threads", type=int, default=0, help="expert reader threads (0 = default)")
    g.add_argument("--buffered", action="store_true", help="use the OS page cache instead of direct I/O")
    g.add_argument("--policy", choices=["lru", "lfu"], default="lfu", help="expert cache eviction policy")
    g.add_argument("--prefetch", choices=["off", "next", "shared"], default="shared", help="next-layer prefetch mode")
    g.add_argument("--prefetch-extra", type=int, default=0, help="predict top_k + N experts for the next layer")
    g.add_argument("--usage-in", metavar="PATH", help="heat profile to seed the cache")
    g.add_argument("--usage-out", metavar="PATH", help="write the heat profile here on close")
    g.add_argument("--pin-fraction", type=float, default=0.0, help="fraction of cache slots pinned at open")
    g.add_argument("--warm-start", action="store_true", help="fill the cache with the hottest experts at open")
    g.add_argument("--max-seq", type=int, default=0, help="KV capacity in tokens (0 = min(model, 4096))")
    g.add_argument("--max-batch", type=int, default=0, help="max tokens per forward chunk (0 = default)")
    g.add_argument("--isa", choices=["auto", "scalar", "avx2", "avx512"], default="auto")
    g.add_argument("--mirror", action="append", default=[], metavar="PATH", help="byte-identical model copy")
    g.add_argument("-v", "--verbose", action="count", default=0, help="engine log level")


def engine_kwargs(args) -> dict:
    return dict(cache_gb=args.cache_gb, threads=args.threads, io_threads=args.io_threads,
                direct_io=not args.buffered, policy=args.policy, prefetch=args.prefetch,
                prefetch_extra=args.prefetch_extra, usage_in=args.usage_in, usage_out=args.usage_out,
                pin_fraction=args.pin_fraction, warm_start=args.warm_start, max_seq=args.max_seq,
                max_batch=args.max_batch, isa=args.isa, mirrors=list(args.mirror), verbose=args.verbose)


def add_spec_args(g) -> None:
    g.add_argument("--speculative", choices=["none", "ngram"], default="none",
                   help="prompt-lookup speculative decoding, verified on the GPU (lossless)")
    g.add_argument("--draft-len", type=int, default=4, help="max draft tokens per forward (default 4)")
    g.add_argument("--ngram-n", type=int, default=3, help="longest n-gram matched for drafting (default 3)")


def add_sampling_args(p: argparse.ArgumentParser, temperature: float, max_tokens: int) -> None:
    g = p.add_argument_group("sampling")
    g.add_argument("-n", "--max-tokens", type=int, default=max_tokens, help=f"tokens to generate (default {max_tokens})")
    g.add_argument("--temperature", type=float, default=temperature, help=f"0 = greedy (default {temperature})")
    g.add_argument("--top-k", type=int, default=0)
    g.add_argument("--top-p", type=float, default=1.0)
    g.add_argument("--min-p", type=float, default=0.0)
    g.add_argument("--repetition-penalty", type=float, default=1.0)
    g.add_argument("--seed", type=int, default=None)
    add_spec_args(g)


def bench_ids(kind: str, n: int, vocab: int, seed: int, offset: int = 0) -> list[int]:
    """The token ids `bench` feeds (cli.py:400-404): seeded random ids, or the fixed
    sequence (i + offset) * 7919 + 13 mod vocab."""
    if kind == "random":
        return np.random.default_rng((seed, offset)).integers(0, vocab, size=n).tolist()
    return [((i + offset) * 7919 + 13) % vocab for i in range(n)]


def cmd_info(args) -> int:
    with Engine(args.model, **engine_kwargs(args)) as eng:
        info = dict(eng.info)
        info["kv_capacity"] = eng.kv_capacity
    if args.json:
        print(json.dumps(info, indent=1, default=str))
        return 0
    print(f"{Path(args.model).name}: arch={info['arch']} layers={info['n_layers']} d_model={info['d_model']} "
          f"vocab={info['vocab_size']} experts={info['n_experts']} top_k={info['top_k']} "
          f"params={info['params_total'] / 1e9:.2f}B ({info['params_active'] / 1e9:.2f}B active) "
          f"cache_slots={info['cache_slots']} kv_capacity={info['kv_capacity']}")
    return 0


def cmd_bench(args) -> int:
    mode = check_speculative(args.speculative, args.draft_len, args.ngram_n)
    if mode != "none" and args.ids != "greedy":
        raise CLIError("--speculative needs --ids greedy (drafts are checked against the model's own continuation)")
    with Engine(args.model, **engine_kwargs(args)) as eng:
        info = eng.info
        V = int(info["vocab_size"])
        total = args.warmup + args.prompt_tokens + args.gen_tokens
        if total > eng.kv_capacity:
            raise CLIError(f"warmup + prompt + gen = {total} tokens exceeds the KV capacity {eng.kv_capacity}; "
                           f"raise --max-seq or lower the token counts")
        if mode != "none" and args.prompt_tokens < 1:
            raise CLIError("--speculative needs --prompt-tokens >= 1")
        if args.route_replay:
            eng.route_replay(args.route_replay)
        if args.trace:
            eng.trace_start(args.trace)
        feed = "fixed" if args.ids == "greedy" else args.ids
        ctx: list[int] = []
        if args.warmup:
            ctx = bench_ids(feed, args.warmup, V, args.seed, offset=10_000_000)
            eng.eval(ctx)
        prompt = bench_ids(feed, args.prompt_tokens, V, args.seed)
        ctx += prompt
        eng.reset_stats()
        t0 = time.perf_counter()
        logits = eng.eval(prompt) if prompt else None
        prefill_s = time.perf_counter() - t0
        sp = eng.stats()
        eng.reset_stats()
        verify = None
        if mode != "none":
            # the engine holds ctx; generate() re-feeds its last token and decodes from there
            t0 = time.perf_counter()
            toks = list(generate(eng, ctx, args.gen_tokens, Sampler.greedy(), (), mode, args.draft_len, args.ngram_n,
                                 held=ctx))
            decode_s = time.perf_counter() - t0
            st = toks[-1].stats if toks else None
            verify = {} if st is None else dict(
                speculative=mode, draft_len=args.draft_len, ngram_n=args.ngram_n, forwards=st.forwards,
                draft_steps=st.draft_steps, drafted=st.drafted, accepted=st.accepted,
                acceptance_rate=st.acceptance_rate, tokens_per_forward=st.tokens_per_forward)
        else:
            dec = bench_ids(feed, args.gen_tokens, V, args.seed, offset=args.prompt_tokens)
            nxt = int(np.argmax(logits)) if (args.ids == "greedy" and logits is not None) else None
            t0 = time.perf_counter()
            for i in range(args.gen_tokens):
                tok = nxt if nxt is not None else dec[i]
                lg = eng.eval([tok])
                if args.ids == "greedy":
                    nxt = int(np.argmax(lg))
            decode_s = time.perf_counter() - t0
        sd = eng.stats()
        if args.trace:
            eng.trace_stop()

    res = {
        "model": str(args.model), "arch": info.get("arch"), "params_total": info.get("params_total"),
        "params_active": info.get("params_active"), "isa": info.get("isa_name", "gfx950"),
        "threads": info.get("n_threads"), "io_threads": info.get("n_io_threads"), "cache_slots": info.get("cache_slots"),
        "options": engine_kwargs(args), "ids": args.ids, "route_replay": args.route_replay,
        "prefill_tokens": args.prompt_tokens, "prefill_s": prefill_s,
        "prefill_tok_s": args.prompt_tokens / prefill_s if prefill_s > 0 and args.prompt_tokens else 0.0,
        "decode_tokens": args.gen_tokens, "decode_s": decode_s,
        "decode_tok_s": args.gen_tokens / decode_s if decode_s > 0 and args.gen_tokens else 0.0,
        "prefill_stats": sp, "decode_stats": sd,
    }
    if verify is not None:
        res["verify"] = verify
    if args.json:
        print(json.dumps(res, indent=1, default=str))
        return 0
    label = " (routing replayed from trace: synthetic workload)" if args.route_replay else ""
    print(f"hearth_amd bench: {Path(args.model).name}  arch={res['arch']}  cache_slots={res['cache_slots']}{label}")
    if args.prompt_tokens:
        print(f"  prefill  {args.prompt_tokens:6d} tok  {prefill_s:8.3f} s  {res['prefill_tok_s']:9.2f} tok/s  "
              f"hit {sp['hit_rate']:.1%}")
    if args.gen_tokens:
        print(f"  decode   {args.gen_tokens:6d} tok  {decode_s:8.3f} s  {res['decode_tok_s']:9.2f} tok/s  "
              f"hit {sd['hit_rate']:.1%}  prefetch used {sd['prefetch_used']}/{sd['prefetch_issued']}")
        if verify:
            print(f"  verify   {verify['forwards']} forwards, {verify['accepted']}/{verify['drafted']} drafts accepted "
                  f"({verify['acceptance_rate']:.1%}), {verify['tokens_per_forward']:.2f} tokens per forward")
    return 0


def _parse_ids(s: str) -> list[int]:
    try:
        ids = [int(x) for x in s.replace(",", " ").split()]
    except ValueError:
        raise CLIError(f"--ids must be integers separated by commas, got {s!r}") from None
    if not ids:
        raise CLIError("--ids is empty")
    return ids


def cmd_run(args) -> int:
    mode = check_speculative(args.speculative, args.draft_len, args.ngram_n)
    try:
        sampler = Sampler(temperature=args.temperature, top_k=args.top_k, top_p=args.top_p, min_p=args.min_p,
                          repetition_penalty=args.repetition_penalty, seed=args.seed)
    except ValueError as e:
        raise CLIError(str(e)) from None
    prompt = _parse_ids(args.ids)
    with Engine(args.model, **engine_kwargs(args)) as eng:
        V = eng.vocab_size
        if min(prompt) < 0 or max(prompt) >= V:
            raise CLIError(f"prompt ids must be in [0, {V})")
        stop = () if args.ignore_eos else tuple(eng.info["eos_ids"])
        out, st = [], None
        for t in generate(eng, prompt, args.max_tokens, sampler, stop, mode, args.draft_len, args.ngram_n):
            out.append(t.id)
            st = t.stats
            if not args.quiet and not args.json_out:
                print(t.id, end=" ", flush=True)
    if not args.quiet and not args.json_out:
        print()
    stats = st.as_dict() if st is not None else {}
    if args.json_out:
        Path(args.json_out).write_text(json.dumps({"prompt_ids": prompt, "output_ids": out, "stats": stats}, indent=1))
    if not args.quiet and st is not None:
        print(f"[{st.new_tokens} tokens, {st.decode_tok_s:.1f} tok/s decode, {st.forwards} forwards, "
              f"acceptance {st.acceptance_rate:.1%}]", file=sys.stderr)
    return 0


def build_parser() -> argparse.ArgumentParser:
    p = argparse.ArgumentParser(prog="hearth_amd", description="Speculative verification of MoE models on an MI355X.")
    sub = p.add_subparsers(dest="cmd", metavar="<command>")
    sub.required = True

    s = sub.add_parser("info", help="open a model container and print its engine info")
    s.add_argument("model")
    s.add_argument("--json", action="store_true")
    add_engine_args(s)
    s.set_defaults(fn=cmd_info)

    s = sub.add_parser("run", help="generate from prompt token ids")
    s.add_argument("model")
    s.add_argument("--ids", required=True, help="prompt as token ids, e.g. '1,17,42'")
    s.add_argument("--ignore-eos", action="store_true", help="do not stop at end-of-sequence tokens")
    s.add_argument("--json-out", metavar="PATH", help="write prompt/output ids and stats as JSON")
    s.add_argument("-q", "--quiet", action="store_true", help="no token or stats output")
    add_sampling_args(s, temperature=0.0, max_tokens=128)
    add_engine_args(s)
    s.set_defaults(fn=cmd_run)

    s = sub.add_parser("bench", help="measure prefill/decode speed and speculative verification")
    s.add_argument("model")
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
    s.set_defaults(fn=cmd_bench)
    return p


def main(argv=None) -> int:
    args = build_parser().parse_args(argv)
    try:
        return args.fn(args)
    except (CLIError, HearthError, ValueError) as e:
        print(f"hearth_amd: error: {e}", file=sys.stderr)
        return 2
