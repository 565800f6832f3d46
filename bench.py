"""Speculative-verify throughput on one MI355X: the Qwen3-30B-A3B-shaped Q4/Q8 model,
greedy linear-chain verification with k = 8 drafts at a 4096-token context.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--layers 48] [--ctx 4096] [--k 8]

Workload (one step = one verify of [last] + k drafts: eval on the GPU, greedy
acceptance on the GPU, commit; generate.py:365-392 of the reference):
  - model: 48 layers, hidden 2048, 32 query / 4 KV heads of 128, 128 experts top-8 of
    FFN 768, vocab 151936; Q4 experts, Q8 attention / embedding / lm_head, F32 routers;
    random weights (synthetic, written to a .hearth container first);
  - context: a 4096-token random prompt prefilled before timing;
  - drafts: the model's own greedy continuation (computed by single-token decodes
    beforehand) with each draft replaced by a uniform random token with probability 0.3.
    Every step's accepted tokens are checked against that continuation, which also
    checks batch == sequential at full scale.
value = accepted tokens / s = sum over steps of (accepted drafts + 1) / wall time of the
steps (inputs already resident in HBM; each step returns its result to the host).

The roofline fields come from a second, profiled pass over the same steps (HIP events
around every launch group on the engine's stream): the dominant kernel class is the
grouped Q4 expert GEMM; its algorithmic bytes are the distinct experts each step's
routing touched times the slab bytes (2,506,752 per expert). cpu_baseline times the
reference engine itself (compiled from its C sources into oracle/_ref) on the host
cores on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "accepted tok/s, Qwen3-30B-A3B-shape verify k=8 (1 GPU); Q4 MoE HBM GB/s"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def model_path(layers: int, ctx: int, k: int) -> Path:
    from hearth_amd import container
    d = Path(os.environ.get("HEARTH_BENCH_DIR", tempfile.gettempdir())) / "hearth_bench"
    d.mkdir(parents=True, exist_ok=True)
    p = d / f"qwen3_30b_a3b_L{layers}.hearth"
    if not p.is_file():
        t = time.time()
        shape = container.Shape(**{**container.QWEN3_30B_A3B.__dict__, "max_seq": ctx + 1024})
        container.make_shaped(p.with_suffix(".tmp"), shape, seed=0, n_layers=layers)
        os.replace(p.with_suffix(".tmp"), p)
        log(f"[bench] wrote {p} ({p.stat().st_size / 1e9:.2f} GB) in {time.time() - t:.1f}s")
    return p


def make_drafts(cont, seed):
    """Drafts for each position: the continuation with p = 0.3 uniform replacements."""
    from hearth_amd import container
    n = len(cont)
    corrupt = container.uniforms(seed, n) < 0.3
    rnd = container.uniform_ints(seed + 1, n, container.QWEN3_30B_A3B.vocab)
    return np.where(corrupt, rnd, np.asarray(cont)).astype(np.int32)


def run_steps(eng, cont, noisy, base, k, steps, check=True):
    """steps verify calls from position base; returns (tokens per step, seconds per step)."""
    import time as _t
    pos = base
    toks, secs = [], []
    last = int(cont[0])
    for s in range(steps):
        i = pos - base            # index into the continuation of the token after `last`
        drafts = noisy[i + 1:i + 1 + k]
        if len(drafts) < k:
            raise RuntimeError("continuation too short for the requested steps")
        t0 = _t.perf_counter()
        path, final, _ = eng.verify_greedy(np.concatenate([[last], drafts]).astype(np.int32))
        secs.append(_t.perf_counter() - t0)
        n_acc = len(path) - 1
        if check:
            want = list(cont[i + 1:i + 1 + n_acc]) + [int(cont[i + 1 + n_acc])]
            got = [int(d) for d in drafts[:n_acc]] + [final]
            if got != want:
                raise RuntimeError(f"step {s}: verify emitted {got}, greedy decoding gives {want}")
        toks.append(n_acc + 1)
        pos += n_acc + 1
        last = final
    return toks, secs


def cpu_baseline(path: Path, prompt, noisy, cont, k: int, steps: int, threads: int):
    """The reference engine (oracle/_ref/libhearth_ref.so) on the same container: the
    prompt is prefilled, then `steps` greedy verify steps (eval all_logits + acceptance
    + rewind, generate.py:365-392) are timed."""
    ref = ROOT / "oracle" / "_ref" / "libhearth_ref.so"
    if not ref.is_file():
        return None
    from hearth_amd.engine import Engine
    e = Engine(path, lib=str(ref), threads=threads, cache_gb=64.0, prefetch="off", max_seq=len(prompt) + 512,
               max_batch=512)
    t = time.time()
    e.eval(prompt)
    prefill_s = time.time() - t
    base = e.pos
    last = int(cont[0])
    toks, secs = [], []
    for s in range(steps):
        i = e.pos - base
        drafts = noisy[i + 1:i + 1 + k]
        t0 = time.perf_counter()
        rows = e.eval(np.concatenate([[last], drafts]).astype(np.int32), all_logits=True)
        n_acc, final = 0, None
        for j, d in enumerate(drafts):
            a = int(np.argmax(rows[j]))
            if a != int(d):
                final = a
                break
            n_acc += 1
        if final is None:
            final = int(np.argmax(rows[k]))
        e.rewind(base + i + 1 + n_acc)
        secs.append(time.perf_counter() - t0)
        toks.append(n_acc + 1)
        last = final
    e.close()
    return dict(value=sum(toks) / sum(secs), unit="tok/s", cores=threads, kind="reference",
                sample=f"reference engine built from its C sources, {threads} threads, same 48-layer container and "
                       f"{len(prompt)}-token context, {steps} verify steps after prefill "
                       f"(prefill {prefill_s:.1f}s untimed); {sum(secs) / steps * 1e3:.1f} ms/step")


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="speculative-verify throughput on one MI355X")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--k", type=int, default=8)
    ap.add_argument("--cpu-steps", type=int, default=6)
    ap.add_argument("--no-cpu", action="store_true")
    a = ap.parse_args(argv)
    if a.gpus != 1:
        print(f"bench.py runs on exactly one GPU: this build has no multi-GPU path (asked for {a.gpus})",
              file=sys.stderr)
        return 2
    from hearth_amd import container
    from hearth_amd.engine import Engine

    path = model_path(a.layers, a.ctx, a.k)
    prompt = container.uniform_ints(1234, a.ctx, container.QWEN3_30B_A3B.vocab).astype(np.int32)
    need = (a.warmup + a.steps) * (a.k + 1) + a.k + 2
    t = time.time()
    eng = Engine(path, max_seq=a.ctx + need + 16, max_batch=512)
    log(f"[bench] open {time.time() - t:.1f}s")
    # the engine holds prompt[:-1]; prompt[-1] is the first token a verify step feeds
    # (generate.py keeps engine.pos == len(seq) - 1)
    t = time.time()
    eng.eval(prompt[:-1])
    log(f"[bench] prefill {a.ctx - 1} tokens {time.time() - t:.1f}s")
    base = eng.pos
    # the model's greedy continuation by single-token decodes
    t = time.time()
    cont = [int(prompt[-1])]
    for _ in range(need):
        cont.append(int(np.argmax(eng.eval([cont[-1]]))))
    log(f"[bench] greedy continuation of {need} tokens {time.time() - t:.1f}s")
    eng.rewind(base)
    noisy = make_drafts(cont, seed=99)
    # warmup + timed
    run_steps(eng, cont, noisy, base, a.k, a.warmup)
    eng.rewind(base)
    eng.reset_stats()
    toks, secs = run_steps(eng, cont, noisy, base, a.k, a.warmup + a.steps)
    toks, secs = toks[a.warmup:], secs[a.warmup:]
    st = eng.stats()
    value = sum(toks) / sum(secs)
    ms = sorted(s * 1e3 for s in secs)
    log(f"[bench] {a.steps} steps: {value:.1f} tok/s, {sum(toks) / a.steps:.2f} tok/step, "
        f"p50 {statistics.median(ms):.3f} ms")
    # profiled pass over the same steps
    eng.rewind(base)
    eng.set_profiling(True)
    eng.reset_kstats()
    eng.reset_stats()
    ptoks, psecs = run_steps(eng, cont, noisy, base, a.k, a.warmup + a.steps)
    ks = eng.kstats()
    pst = eng.stats()
    eng.set_profiling(False)
    n_prof = a.warmup + a.steps
    expert_gbs = ks["expert_bytes"] / ks["expert_s"] / 1e9 if ks["expert_s"] > 0 else 0.0
    L, D, V = a.layers, 2048, 151936
    dense_bytes_step = L * (4096 * 2112 + 2 * 512 * 2112 + 2048 * 4224) + V * 2112
    dense_gbs = dense_bytes_step * n_prof / (ks["attn_s"] + ks["head_s"]) / 1e9 if ks["attn_s"] > 0 else 0.0
    per_launch_bytes = ks["expert_bytes"] / max(1, ks["expert_launches"])
    per_launch_s = ks["expert_s"] / max(1, ks["expert_launches"])
    eng.close()
    cpu = None
    if not a.no_cpu:
        try:
            cpu = cpu_baseline(path, prompt[:-1], noisy, cont, a.k, a.cpu_steps, threads=os.cpu_count() or 1)
        except Exception as ex:   # the baseline is reported, never required
            log(f"[bench] cpu baseline failed: {ex}")
    gpu_total = sum(ks[x] for x in ("attn_s", "router_s", "expert_s", "norm_s", "head_s", "dense_s"))
    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "tok/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(sum(secs) / a.steps * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": f"Qwen3-30B-A3B-shaped Q4/Q8 greedy chain verify k={a.k} at context {a.ctx}, "
                               f"drafts = greedy continuation with 30% random replacement", "layers": a.layers,
                   "ctx": a.ctx, "k": a.k, "tokens_per_step": round(sum(toks) / a.steps, 3),
                   "step_ms_p50": round(statistics.median(ms), 4), "step_ms_p90": round(ms[int(0.9 * (len(ms) - 1))], 4),
                   "expert_loads_per_step": round(st["expert_loads_unique"] / a.steps, 1)},
        "roofline": {"bound": "hbm", "achieved": round(expert_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(expert_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "grouped Q4 expert GEMM (gate/up + down)",
                     "bytes_per_launch": int(per_launch_bytes), "s_per_launch": per_launch_s},
        "gpu_time_split": {k: round(ks[k] / n_prof * 1e3, 4) for k in ("attn_s", "router_s", "expert_s", "norm_s", "head_s")}
                          | {"sum_ms": round(gpu_total / n_prof * 1e3, 4),
                             "dense_matvec_gbs": round(dense_gbs, 1)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
