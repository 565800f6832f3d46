"""Speculative-verify throughput on one MI355X: the Qwen3-30B-A3B-shaped Q4/Q8 model,
greedy linear-chain verification with k = 8 drafts at a 4096-token context.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--layers 48] [--ctx 4096] [--k 8]
    python bench.py --workload {chain,tree,experts,dsv3,generate}

The default workload (chain) is described below; the others print their own JSON line:
  tree     the same model, one 4x4x4 draft tree (85 nodes) per step at a 2048-token
           context, stochastic acceptance at temperature 0.8 / top-p 0.95 against
           draft distributions q = softmax(N(0, 2)) (q travels from host memory);
  experts  the grouped Q4 expert kernels alone at T = 1, 9, 33, 65 tokens with Zipf(1.1)
           routing replayed from a trace: GB/s and int8 MFMA rate per T;
  dsv3     the DeepSeek-V3 shape (MLA, 256 experts top-8 + shared, 3 dense + 20 MoE
           layers), chain verify k = 8 at 4096, with the experts streamed from pinned
           host memory through an HBM cache below the expert set (and resident, for
           comparison);
  generate the same model, greedy generation of --gen tokens after a 4096-token prompt
           with prompt-lookup drafts (k = 8, n-grams up to 3): generate() with the
           device loop (drafting, verify, acceptance and stop/length rules on the GPU,
           no host round trip per step) against the host steps (one verify call per
           step); both must yield the same tokens.

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

roofline: the grouped Q4 expert gate/up kernel (k_expert_tk<4, TK_GATEUP_Q>: gate and up,
SwiGLU and the act-quant of its rows; k_expert_tk<4, 2> in rocprofv3 traces), timed with HIP
event pairs recorded on the engine's stream around each of its launches during the
timed steps; achieved = its algorithmic bytes (distinct experts routed in the layer x
1,671,168 B of Q4 gate+up rows each) / its summed launch durations. A second pass over
the same steps with events around every launch group gives the per-phase GPU time
split. cpu_baseline times the reference engine itself (compiled from its C sources into
oracle/_ref) on up to 16 host cores on a bounded sample of the same workload.
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


TRAFFIC_PROFILE = ROOT / "profiles" / "k_expert_tk_gateup_verify_k8_ctx4096_traffic.md"


def measured_traffic():
    """HBM bytes per launch of the roofline kernel from its committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (copy-calibrated), or None."""
    try:
        for line in TRAFFIC_PROFILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


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


def run_steps(eng, cont, noisy, base, k, steps, check=True, before=None):
    """steps verify calls from position base; returns (tokens per step, seconds per step).
    before(s), when given, runs ahead of step s outside its timing."""
    import time as _t
    pos = base
    toks, secs = [], []
    last = int(cont[0])
    for s in range(steps):
        if before is not None:
            before(s)
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
    cpus, phys = host_cpus()
    return dict(value=sum(toks) / sum(secs), unit="tok/s", cores=threads, kind="reference",
                host_cpus=cpus, host_physical_cores=phys,
                sample=f"reference engine built from its C sources, {threads} threads (this process may use "
                       f"{cpus} CPUs; the host has {phys} physical cores), same 48-layer container and "
                       f"{len(prompt)}-token context, {steps} verify steps after prefill "
                       f"(prefill {prefill_s:.1f}s untimed); {sum(secs) / steps * 1e3:.1f} ms/step")


def host_cpus():
    """(CPUs this process may run on, distinct physical cores listed in /proc/cpuinfo)"""
    try:
        cpus = len(os.sched_getaffinity(0))
    except AttributeError:
        cpus = os.cpu_count() or 1
    cores, phys, core = set(), None, None
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k = k.strip()
            if k == "physical id":
                phys = v.strip()
            elif k == "core id":
                core = v.strip()
            elif not k and core is not None:
                cores.add((phys, core))
                phys = core = None
        if core is not None:
            cores.add((phys, core))
    except OSError:
        pass
    return cpus, len(cores) or None


def summarize_trace(path: str, nsteps: int, last_kernel: str = "k_accept_walk") -> int:
    """Per-verify-step kernel table from a rocprofv3 --kernel-trace CSV (run_kernel_trace.csv):
    a step is the dispatches after one `last_kernel` (the acceptance's last kernel:
    k_accept_walk greedy, k_sample_walk sampled) up to and including the next; the
    last nsteps steps are averaged."""
    import collections
    import csv
    import re
    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    ends = [i for i, r in enumerate(rows) if last_kernel in r["Kernel_Name"]]
    steps = [rows[a + 1:b + 1] for a, b in zip(ends[:-1], ends[1:])][-nsteps:]
    if not steps:
        print("no verify steps in the trace")
        return 1
    tot, cnt = collections.defaultdict(float), collections.Counter()
    wall = busy = 0.0
    for s in steps:
        wall += (int(s[-1]["End_Timestamp"]) - int(s[0]["Start_Timestamp"])) / 1e3
        for r in s:
            d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            name = re.sub(r"\(.*", "", r["Kernel_Name"].replace("(anonymous namespace)::", ""))
            tot[name] += d
            cnt[name] += 1
            busy += d
    n = len(steps)
    print(f"{n} verify steps: first dispatch to last end {wall / n:.1f} us/step, kernel time {busy / n:.1f} us/step")
    print(f"{'kernel':34s} {'us/step':>10s} {'calls/step':>10s} {'avg us':>9s}")
    for k, v in sorted(tot.items(), key=lambda x: -x[1]):
        print(f"{k:34s} {v / n:10.1f} {cnt[k] / n:10.1f} {v / cnt[k]:9.2f}")
    return 0


def calibrate_copy(mib: int) -> int:
    """Device-to-device copies of a known size through the HIP runtime (the copy kernel
    reads and writes mib MiB per dispatch), to scale FETCH_SIZE / WRITE_SIZE counters."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    n = mib << 20
    src, dst = ctypes.c_void_p(), ctypes.c_void_p()
    for p in (src, dst):
        if hip.hipMalloc(ctypes.byref(p), ctypes.c_size_t(n)) != 0:
            raise RuntimeError("hipMalloc failed")
    try:
        if hip.hipMemset(src, 1, ctypes.c_size_t(n)) != 0:
            raise RuntimeError("hipMemset failed")
        for _ in range(3):
            if hip.hipMemcpy(dst, src, ctypes.c_size_t(n), 3) != 0:   # hipMemcpyDeviceToDevice
                raise RuntimeError("hipMemcpy failed")
        if hip.hipDeviceSynchronize() != 0:
            raise RuntimeError("hipDeviceSynchronize failed")
    finally:
        hip.hipFree(src)
        hip.hipFree(dst)
    print(f"copied {mib} MiB device to device 3 times")
    return 0


def bench_chain(a) -> dict:
    """Qwen3-30B-A3B shape, greedy chain verify k=8 at a 4096-token context (the
    headline workload)."""
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
    # warmup, then the timed steps (no instrumentation)
    run_steps(eng, cont, noisy, base, a.k, a.warmup)
    eng.rewind(base)      # the timed steps re-verify from the same position
    eng.reset_stats()
    toks, secs = run_steps(eng, cont, noisy, base, a.k, a.steps)
    st = eng.stats()
    value = sum(toks) / sum(secs)
    ms = sorted(s * 1e3 for s in secs)
    log(f"[bench] {a.steps} steps: {value:.1f} tok/s, {sum(toks) / a.steps:.2f} tok/step, "
        f"p50 {statistics.median(ms):.3f} ms")
    # the same steps again with HIP event pairs around the grouped expert launches only:
    # the roofline kernel's launch durations
    eng.rewind(base)
    eng.set_profiling(1)
    eng.reset_kstats()
    _, secs_ev = run_steps(eng, cont, noisy, base, a.k, a.steps)
    kx = eng.kstats()
    eng.set_profiling(0)
    # a second pass over the same steps with events around every launch group: the
    # per-phase split (reported, not used for value or roofline)
    eng.rewind(base)
    eng.set_profiling(2)
    eng.reset_kstats()
    run_steps(eng, cont, noisy, base, a.k, a.steps)
    ks = eng.kstats()
    eng.set_profiling(0)
    n_launch = max(1, kx["expert_launches"])
    gu_gbs = kx["expert_bytes"] / kx["expert_s"] / 1e9 if kx["expert_s"] > 0 else 0.0
    dn_gbs = kx["expert_down_bytes"] / kx["expert_down_s"] / 1e9 if kx["expert_down_s"] > 0 else 0.0
    # every weight matrix a step reads once (attention projections, lm_head, the routed
    # experts' gate/up/down) over the GPU time of the launches that read them
    mat_bytes = ks["dense_bytes"] + ks["expert_bytes"] + ks["expert_down_bytes"]
    mat_s = ks["proj_s"] + ks["expert_s"] + ks["expert_down_s"] + ks["head_s"] + ks["dense_s"]
    eng.close()
    cpu = None
    if not a.no_cpu:
        try:
            cpu = cpu_baseline(path, prompt[:-1], noisy, cont, a.k, a.cpu_steps, threads=host_threads())
        except Exception as ex:   # the baseline is reported, never required
            log(f"[bench] cpu baseline failed: {ex}")
    phases = ("proj_s", "attn_s", "router_s", "expert_s", "expert_down_s", "norm_s", "head_s", "dense_s")
    gpu_total = sum(ks[x] for x in phases)
    return {
        "metric": METRIC, "value": round(value, 2), "unit": "tok/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(sum(secs) / a.steps * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": f"Qwen3-30B-A3B-shaped Q4/Q8 greedy chain verify k={a.k} at context {a.ctx}, "
                               f"drafts = greedy continuation with 30% random replacement", "layers": a.layers,
                   "ctx": a.ctx, "k": a.k, "tokens_per_step": round(sum(toks) / a.steps, 3),
                   "step_ms_p50": round(statistics.median(ms), 4), "step_ms_p90": round(ms[int(0.9 * (len(ms) - 1))], 4),
                   "expert_loads_per_step": round(st["expert_loads_unique"] / a.steps, 1),
                   "ms_per_step_with_expert_events": round(sum(secs_ev) / a.steps * 1e3, 4)},
        "roofline": {"bound": "hbm", "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "traffic_source": str(TRAFFIC_PROFILE.relative_to(ROOT)),
                     "kernel": "k_expert_tk<4, TK_GATEUP_Q> (grouped Q4 expert gate+up, SwiGLU, act-quant)",
                     "bytes_per_launch": int(kx["expert_bytes"] / n_launch),
                     "us_per_launch": round(kx["expert_s"] / n_launch * 1e6, 3),
                     "down_projection_gbs": round(dn_gbs, 1),
                     "matvec_aggregate": {
                         "achieved": round(mat_bytes / mat_s / 1e9, 1) if mat_s > 0 else 0.0,
                         "frac": round(mat_bytes / mat_s / 1e9 / HBM_PEAK_GBS, 4) if mat_s > 0 else 0.0,
                         "bytes_per_step": int(mat_bytes / a.steps),
                         "what": "all weight matrices of a step (attention q/k/v/o, lm_head, routed experts "
                                 "gate/up/down, with SwiGLU and act-quant epilogues) / GPU time of the "
                                 "launches that read them (HIP events around each launch group)"}},
        "gpu_time_split_ms_per_step": {k: round(ks[k] / a.steps * 1e3, 4) for k in phases}
                                      | {"sum": round(gpu_total / a.steps * 1e3, 4)},
        "cpu_baseline": cpu,
    }


def host_threads() -> int:
    """host cores for the CPU baseline: this process's CPU share (at most 16)"""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def tree_4x4x4() -> np.ndarray:
    """parent indices of the 85-node tree: root, 4 children, 16 grandchildren, 64 leaves"""
    parent, level = [-1], [0]
    for _ in range(3):
        nxt = []
        for p in level:
            for _ in range(4):
                parent.append(p)
                nxt.append(len(parent) - 1)
        level = nxt
    return np.array(parent, dtype=np.int32)


def bench_tree(a) -> dict:
    """Qwen3-30B-A3B shape, one 4x4x4 draft tree (85 nodes) per step over a 2048-token
    context, stochastic acceptance at temperature 0.8 / top-p 0.95 against draft
    distributions q = softmax(N(0, 2) logits), seeded uniforms."""
    from hearth_amd import container
    from hearth_amd.engine import Engine, make_sampler

    ctx = 2048
    V = container.QWEN3_30B_A3B.vocab
    path = model_path(a.layers, 4096, a.k)
    parent = tree_4x4x4()
    n = len(parent)
    rng = np.random.default_rng(2024)
    n_sets = 4
    qs, drafts = [], []
    for _ in range(n_sets):     # draft distributions and tokens drawn from them (children of node p ~ q[p])
        z = rng.standard_normal((n, V)) * 2.0
        q = np.exp(z - z.max(1, keepdims=True))
        q /= q.sum(1, keepdims=True)
        cdf = np.cumsum(q, 1)
        d = np.zeros(n, dtype=np.int32)
        for c in range(1, n):
            d[c] = min(int(np.searchsorted(cdf[parent[c]], rng.random() * cdf[parent[c], -1], "right")), V - 1)
        qs.append(q)
        drafts.append(d)
    smp = make_sampler(temperature=0.8, top_p=0.95)
    prompt = container.uniform_ints(4321, ctx, V).astype(np.int32)
    total = a.warmup + a.steps
    eng = Engine(path, max_seq=ctx + total * n + 64, max_batch=512)
    eng.eval(prompt[:-1])
    last = int(prompt[-1])
    # the draft distributions live in HBM, as a draft model on the same GPU leaves them
    # (hearth_gpu_verify_sample_dq): uploaded once, before the timed steps
    qd = [eng.device_array(q) for q in qs]

    def step(s):
        toks = drafts[s % n_sets].copy()
        toks[0] = last
        u = container.uniforms(7000 + s, 2 * n)
        t0 = time.perf_counter()
        p, fin, _ = eng.verify_sample(toks, parent, smp, q=qd[s % n_sets], u=u)
        return p, fin, time.perf_counter() - t0

    for s in range(a.warmup):
        p, last, _ = step(s)
    toks, secs = [], []
    for s in range(a.warmup, total):
        p, last, dt = step(s)
        toks.append(len(p))
        secs.append(dt)
    eng.close()
    value = sum(toks) / sum(secs)
    ms = sorted(x * 1e3 for x in secs)
    log(f"[bench] tree: {value:.1f} tok/s, {sum(toks) / a.steps:.2f} tok/step, p50 {statistics.median(ms):.3f} ms")
    return {
        "metric": "accepted tok/s, Qwen3-30B-A3B-shape 4x4x4 tree verify, sampled acceptance (1 GPU)",
        "value": round(value, 2), "unit": "tok/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(sum(secs) / a.steps * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "Qwen3-30B-A3B-shaped Q4/Q8 tree verify (4x4x4, 85 nodes) at context 2048, "
                               "rejection sampling at temperature 0.8 / top-p 0.95, q = softmax(N(0,2)) per node",
                   "layers": a.layers, "ctx": ctx, "nodes": n, "tokens_per_step": round(sum(toks) / a.steps, 3),
                   "step_ms_p50": round(statistics.median(ms), 4),
                   "q_bytes_per_step": int(n * V * 8),
                   "note": "q [85][151936] float64 (103 MB) per step is read in place from HBM "
                           "(hearth_gpu_verify_sample_dq); handing it over from host memory instead adds its "
                           "PCIe copy to every step"},
    }


def bench_experts(a) -> dict:
    """The routed-expert kernels alone at the Qwen3-30B-A3B shape (128 experts, gate/up
    2048 -> 768, down 768 -> 2048, Q4): T tokens per forward with Zipf(1.1) routing
    replayed from a trace, on the 48-layer model; per T the grouped gate/up and down
    launches are timed with HIP events."""
    from hearth_amd import container
    from hearth_amd.engine import Engine

    sh = container.QWEN3_30B_A3B
    path = model_path(a.layers, 4096, a.k)
    n_moe = a.layers
    d = Path(tempfile.mkdtemp())
    res = {}
    gu_bytes = 2 * sh.expert_ffn * (sh.d_model // 64) * 34     # one expert's Q4 gate + up
    dn_bytes = sh.d_model * (sh.expert_ffn // 64) * 34
    with Engine(path, max_seq=4096, max_batch=512) as eng:
        base_toks = container.uniform_ints(99, 256, sh.vocab).astype(np.int32)
        eng.eval(base_toks)
        base = eng.pos
        for T in (1, 9, 33, 65):
            ids = container.zipf_routes(1000 + T, 4096, n_moe, sh.n_experts, sh.top_k)
            tr = container.write_route_trace(d / f"zipf{T}.hrtr", ids, a.layers, sh.n_experts)
            eng.route_replay(tr)
            toks = container.uniform_ints(300 + T, T, sh.vocab).astype(np.int32)
            reps = 20
            for _ in range(3):
                eng.eval(toks)
                eng.rewind(base)
            eng.set_profiling(1)
            eng.reset_kstats()
            eng.reset_stats()
            for _ in range(reps):
                eng.eval(toks)
                eng.rewind(base)
            kx = eng.kstats()
            st = eng.stats()
            eng.set_profiling(0)
            eng.route_replay(None)
            n_exp = kx["expert_bytes"] / gu_bytes        # distinct experts over all layers and reps
            pairs = reps * T * sh.top_k * n_moe
            # int8 MFMA operations: useful = 2 * rows * cols per (token, expert) pair; the
            # kernels issue 16-token tiles, so issued = useful rounded up per expert to 16
            useful = 2.0 * pairs * (3 * sh.expert_ffn * sh.d_model)
            issued = 2.0 * n_exp * 16 * ((T * sh.top_k / max(n_exp / (reps * n_moe), 1) + 15) // 16) \
                * (3 * sh.expert_ffn * sh.d_model)
            secs = kx["expert_s"] + kx["expert_down_s"]
            res[T] = {
                "experts_per_layer": round(n_exp / (reps * n_moe), 2),
                "gateup_gbs": round(kx["expert_bytes"] / kx["expert_s"] / 1e9, 1),
                "down_gbs": round(kx["expert_down_bytes"] / kx["expert_down_s"] / 1e9, 1),
                "all_gbs": round((kx["expert_bytes"] + kx["expert_down_bytes"]) / secs / 1e9, 1),
                "hbm_frac": round((kx["expert_bytes"] + kx["expert_down_bytes"]) / secs / 1e9 / HBM_PEAK_GBS, 4),
                "us_per_layer": round(secs / (reps * n_moe) * 1e6, 2),
                "int8_tops_useful": round(useful / secs / 1e12, 2),
                "mfma_util_useful": round(useful / secs / 1e12 / 5000.0, 5),
                "int8_tops_issued_est": round(issued / secs / 1e12, 2),
            }
            log(f"[bench] experts T={T}: {res[T]}")
    best = res[65]
    return {
        "metric": "Q4 routed-expert kernels, Qwen3-30B-A3B shape, Zipf(1.1) top-8: HBM GB/s at T=65",
        "value": best["all_gbs"], "unit": "GB/s", "n_gpus": 1, "steps": 20, "warmup": 3,
        "ms_per_step": round(best["us_per_layer"] / 1e3, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "grouped Q4 expert gate/up + down kernels of the 48 MoE layers, T tokens with "
                               "Zipf(1.1) routes replayed, per T in {1, 9, 33, 65}", "per_T": res,
                   "mfma_peak_int8_tops": 5000.0},
    }


def dsv3_model_path(ctx: int) -> Path:
    from hearth_amd import container
    d = Path(os.environ.get("HEARTH_BENCH_DIR", tempfile.gettempdir())) / "hearth_bench"
    d.mkdir(parents=True, exist_ok=True)
    p = d / "deepseek_v3_3d20m.hearth"
    if not p.is_file():
        t = time.time()
        shape = container.Shape(**{**container.DEEPSEEK_V3.__dict__, "max_seq": ctx + 1024})
        container.make_shaped(p.with_suffix(".tmp"), shape, seed=0, n_unique_slabs=32)
        os.replace(p.with_suffix(".tmp"), p)
        log(f"[bench] wrote {p} ({p.stat().st_size / 1e9:.2f} GB) in {time.time() - t:.1f}s")
    return p


def bench_dsv3(a) -> dict:
    """DeepSeek-V3 shape (3 dense + 20 MoE layers), greedy chain verify k=8 at a
    4096-token context with the routed experts streamed from pinned host memory through
    an HBM cache smaller than the expert set (HEARTH_GPU_EXPERT_CACHE_GB, default 56),
    next-layer prefetch on; the same steps with every expert resident for comparison.
    --routes uniform replays routes drawn uniformly (each token 8 distinct experts of 256 in
    every MoE layer, hearth_route_replay) instead of the synthetic router's, whose choices
    concentrate on a subset of each layer: the regime where most demands miss a cache of
    half the expert set."""
    from hearth_amd import container
    from hearth_amd.engine import Engine

    ctx, k = 4096, a.k
    sh = container.DEEPSEEK_V3
    V = sh.vocab
    path = dsv3_model_path(ctx)
    prompt = container.uniform_ints(5678, ctx, V).astype(np.int32)
    need = (a.warmup + a.steps) * (k + 1) + k + 2
    cap = ctx + need + 16
    trace = None
    if a.routes == "uniform":
        n_moe = sh.n_layers - sh.n_dense
        ids = container.zipf_routes(4242, cap + 64, n_moe, sh.n_experts, sh.top_k, s=0.0)   # s = 0: uniform
        trace = container.write_route_trace(Path(tempfile.mkdtemp()) / "uniform.hrtr", ids, sh.n_layers,
                                            sh.n_experts)
    t = time.time()
    eng = Engine(path, max_seq=cap, max_batch=512)
    log(f"[bench] resident open {time.time() - t:.1f}s")
    if trace is not None:
        eng.route_replay(trace)
    eng.eval(prompt[:-1])
    base = eng.pos
    snap = eng.kv_export(base)
    cont = [int(prompt[-1])]
    for _ in range(need):
        cont.append(int(np.argmax(eng.eval([cont[-1]]))))
    eng.rewind(base)
    noisy = np.where(container.uniforms(98, len(cont)) < 0.3, container.uniform_ints(99, len(cont), V),
                     np.asarray(cont)).astype(np.int32)
    # warmup steps, then the timed steps continue from where they ended (new tokens, so
    # the streamed run below demands experts its warm cache has not seen)
    r_toks, r_secs = run_steps(eng, cont, noisy, base, k, a.warmup + a.steps)
    r_toks, r_secs = r_toks[a.warmup:], r_secs[a.warmup:]
    eng.close()
    resident = sum(r_toks) / sum(r_secs)
    log(f"[bench] dsv3 resident: {resident:.1f} tok/s, {sum(r_secs) / a.steps * 1e3:.2f} ms/step")
    if a.resident_only:
        return {"metric": "accepted tok/s, DeepSeek-V3-shape verify k=8, experts resident (1 GPU)",
                "value": round(resident, 3), "unit": "tok/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
                "ms_per_step": round(sum(r_secs) / a.steps * 1e3, 3), "higher_is_better": True, "scaling": "weak",
                "vs_baseline": None, "dtype": "int8", "data": "synthetic",
                "config": {"workload": "DeepSeek-V3-shaped MLA MoE, every expert resident, chain verify k=8 at 4096",
                           "tokens_per_step": round(sum(r_toks) / a.steps, 3)}}
    budget = os.environ.get("HEARTH_GPU_EXPERT_CACHE_GB") or "56"
    os.environ["HEARTH_GPU_EXPERT_CACHE_GB"] = budget
    t = time.time()
    eng = Engine(path, max_seq=cap, max_batch=512, prefetch="shared")
    open_s = time.time() - t
    log(f"[bench] streamed open {open_s:.1f}s")
    info0 = eng.store_info()
    if trace is not None:
        eng.route_replay(trace)
    eng.kv_import(snap, base)
    marks = {}

    def mark(s):   # counters at the start of the first timed step
        if s == a.warmup:
            eng.reset_stats()
            marks["copy_s"] = eng.store_info()["copy_s"]

    toks, secs = run_steps(eng, cont, noisy, base, k, a.warmup + a.steps, before=mark)
    toks, secs = toks[a.warmup:], secs[a.warmup:]
    c0 = marks["copy_s"]
    st = eng.stats()
    info = eng.store_info()
    eng.close()
    assert toks == r_toks, "streamed steps accepted other tokens than the resident ones"
    value = sum(toks) / sum(secs)
    copy_s = info["copy_s"] - c0
    loads = st["cache_misses"] + st["prefetch_issued"]
    log(f"[bench] dsv3 streamed: {value:.1f} tok/s, {sum(secs) / a.steps * 1e3:.2f} ms/step, "
        f"{loads / a.steps:.0f} loads/step, hit rate {st['hit_rate']:.3f}")
    E_all = 20 * container.DEEPSEEK_V3.n_experts
    return {
        "metric": "accepted tok/s, DeepSeek-V3-shape verify k=8, experts streamed from pinned host memory (1 GPU)",
        "value": round(value, 3), "unit": "tok/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(sum(secs) / a.steps * 1e3, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "DeepSeek-V3-shaped MLA MoE (3 dense + 20 MoE layers, 256 experts top-8 + shared, "
                               "Q4 experts / Q8 dense), greedy chain verify k=8 at context 4096, drafts = greedy "
                               "continuation with 30% random replacement" +
                               (", routes replayed uniformly at random" if trace is not None else ""),
                   "routes": a.routes, "streamed_open_s": round(open_s, 2),
                   "expert_cache_gb": float(budget), "cache_slots": info0["slots"], "experts_total": E_all,
                   "slot_bytes": info0["slot_bytes"], "host_tier_bytes": info0["host_tier_bytes"],
                   "tokens_per_step": round(sum(toks) / a.steps, 3),
                   "loads_per_step": round(loads / a.steps, 1), "hit_rate": round(st["hit_rate"], 4),
                   "prefetch_issued": st["prefetch_issued"], "prefetch_used": st["prefetch_used"],
                   "bytes_streamed_per_step": int(st["bytes_read"] / a.steps),
                   "host_link_gbs": round(st["bytes_read"] / copy_s / 1e9, 2) if copy_s > 0 else None,
                   "copy_busy_frac": round(copy_s / sum(secs), 3),
                   "resident_tok_s": round(resident, 2),
                   "resident_ms_per_step": round(sum(r_secs) / a.steps * 1e3, 3)},
    }


def bench_generate(a) -> dict:
    """End-to-end generation with n-gram drafts on the Qwen3-30B-A3B shape, greedy and
    sampled (temperature 0.8, top-p 0.95): the device loop against the host steps, the
    same tokens required. value is the path generate() takes by default."""
    from hearth_amd import container
    from hearth_amd import generate as G
    from hearth_amd.engine import Engine
    from hearth_amd.generate import Sampler, generate_ids

    path = model_path(a.layers, a.ctx, a.k)
    # a prompt that repeats itself (a document quoted back), so the lookup finds drafts
    rnd = container.uniform_ints(4321, a.ctx // 2, container.QWEN3_30B_A3B.vocab)
    prompt = [int(t) for t in np.concatenate([rnd, rnd])[:a.ctx]]
    eng = Engine(path, max_seq=a.ctx + a.gen + 64, max_batch=512)
    samplers = {"greedy": lambda: Sampler.greedy(), "sampled": lambda: Sampler(temperature=0.8, top_p=0.95, seed=11)}
    res = {}
    for mode, make in samplers.items():
        for spec, k in (("ngram", a.k), ("none", 0)):
            for loop in (False, True, False, True):   # warm both, then keep the second of each
                ids, st = generate_ids(eng, prompt, a.gen, make(), (), spec, k, 3, device_loop=loop)
                res[mode, spec, loop] = (ids, st)
                log(f"[bench] {mode} {spec} k={k} device_loop={loop}: {st.new_tokens} tokens, {st.forwards} forwards, "
                    f"accepted {st.accepted}/{st.drafted}, decode {st.decode_tok_s:.1f} tok/s")
            if res[mode, spec, False][0] != res[mode, spec, True][0]:
                raise RuntimeError(f"{mode} {spec}: the device loop and the host steps generated different tokens")
    default_loop = G._use_device_loop(eng, Sampler.greedy(), frozenset(), None, True, a.k)
    eng.close()
    if res["greedy", "ngram", True][0] != res["greedy", "none", True][0]:
        raise RuntimeError("speculative and plain greedy generation differ")
    d_st = res["greedy", "ngram", default_loop][1]
    rate = lambda m, s, l: round(res[m, s, l][1].decode_tok_s, 2)
    ms = lambda m, s, l: round(res[m, s, l][1].decode_s / max(1, res[m, s, l][1].forwards) * 1e3, 4)
    return {
        "metric": "greedy_generate_decode_tok_s", "value": round(d_st.decode_tok_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": d_st.forwards, "warmup": 1, "ms_per_step": round(d_st.decode_s / max(1, d_st.forwards) * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": f"Qwen3-30B-A3B-shaped greedy generation of {a.gen} tokens after a {a.ctx}-token "
                               f"self-repeating prompt, prompt-lookup drafts k={a.k} n<=3, generate()'s default "
                               f"path ({'device loop' if default_loop else 'host steps'})",
                   "layers": a.layers, "ctx": a.ctx, "k": a.k, "gen": a.gen,
                   "tokens_per_forward": round(d_st.tokens_per_forward, 3),
                   "acceptance_rate": round(d_st.acceptance_rate, 4),
                   "greedy_device_loop_decode_tok_s": rate("greedy", "ngram", True),
                   "greedy_host_steps_decode_tok_s": rate("greedy", "ngram", False),
                   "greedy_device_loop_ms_per_forward": ms("greedy", "ngram", True),
                   "greedy_host_steps_ms_per_forward": ms("greedy", "ngram", False),
                   "plain_device_loop_decode_tok_s": rate("greedy", "none", True),
                   "plain_host_steps_decode_tok_s": rate("greedy", "none", False),
                   "sampled_device_loop_decode_tok_s": rate("sampled", "ngram", True),
                   "sampled_host_steps_decode_tok_s": rate("sampled", "ngram", False),
                   "sampled_plain_device_loop_decode_tok_s": rate("sampled", "none", True),
                   "sampled_plain_host_steps_decode_tok_s": rate("sampled", "none", False)},
    }


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="speculative-verify throughput on one MI355X")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--k", type=int, default=8)
    ap.add_argument("--workload", choices=("chain", "tree", "experts", "dsv3", "generate"), default="chain",
                    help="chain: Qwen3-30B-A3B chain verify k=8 at 4096 (the headline); tree: 4x4x4 tree with "
                         "sampled acceptance at 2048; experts: the routed-expert kernels alone, Zipf routing; "
                         "dsv3: DeepSeek-V3 shape with streamed experts; generate: greedy generation with "
                         "n-gram drafts, device loop against host steps")
    ap.add_argument("--gen", type=int, default=256, help="generate: tokens to generate")
    ap.add_argument("--resident-only", action="store_true", help="dsv3: skip the streamed run")
    ap.add_argument("--routes", choices=("model", "uniform"), default="model",
                    help="dsv3: the synthetic router's routes, or uniform random routes replayed")
    ap.add_argument("--cpu-steps", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--summarize-trace", metavar="CSV",
                    help="print the per-verify-step kernel table of a rocprofv3 kernel trace and exit")
    ap.add_argument("--calibrate-copy", metavar="MIB", type=int,
                    help="only run device-to-device copies of MIB MiB (counter calibration) and exit")
    a = ap.parse_args(argv)
    if a.summarize_trace:
        return summarize_trace(a.summarize_trace, 10, "k_sample_walk" if a.workload == "tree" else "k_accept_walk")
    if a.calibrate_copy:
        return calibrate_copy(a.calibrate_copy)
    if a.gpus != 1:
        print(f"bench.py runs on exactly one GPU: this build has no multi-GPU path (asked for {a.gpus})",
              file=sys.stderr)
        return 2
    out = {"chain": bench_chain, "tree": bench_tree, "experts": bench_experts, "dsv3": bench_dsv3,
           "generate": bench_generate}[a.workload](a)
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
