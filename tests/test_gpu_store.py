"""The HBM expert cache (hearth_amd/csrc/expert_store.cpp) on the GPU.

With HEARTH_GPU_EXPERT_CACHE_GB far below the expert set, every MoE layer streams its
experts from host memory through a pool of E slots:

- logits (prompt, chain verify, tree verify + commit) are bit-identical to the engine
  with every expert resident: the cache moves bytes, never changes numerics
  (reference INV-DET-1);
- hits, misses and evictions equal a replay of the victim policy (LRU: least recently
  used; LFU: lowest decayed heat, then least recent, store.c:166-199) over the routing
  trace: per call and MoE layer the active experts in ascending order (prefetch off);
- hearth_get_stats reports them (cache_hits / cache_misses / evictions / bytes_read);
- next-layer prefetch (model.c:935-984, store.c:541-561) -- the router of the next MoE
  layer on the predicted input (h, plus the shared expert's output in shared mode) --
  changes no logit, and its counters are consistent: every load is a miss or an issued
  prefetch, a prefetched expert is used at most once and wasted only if never used.
"""
from __future__ import annotations

import numpy as np
import pytest

from hearth_amd import container
from hearth_amd.engine import Engine

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _run(path, calls, **kw):
    """logits of each call (lists of tokens, or ("tree", tokens, parent, path))"""
    out = []
    with Engine(path, max_seq=512, **kw) as e:
        for c in calls:
            if c[0] == "tree":
                _, tok, par, commit = c
                out.append(e.verify_tree(tok, par))
                e.commit_path(commit)
            else:
                out.append(e.eval(c, all_logits=True))
        stats = e.stats()
    return out, stats


def _replay(trace_routes, call_sizes, n_moe, E, n_slots, policy):
    """hits, misses, evictions of the cache policy over the calls' routes"""
    slot_key = [-1] * n_slots
    slot_seq = [0] * n_slots
    where = {}
    heat = {}
    seq = 0
    hits = misses = evictions = 0
    row = 0
    for n in call_sizes:
        rows = trace_routes[row:row + n]
        row += n
        for m in range(n_moe):
            active = sorted(set(int(x) for x in rows[:, m, :].ravel()))
            busy = {where[(m, e)] for e in active if (m, e) in where}
            for e in active:
                k = (m, e)
                if k in where:
                    hits += 1
                    s = where[k]
                else:
                    misses += 1
                    free = [s for s in range(n_slots) if slot_key[s] == -1]
                    if free:
                        s = free[0]
                    else:
                        cand = [s for s in range(n_slots) if s not in busy]
                        if policy == "lfu":
                            s = min(cand, key=lambda s: (heat.get(slot_key[s], 0.0), slot_seq[s], s))
                        else:
                            s = min(cand, key=lambda s: (slot_seq[s], s))
                        del where[slot_key[s]]
                        evictions += 1
                    slot_key[s] = k
                    where[k] = s
                    busy.add(s)
                seq += 1
                slot_seq[s] = seq
                heat[k] = heat.get(k, 0.0) + 1.0
        if policy == "lfu":
            for k in heat:
                heat[k] *= 0.995
    return hits, misses, evictions


@pytest.mark.parametrize("policy", ["lru", "lfu"])
def test_streamed_experts_bit_identical_and_policy(tiny_model, monkeypatch, tmp_path, policy):
    toks = container.uniform_ints(51, 60, container.TINY.vocab)
    calls = [list(toks[:40]), list(toks[40:45]), [int(t) for t in toks[45:46]],
             ("tree", np.array([7, 11, 900, 5, 12], np.int32), np.array([-1, 0, 0, 1, 2], np.int32), [0, 1, 3])]
    ref, _ = _run(tiny_model, calls)
    monkeypatch.setenv("HEARTH_GPU_EXPERT_CACHE_GB", "0.001")
    with Engine(tiny_model, max_seq=512, policy=policy, prefetch="off") as e:
        tr = tmp_path / "r.hrtr"
        e.trace_start(tr)
        got = []
        for c in calls:
            if c[0] == "tree":
                _, tok, par, commit = c
                got.append(e.verify_tree(tok, par))
                e.commit_path(commit)
            else:
                got.append(e.eval(c, all_logits=True))
        e.trace_stop()
        st = e.stats()
        assert e.info["cache_slots"] == 16
        after = e.eval([3])
    for a, b in zip(ref, got):
        assert np.array_equal(_bits(a), _bits(b))
    assert st["cache_slots"] == 16 and st["cache_misses"] > 0 and st["evictions"] > 0
    routes = np.frombuffer(tr.read_bytes()[24:], dtype="<u2").reshape(-1, 4, 4)
    sizes = [40, 5, 1, 5]
    want = _replay(routes, sizes, 4, 16, 16, policy)
    assert (st["cache_hits"], st["cache_misses"], st["evictions"]) == want
    assert st["cache_hits"] + st["cache_misses"] == st["expert_loads_unique"]
    assert st["bytes_read"] == st["cache_misses"] * 208896
    # the committed KV after streaming is the resident engine's
    with Engine(tiny_model, max_seq=512) as e2:
        for c in calls:
            if c[0] == "tree":
                e2.verify_tree(c[1], c[2], want_logits=False)
                e2.commit_path(c[3])
            else:
                e2.eval(c)
        assert np.array_equal(_bits(after), _bits(e2.eval([3])))


def test_streamed_experts_deepseek_shape(variant_models, monkeypatch):
    path = variant_models("dsv3")
    toks = container.uniform_ints(52, 30, 4096)
    ref, _ = _run(path, [list(toks[:25]), list(toks[25:])])
    monkeypatch.setenv("HEARTH_GPU_EXPERT_CACHE_GB", "0.0001")
    got, st = _run(path, [list(toks[:25]), list(toks[25:])], prefetch="off")
    for a, b in zip(ref, got):
        assert np.array_equal(_bits(a), _bits(b))
    assert st["cache_slots"] == 16 and st["evictions"] > 0


SLAB = {"tiny": 208896}


@pytest.mark.parametrize("name", ["tiny", "dsv3"])
@pytest.mark.parametrize("mode,extra", [("shared", 0), ("next", 2)])
def test_prefetch_bit_identical_and_counters(tiny_model, variant_models, monkeypatch, name, mode, extra):
    path = tiny_model if name == "tiny" else variant_models(name)
    vocab = container.TINY.vocab if name == "tiny" else 4096
    toks = [int(t) for t in container.uniform_ints(53, 100, vocab)]
    calls = [toks[:40]] + [toks[i:i + 5] for i in range(40, 100, 5)]
    ref, _ = _run(path, calls)
    monkeypatch.setenv("HEARTH_GPU_EXPERT_CACHE_GB", "0.001")
    off, st_off = _run(path, calls, prefetch="off")
    got, st = _run(path, calls, prefetch=mode, prefetch_extra=extra)
    for a, b, c in zip(ref, off, got):
        assert np.array_equal(_bits(a), _bits(b))
        assert np.array_equal(_bits(a), _bits(c))
    assert st_off["prefetch_issued"] == 0
    assert st["cache_hits"] + st["cache_misses"] == st["expert_loads_unique"] == st_off["expert_loads_unique"]
    assert st["prefetch_issued"] > 0 and st["prefetch_used"] > 0
    assert st["prefetch_used"] + st["prefetch_wasted"] <= st["prefetch_issued"]
    assert st["prefetch_used"] <= st["cache_hits"]
    slab = st_off["bytes_read"] // st_off["cache_misses"]
    if name in SLAB:
        assert slab == SLAB[name]
    assert st["bytes_read"] == (st["cache_misses"] + st["prefetch_issued"]) * slab
    # the predictions of these models are good enough to save demand loads
    assert st["cache_misses"] < st_off["cache_misses"]


def test_host_tier_equals_staged_loads(tiny_model, monkeypatch):
    """A load that copies the pinned slot image (the default) and a staged load that
    repacks the container's slab on the device fill a slot with the same bytes: equal
    logits and counters; hearth_gpu_get_store_info reports the tier."""
    toks = [int(t) for t in container.uniform_ints(54, 70, container.TINY.vocab)]
    calls = [toks[:40], toks[40:45], toks[45:54], toks[54:]]
    ref, _ = _run(tiny_model, calls)
    with Engine(tiny_model, max_seq=512) as e:
        assert e.store_info() == dict(streamed=0, host_tier=0, slots=0, slot_bytes=0, host_tier_bytes=0, copy_s=0.0)
    monkeypatch.setenv("HEARTH_GPU_EXPERT_CACHE_GB", "0.0001")
    got = {}
    for tier in ("1", "0"):
        monkeypatch.setenv("HEARTH_GPU_HOST_TIER", tier)
        with Engine(tiny_model, max_seq=512, prefetch="off") as e:
            out = [e.eval(c, all_logits=True) for c in calls]
            got[tier] = (out, e.stats(), e.store_info())
    n_slabs = container.TINY.n_layers * container.TINY.n_experts
    for tier, (out, st, info) in got.items():
        for a, b in zip(ref, out):
            assert np.array_equal(_bits(a), _bits(b)), f"HEARTH_GPU_HOST_TIER={tier}"
        assert info["streamed"] == 1 and info["slots"] == 16 and info["slot_bytes"] == 208896
        assert info["host_tier"] == int(tier)
        assert info["host_tier_bytes"] == (n_slabs * 208896 if tier == "1" else 0)
        assert st["cache_misses"] > 0 and st["bytes_read"] == st["cache_misses"] * 208896
        assert info["copy_s"] > 0.0
    keys = ("cache_hits", "cache_misses", "evictions", "bytes_read")
    assert [got["1"][1][k] for k in keys] == [got["0"][1][k] for k in keys]


@pytest.mark.parametrize("tier", ["1", "0"])
@pytest.mark.parametrize("fail_at", [1, 7, 23])
def test_failed_load_changes_nothing(tiny_model, monkeypatch, tier, fail_at):
    """HEARTH_GPU_STORE_FAIL_LOAD=n makes the n-th expert load since open fail once on the
    host, before anything is enqueued (hearth.h:131-132: a failed call changes nothing).
    The call returns an error with the position and every counter as before it; the slot
    whose load failed is not left mapped, so the same call run again is a miss there,
    loads the expert and gives the resident engine's logits bit for bit."""
    toks = [int(t) for t in container.uniform_ints(55, 60, container.TINY.vocab)]
    calls = [toks[:30], toks[30:39], toks[39:48]]
    ref, _ = _run(tiny_model, calls)
    monkeypatch.setenv("HEARTH_GPU_EXPERT_CACHE_GB", "0.0001")
    monkeypatch.setenv("HEARTH_GPU_HOST_TIER", tier)
    monkeypatch.setenv("HEARTH_GPU_STORE_FAIL_LOAD", str(fail_at))
    failed = 0
    with Engine(tiny_model, max_seq=512, prefetch="off") as e:
        got = []
        for c in calls:
            before_pos, before = e.pos, e.stats()
            try:
                got.append(e.eval(c, all_logits=True))
            except Exception:
                failed += 1
                assert e.pos == before_pos
                after = e.stats()
                for k in ("cache_hits", "cache_misses", "evictions", "bytes_read", "expert_loads_unique"):
                    assert after[k] == before[k], k
                got.append(e.eval(c, all_logits=True))   # the injected failure fires once
        st = e.stats()
    assert failed == 1
    for a, b in zip(ref, got):
        assert np.array_equal(_bits(a), _bits(b))
    assert st["cache_hits"] + st["cache_misses"] == st["expert_loads_unique"]
    assert st["bytes_read"] == st["cache_misses"] * 208896
