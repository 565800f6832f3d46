"""The verify step at the DeepSeek-V3 width, bit for bit against the oracle, with the
routed experts resident in HBM and streamed through the HBM expert cache.

Model: container.make_shaped at the full DeepSeek-V3 width: hidden 7168, 128 heads of
multi-head latent attention (q_lora 1536, kv_lora 512, nope 128, rope 64, v 128),
256 routed experts top-8 of FFN 2048 plus a shared expert of 2048, sigmoid scores with
a selection bias, 8 groups keeping 4, routed scale 2.5, dense FFN 18432, vocab 129280;
Q4 experts, Q8 attention / dense / shared / embedding / lm_head. The depth is cut to
1 dense + 2 MoE layers so that the oracle's single-token loop finishes in seconds;
every kernel configuration of a layer is the full model's. 32 physical expert slabs
back the 512 (layer, expert) entries (aliases); every entry still gets its own HBM
copy or cache load.

The oracle starts from the GPU's 4095-row KV snapshot (hearth_gpu_kv_export ->
ho_kv_import).

Cases:
- chain verify k = 8 at a 4095-token context (drafts: the greedy continuation with 3
  of 8 replaced), every expert resident: logits and routes equal the oracle's, greedy
  acceptance equals the CPU walk;
- the same step with the experts streamed from pinned host memory through 256 HBM
  slots (half the expert set), next-layer prefetch on: logits, path and KV equal the
  resident engine's; and with staged loads (HEARTH_GPU_HOST_TIER=0) as well.
"""
from __future__ import annotations

import dataclasses
import os

import numpy as np
import pytest

import oracle_py as O
from hearth_amd import container
from hearth_amd.engine import Engine

pytestmark = pytest.mark.gpu

SHAPE = dataclasses.replace(container.DEEPSEEK_V3, n_layers=3, n_dense=1)
CTX = 4095
THREADS = max(1, min(16, os.cpu_count() or 1))


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _assert_same(gpu, ora, what):
    bad = int((_bits(gpu) != _bits(ora)).sum())
    assert bad == 0, f"{what}: {bad} of {gpu.size} values differ"


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    path = tmp_path_factory.mktemp("dsv3w") / "deepseek_v3_3layers.hearth"
    container.make_shaped(path, SHAPE, seed=6, n_unique_slabs=32)
    return path


@pytest.fixture(scope="module")
def step(model):
    """Resident engine: 4095-token prefill, the KV snapshot, the drafts and the verify
    step's results (path, final token, logits, routes)."""
    O.gpu_numerics()
    eng = Engine(model, max_seq=CTX + 64, max_batch=512)
    try:
        assert eng.store_info()["streamed"] == 0
        prompt = container.uniform_ints(4343, CTX, SHAPE.vocab).astype(np.int32)
        eng.eval(prompt)
        snap = eng.kv_export(CTX)
        cont = [int(prompt[-1])]
        for _ in range(8):
            cont.append(int(np.argmax(eng.eval([cont[-1]]))))
        drafts = np.array(cont[1:9], dtype=np.int32)
        drafts[[2, 5, 6]] = (drafts[[2, 5, 6]] + 7919) % SHAPE.vocab
        toks = np.concatenate([[prompt[-1]], drafts]).astype(np.int32)
        eng.kv_import(snap, CTX)
        tr = model.parent / "chain.hrtr"
        eng.trace_start(tr)
        path, final, lg = eng.verify_greedy(toks, want_logits=True)
        eng.trace_stop()
        after = eng.kv_export(eng.pos)
    finally:
        eng.close()
    routes = np.frombuffer(tr.read_bytes()[24:], dtype="<u2").reshape(len(toks), 2, SHAPE.top_k)
    return dict(snap=snap, toks=toks, path=path, final=final, lg=lg, routes=routes, after=after)


def test_chain_verify_k8_ctx4095_resident(step, model):
    m = O.Model(model, cap=CTX + 64, threads=THREADS)
    m.kv_import(step["snap"], CTX)
    lo, ro = m.eval(step["toks"], routes=True)
    _assert_same(step["lg"], lo, "chain verify logits vs the oracle")
    assert np.array_equal(step["routes"].astype(np.int32), ro), "routes differ from the oracle"
    rc, opath, ofin = O.accept_tree(lo, step["toks"], np.arange(-1, len(step["toks"]) - 1))
    assert rc == 0 and step["path"] == opath and step["final"] == ofin
    assert step["path"][:3] == [0, 1, 2] and len(step["path"]) == 3, step["path"]   # draft 3 was replaced


@pytest.mark.parametrize("tier", ["1", "0"])
def test_chain_verify_streamed_equals_resident(step, model, monkeypatch, tier):
    monkeypatch.setenv("HEARTH_GPU_EXPERT_CACHE_GB", "0.0001")
    monkeypatch.setenv("HEARTH_GPU_HOST_TIER", tier)
    with Engine(model, max_seq=CTX + 64, max_batch=512, prefetch="next") as eng:
        info = eng.store_info()
        assert info["streamed"] == 1 and info["slots"] == SHAPE.n_experts
        assert info["slot_bytes"] == 23396352          # a Q4 slot: the slab's own size
        if tier == "1":
            assert info["host_tier"] == 1 and info["host_tier_bytes"] == 32 * 23396352
        else:
            assert info["host_tier"] == 0 and info["host_tier_bytes"] == 0
        eng.reset_stats()
        for _ in range(2):     # a second step over a warm cache
            eng.kv_import(step["snap"], CTX)
            path, final, lg = eng.verify_greedy(step["toks"], want_logits=True)
            _assert_same(lg, step["lg"], "streamed logits vs resident")
            assert path == step["path"] and final == step["final"]
            _assert_same(eng.kv_export(eng.pos), step["after"], "KV after the step")
        st = eng.stats()
        info = eng.store_info()
    assert st["cache_misses"] > 0 and st["bytes_read"] >= st["cache_misses"] * 23396352
    assert info["copy_s"] > 0.0
