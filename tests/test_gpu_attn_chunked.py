"""The chunked attention order (HEARTH_GPU_ATTN_CHUNKED) on the GPU against the oracle's
restatement of the same order, bit for bit: tiny models of every query-group width the
kernel instantiates (4, 2 and 1 heads per KV head at head_dim 64), contexts of one to
eleven 64-row chunks, chains, trees, batch == sequential, captured graphs == direct
launches; switching orders. The Qwen3-30B-A3B shape (head_dim 128, 8 heads per KV head)
at the bench's contexts is in test_gpu_qwen3_shape.py."""
from __future__ import annotations

import os

import numpy as np
import pytest

import oracle_py as O
from hearth_amd import container
from hearth_amd.engine import Engine

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, os.cpu_count() or 1))


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _assert_same(gpu, ora, what):
    bad = int((_bits(gpu) != _bits(ora)).sum())
    assert bad == 0, f"{what}: {bad} of {gpu.size} values differ from the oracle"


@pytest.fixture
def chunked_oracle():
    O.gpu_numerics(O.ATTN_CHUNKED)
    yield
    O.gpu_numerics()


@pytest.mark.parametrize("name", ["tiny", "qwen2", "olmoe"])
def test_prompt_and_chain_equal_oracle(tiny_model, variant_models, chunked_oracle, name):
    path = tiny_model if name == "tiny" else variant_models(name)
    toks = container.uniform_ints(41, 700, 4096)
    with Engine(path, max_seq=1024, attn="chunked") as e:
        assert e.attn_mode == "chunked"
        lg = e.eval(toks[:690], all_logits=True)           # 690 rows: eleven chunks, the last partial
        lv = e.eval(toks[690:699], all_logits=True)        # a 9-token chain (a captured graph)
    m = O.Model(path, cap=1024, threads=THREADS)
    _assert_same(lg, m.eval(toks[:690]), f"{name} prompt")
    _assert_same(lv, m.eval(toks[690:699]), f"{name} chain")


def test_tree_batch_and_graphs(tiny_model, chunked_oracle, monkeypatch):
    prompt = container.uniform_ints(5, 150, container.TINY.vocab)
    tok = np.array([17, 5, 9, 300, 4000, 12, 8], dtype=np.int32)
    par = np.array([-1, 0, 0, 1, 1, 2, 4], dtype=np.int32)

    def run():
        with Engine(tiny_model, max_seq=1024, attn="chunked") as e:
            e.eval(prompt)
            lt = e.verify_tree(tok, par)
            chains = []
            for node in range(len(tok)):
                path, v = [], node
                while v >= 0:
                    path.append(v)
                    v = par[v]
                e.rewind(150)
                chains.append(e.eval(tok[path[::-1]], all_logits=True)[-1])
            e.reset()
            seq = np.stack([e.eval([t]) for t in prompt[:70]])
            return lt, np.stack(chains), seq

    lt, chains, seq = run()
    assert np.array_equal(_bits(lt), _bits(chains)), "tree nodes differ from their root chains"
    m = O.Model(tiny_model, cap=1024, threads=THREADS)
    batch = m.eval(prompt)
    _assert_same(seq, batch[:70], "one token at a time against the oracle's batch")
    _assert_same(lt, m.eval_tree(tok, par), "tree")
    monkeypatch.setenv("HEARTH_GPU_GRAPH", "0")
    direct = run()
    for a, b in zip(direct, (lt, chains, seq)):
        assert np.array_equal(_bits(a), _bits(b)), "captured graphs differ from direct launches"


def test_mode_switch(tiny_model, variant_models):
    """The order can be switched between calls (captured graphs of the other order are
    dropped); MLA models stay canonical."""
    toks = container.uniform_ints(3, 100, 4096)
    with Engine(tiny_model, max_seq=256) as e:
        assert e.attn_mode == "canonical"
        a = e.eval(toks[:9], all_logits=True)
        e.attn_mode = "chunked"
        e.reset()
        b = e.eval(toks[:9], all_logits=True)
        e.attn_mode = "canonical"
        e.reset()
        c = e.eval(toks[:9], all_logits=True)
    assert np.array_equal(_bits(a), _bits(c))
    O.gpu_numerics(O.ATTN_CHUNKED)
    try:
        _assert_same(b, O.Model(tiny_model, cap=256).eval(toks[:9]), "chunked after a switch")
    finally:
        O.gpu_numerics()
    with Engine(variant_models("dsv3"), max_seq=256) as e:
        with pytest.raises(ValueError):
            e.attn_mode = "chunked"
        assert e.attn_mode == "canonical"
