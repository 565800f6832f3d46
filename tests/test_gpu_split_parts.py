"""Expert kernels whose rows split into several parts, at widths the tiny models do not
reach, against the restatement bit for bit.

The small-batch expert kernel (k_expert_tk) cuts each Q4 weight row into parts of 8
block pairs (1024 columns) and passes the running sums from part to part through LDS,
in the reference's block order. The tiny models' rows have 4 pairs (one part); the
Qwen3 width has 16 (two full parts). This model has d_model 1280 (gate/up rows of 10
pairs: a full part and a partial one of 2) and expert_ffn 1152 (down rows of 9 pairs: 8
and 1), 64 experts top-8 (the small routing at K = 8) and 10 query heads over 2 KV heads
(query groups of 5). Checked: the logits and routes of a 120-token prompt, chain verify
steps of 1, 9 and 16 tokens after it (experts of 1 to 16 tokens), and the KV rows.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import oracle_py as O
from hearth_amd import container
from hearth_amd.engine import Engine

pytestmark = pytest.mark.gpu

SHAPE = container.Shape(n_layers=2, d_model=1280, n_heads=10, n_kv_heads=2, head_dim=128, n_experts=64, top_k=8,
                        expert_ffn=1152, vocab=2048, max_seq=512)
THREADS = max(1, min(16, os.cpu_count() or 1))


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    from hearth_amd import _native
    path = tmp_path_factory.mktemp("split") / "split_parts.hearth"
    container.make_tiny(path, _native.quantize, seed=3, shape=SHAPE)
    return path


def test_split_parts_equal_oracle(model, tmp_path):
    O.gpu_numerics()
    toks = container.uniform_ints(77, 146, SHAPE.vocab).astype(np.int32)
    m = O.Model(model, cap=512, threads=THREADS)
    lo, ro = m.eval(toks[:120], routes=True)
    with Engine(model, max_seq=512) as e:
        tr = tmp_path / "r.hrtr"
        e.trace_start(tr)
        lg = e.eval(toks[:120], all_logits=True)
        e.trace_stop()
        assert int((_bits(lg) != _bits(lo)).sum()) == 0, "prompt logits differ from the restatement"
        routes = np.frombuffer(tr.read_bytes()[24:], dtype="<u2").reshape(ro.shape).astype(np.int32)
        assert np.array_equal(routes, ro), "routes differ from the restatement"
        pos = 120
        for T in (1, 9, 16):
            print(f"chain of {T} at {pos}", flush=True)
            step = toks[pos:pos + T]
            lv = e.eval(step, all_logits=True)
            ov = m.eval(step)
            assert int((_bits(lv) != _bits(ov)).sum()) == 0, f"verify of {T} tokens differs from the restatement"
            pos += T
        _assert_kv(e.kv_export(pos), m.kv_export(pos))
    m.close()


def _assert_kv(gpu, ora):
    assert gpu.shape == ora.shape
    assert int((_bits(gpu) != _bits(ora)).sum()) == 0, "KV rows differ from the restatement"
