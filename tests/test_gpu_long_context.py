"""Contexts longer than 8192 rows (the softmax then works through the row in 8192-row
pieces re-read from the scores, and the value sums run 70 and more tiles), in both
attention orders, bit for bit against the oracle: the tiny model with a synthetic
9000-position KV snapshot imported into the engine and the oracle, then a 9-token chain
verify and a 4-node tree verify on top of it."""
from __future__ import annotations

import os

import numpy as np
import pytest

import oracle_py as O
from hearth_amd import _native, container
from hearth_amd.engine import Engine

pytestmark = pytest.mark.gpu

N0 = 9000
THREADS = max(1, min(16, os.cpu_count() or 1))


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.fixture(scope="module")
def long_model(tmp_path_factory):
    path = tmp_path_factory.mktemp("long") / "tiny16k.hearth"
    container.make_tiny(path, _native.quantize, seed=3,
                        shape=container.Shape(**{**container.TINY.__dict__, "max_seq": 16384}))
    return path


@pytest.mark.parametrize("attn", ["canonical", "chunked"])
def test_context_past_8192_rows(long_model, attn):
    s = container.TINY
    rng = np.random.default_rng(17)
    snap = rng.standard_normal((s.n_layers, N0 * 2 * s.n_kv_heads * s.head_dim)).astype(np.float32)
    toks = container.uniform_ints(5, 9, s.vocab).astype(np.int32)
    tree_tok = container.uniform_ints(6, 4, s.vocab).astype(np.int32)
    parent = np.array([-1, 0, 0, 1], dtype=np.int32)
    with Engine(long_model, max_seq=N0 + 64, attn=attn) as e:
        e.kv_import(snap, N0)
        lg = e.eval(toks, all_logits=True)
        e.kv_import(snap, N0)
        lt = e.verify_tree(tree_tok, parent)
    O.gpu_numerics(O.ATTN_CHUNKED if attn == "chunked" else O.ATTN_CANONICAL)
    try:
        m = O.Model(long_model, cap=N0 + 64, threads=THREADS)
        m.kv_import(snap, N0)
        lo = m.eval(toks)
        m.kv_import(snap, N0)
        lto = m.eval_tree(tree_tok, parent)
    finally:
        O.gpu_numerics()
    for got, want, what in ((lg, lo, "chain"), (lt, lto, "tree")):
        bad = int((_bits(got) != _bits(want)).sum())
        assert bad == 0, f"{attn} {what}: {bad} of {got.size} logits differ from the oracle"
