"""Route replay on the GPU (hearth_route_replay; reference model.c:1004-1012, 1885-1960).

The token at position p takes the experts of trace row p % rows for every MoE layer,
with weights from the router's scores; tree nodes use their position pos0 + depth. The
GPU is bit-exact with the restatement replaying the same trace (which is itself pinned
to the reference engine's replay, tests/test_oracle.py) through the three routing
kernels: T > 16 (rank kernel), T <= 16 ungrouped (small kernel), grouped (DeepSeek-V3
style); the routing trace it records is the replayed rows; malformed traces fail with
the reference's error codes and leave the previous replay in force.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle_py as O
from hearth_amd import container
from hearth_amd.engine import Engine, HearthError

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.parametrize("name", ["tiny", "dsv3"])
def test_route_replay_bit_exact(tiny_model, variant_models, tmp_path, name):
    path = tiny_model if name == "tiny" else variant_models(name)
    vocab = container.TINY.vocab if name == "tiny" else 4096
    O.gpu_numerics()
    m = O.Model(path)
    ids = O.synthetic_routes(11, 29, m.n_moe, m.n_experts, m.top_k)
    tr = tmp_path / "replay.hrtr"
    O.write_trace(tr, ids, m.n_layers, m.n_experts)
    toks = [int(t) for t in container.uniform_ints(43, 69, vocab)]
    tree_tok = np.array([7, 11, 900, 5, 12], np.int32)
    tree_par = np.array([-1, 0, 0, 1, 2], np.int32)
    rec = tmp_path / "recorded.hrtr"
    with Engine(path, max_seq=512) as e:
        e.route_replay(tr)
        e.trace_start(rec)
        g1 = e.eval(toks[:64], all_logits=True)
        g2 = e.eval(toks[64:69], all_logits=True)
        gt = e.verify_tree(tree_tok, tree_par)
        e.trace_stop()
    m.set_replay(ids)
    o1 = m.eval(toks[:64])
    o2 = m.eval(toks[64:69])
    ot = m.eval_tree(tree_tok, tree_par)
    assert np.array_equal(_bits(g1), _bits(o1))
    assert np.array_equal(_bits(g2), _bits(o2))
    assert np.array_equal(_bits(gt), _bits(ot))
    got = np.frombuffer(rec.read_bytes()[24:], dtype="<u2").reshape(-1, m.n_moe, m.top_k)
    depth = np.array([0, 1, 1, 2, 2])
    want = np.concatenate([ids[np.arange(69) % 29], ids[(69 + depth) % 29]])
    assert np.array_equal(got, want)


def test_route_replay_off_and_errors(tiny_model, tmp_path):
    O.gpu_numerics()
    m = O.Model(tiny_model)
    ids = O.synthetic_routes(12, 10, m.n_moe, m.n_experts, m.top_k)
    good = tmp_path / "good.hrtr"
    O.write_trace(good, ids, m.n_layers, m.n_experts)
    toks = [int(t) for t in container.uniform_ints(44, 9, container.TINY.vocab)]

    def bad(name, hdr=None, body=None):
        p = tmp_path / name
        h = np.array(hdr if hdr is not None else [0x52545248, 1, m.n_layers, m.n_experts, m.top_k, m.n_moe], "<u4")
        b = ids if body is None else body
        p.write_bytes(h.tobytes() + np.ascontiguousarray(b, "<u2").tobytes())
        return p

    rep = ids.copy()
    rep[3, 1, 2] = rep[3, 1, 0]
    oob = ids.copy()
    oob[5, 0, 1] = m.n_experts
    cases = {
        "missing": (tmp_path / "missing.hrtr", -4),
        "magic": (bad("magic.hrtr", hdr=[0x12345678, 1, m.n_layers, m.n_experts, m.top_k, m.n_moe]), -6),
        "experts": (bad("experts.hrtr", hdr=[0x52545248, 1, m.n_layers, m.n_experts + 1, m.top_k, m.n_moe]), -6),
        "body": (bad("body.hrtr", body=ids.reshape(-1)[:-1]), -6),
        "repeat": (bad("repeat.hrtr", body=rep), -6),
        "range": (bad("range.hrtr", body=oob), -6),
    }
    with Engine(tiny_model, max_seq=512) as e:
        plain = e.eval(toks, all_logits=True)
        e.reset()
        e.route_replay(good)
        for name, (p, code) in cases.items():
            with pytest.raises(HearthError, match=f"code {code}"):
                e.route_replay(p)
        replayed = e.eval(toks, all_logits=True)   # the good trace is still in force
        e.reset()
        e.route_replay("")
        off = e.eval(toks, all_logits=True)
    m.set_replay(ids)
    assert np.array_equal(_bits(replayed), _bits(m.eval(toks)))
    assert np.array_equal(_bits(off), _bits(plain))
    assert not np.array_equal(_bits(off), _bits(replayed))
