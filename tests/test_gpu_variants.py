"""The verify engine on the GPU for the other model families' features, against the
restatement (glibc expf), which tests/test_oracle.py pins bit for bit to the reference
engine compiled from source on the same containers:

- dsv3_gqa: sigmoid scores with a selection bias, group-limited routing (4 groups, top 2
  kept), routed scale 2.5, a shared expert, a leading dense layer, interleaved (GPT-J)
  RoPE, no qk-norm;
- qwen2: q/k/v biases, a shared expert scaled by its sigmoid gate, no renormalisation of
  the top-k weights;
- olmoe: full-width qk-norm, partial RoPE (32 of 64 dims), tied embeddings, embedding /
  residual / logit scales;
- dsv3: the DeepSeek-V3 routing above with multi-head latent attention (q_lora 192,
  kv_lora 128, nope 64, rope 64, v 64);
- mla_noq: latent attention without q compression (kv_lora 256, rope 32, v 128).

Each model: a prompt's logits and routes bit-exact with the restatement, batch ==
sequential, a greedy tree verify that accepts what the restatement accepts, and the
committed KV equal to the accepted chain's.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle_py as O
from hearth_amd import container
from hearth_amd.engine import Engine

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.parametrize("variant", sorted(container.TINY_VARIANTS))
def test_variant_bit_exact_with_oracle(variant_models, variant, tmp_path):
    path = variant_models(variant)
    toks = container.uniform_ints(41, 40, 4096)
    O.gpu_numerics()
    om = O.Model(path)
    lo, ro = om.eval(toks, routes=True)
    with Engine(path, max_seq=512) as e:
        tr = tmp_path / "r.hrtr"
        e.trace_start(tr)
        lg = e.eval(toks, all_logits=True)
        e.trace_stop()
        mism = int((_bits(lg) != _bits(lo)).sum())
        assert mism == 0, f"{variant}: {mism} of {lg.size} logits differ from the restatement"
        routes = np.frombuffer(tr.read_bytes()[24:], dtype="<u2").reshape(ro.shape).astype(np.int32)
        assert np.array_equal(routes, ro)
        # batch == sequential
        e.reset()
        seq = np.stack([e.eval([t]) for t in toks[:12]])
        assert np.array_equal(_bits(seq), _bits(lg[:12]))
        # greedy tree verify at position 30: the first branch follows the model's argmax
        e.reset()
        e.eval(toks[:29])
        first = int(np.argmax(lg[29]))
        tok = np.array([toks[29], first, 7, first, 9], dtype=np.int32)
        par = np.array([-1, 0, 0, 1, 2], dtype=np.int32)
        p, fin, lv = e.verify_greedy(tok, par, want_logits=True)
        rc, opath, ofin = O.accept_tree(lv, tok, par)
        assert rc == 0 and p == opath and fin == ofin
        assert p[:2] == [0, 1]
        # the committed KV is the accepted chain's (tree slots moved into place)
        nxt = e.eval([fin])
        e.reset()
        e.eval(toks[:29])
        e.eval(tok[p])
        assert np.array_equal(_bits(nxt), _bits(e.eval([fin])))
