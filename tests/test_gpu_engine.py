"""The verify engine on the GPU against the oracle and the reference's golden outputs,
on the tiny Qwen3-MoE-shaped model (4 layers, hidden 512, GQA 8/2, 16 experts top-4).

- bit-exact with the restatement (its expf is the libm's restated; RoPE tables come
  from the host libm as in the reference);
- bit-exact with the reference engine's own logits: its golden outputs, and the engine
  itself (oracle/_ref) over a 700-token context; routing agreement with its trace;
- batch == sequential == chunked (INV-DET-2 on the device);
- tree verification == chain evaluation of every root path, and committing a path
  leaves the KV of the chain;
- verify_greedy reproduces the reference's speculative step (generate.py:365-392).
"""
from __future__ import annotations

import numpy as np
import pytest

import golden_io
import oracle_py as O
from hearth_amd import _native, container
from hearth_amd.engine import Engine, HearthError

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng(tiny_model):
    e = Engine(tiny_model, max_seq=1024)
    yield e
    e.close()


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def test_prompt_bit_exact_with_oracle(eng, tiny_model):
    g = golden_io.tiny_ref()
    eng.reset()
    lg = eng.eval(g["prompt"], all_logits=True)
    O.gpu_numerics()
    lo = O.Model(tiny_model).eval(g["prompt"])
    mism = int((_bits(lg) != _bits(lo)).sum())
    assert mism == 0, f"{mism} of {lg.size} logits differ from the restatement"


def test_bit_exact_with_reference_engine_golden(eng):
    """The reference engine's own logits (tests/golden/tiny_ref.npz, written by the
    reference built from its sources on this image's glibc): equal bit for bit, which
    implies the north-star tolerance (1e-3 of max |logit|, top-1 agreement)."""
    g = golden_io.tiny_ref()
    eng.reset()
    lp = eng.eval(g["prompt"], all_logits=True)
    assert np.array_equal(_bits(lp[-8:]), _bits(g["prompt_last8"]))
    assert np.array_equal(lp.argmax(1), g["prompt_argmax"])
    lv = eng.eval(g["verify_tokens"], all_logits=True)
    assert np.array_equal(_bits(lv), _bits(g["verify_logits"]))


@pytest.mark.skipif(not O.REF_LIB.is_file(), reason="reference engine not built (make -C oracle)")
def test_bit_exact_with_reference_engine_700_tokens(tmp_path):
    """A 700-token context on a tiny model against the reference engine itself (compiled
    from its C sources into oracle/_ref), every row: where the quantized activations
    would amplify any 1-ulp difference (an exp that is not the libm's differs from the
    reference on ~10% of such rows), the logits are identical."""
    path = container.make_tiny(tmp_path / "tiny1k.hearth", _native.quantize, seed=3,
                               shape=container.Shape(**{**container.TINY.__dict__, "max_seq": 1024}))
    toks = container.uniform_ints(12, 700, container.TINY.vocab)
    ref = Engine(path, lib=str(O.REF_LIB), threads=8, prefetch="off", max_seq=1024)
    lr = ref.eval(toks, all_logits=True)
    ref.close()
    with Engine(path, max_seq=1024) as e:
        lg = e.eval(toks, all_logits=True)
    bad = int((_bits(lg) != _bits(lr)).any(1).sum())
    assert bad == 0, f"{bad} of 700 rows differ from the reference engine"


def test_routing_agreement_with_reference(eng, tmp_path):
    g = golden_io.tiny_ref()
    eng.reset()
    tr = tmp_path / "r.hrtr"
    eng.trace_start(tr)
    eng.eval(g["prompt"])
    eng.eval(g["verify_tokens"])
    eng.trace_stop()
    routes = np.frombuffer(tr.read_bytes()[24:], dtype="<u2").reshape(-1, 4, 4).astype(np.int32)
    want = np.concatenate([g["routes"][:128], g["routes"][-5:]])
    agree = (np.sort(routes, -1) == np.sort(want, -1)).all(-1).mean()
    assert agree >= 0.999, agree


def test_batch_equals_sequential_and_chunked(tiny_model, eng):
    toks = container.uniform_ints(21, 40, container.TINY.vocab)
    eng.reset()
    batch = eng.eval(toks, all_logits=True)
    eng.reset()
    seq = np.stack([eng.eval([t]) for t in toks])
    assert np.array_equal(_bits(batch), _bits(seq))
    with Engine(tiny_model, max_seq=256, max_batch=7) as e2:
        chunked = e2.eval(toks, all_logits=True)
        assert np.array_equal(_bits(batch), _bits(chunked))
        e2.reset()
        last = e2.eval(toks)
        assert np.array_equal(_bits(last), _bits(batch[-1]))


def test_failed_calls_change_nothing(eng):
    eng.reset()
    eng.eval([1, 2, 3])
    with pytest.raises(ValueError):
        eng.eval([1, container.TINY.vocab])
    assert eng.pos == 3
    with pytest.raises(HearthError):
        eng.eval(list(range(2000)))
    assert eng.pos == 3
    eng.rewind(1)
    assert eng.pos == 1
    with pytest.raises(ValueError):
        eng.rewind(5)


def test_verify_greedy_reproduces_reference_step(eng):
    g = golden_io.tiny_ref()
    eng.reset()
    eng.eval(g["prompt"])
    path, final, lg = eng.verify_greedy(g["verify_tokens"], want_logits=True)
    assert len(path) - 1 == int(g["n_acc"]) and final == int(g["final"])
    assert path == list(range(len(path)))
    assert eng.pos == 128 + len(path)
    assert (lg.argmax(1) == g["verify_logits"].argmax(1)).all()
    # the committed KV is the chain's: the next token's logits equal a plain eval's
    nxt = eng.eval([final])
    eng.reset()
    eng.eval(g["prompt"])
    eng.eval(g["verify_tokens"][:len(path)])
    assert np.array_equal(_bits(nxt), _bits(eng.eval([final])))


def test_tree_equals_chain_on_gpu(eng):
    prompt = container.uniform_ints(5, 40, container.TINY.vocab)
    tok = np.array([17, 5, 9, 300, 4000, 12, 8], dtype=np.int32)
    par = np.array([-1, 0, 0, 1, 1, 2, 4], dtype=np.int32)
    eng.reset()
    eng.eval(prompt)
    lt = eng.verify_tree(tok, par)
    assert eng.pos == 40
    for node in range(len(tok)):
        path, v = [], node
        while v >= 0:
            path.append(v)
            v = par[v]
        path = path[::-1]
        eng.rewind(40)
        lc = eng.eval(tok[path], all_logits=True)
        assert np.array_equal(_bits(lc[-1]), _bits(lt[node])), node
    eng.rewind(40)
    eng.verify_tree(tok, par, want_logits=False)
    # only root paths of the tree commit: siblings, a skipped level or a missing root fail
    for bad in ([0, 1, 2], [0, 6], [1, 4], [0, 2, 4]):
        with pytest.raises(HearthError):
            eng.commit_path(bad)
        assert eng.pos == 40
    eng.commit_path([0, 1, 4, 6])
    assert eng.pos == 44
    after = eng.eval([77])
    eng.rewind(40)
    eng.eval(tok[[0, 1, 4, 6]])
    assert np.array_equal(_bits(after), _bits(eng.eval([77])))


def test_tree_greedy_verify_matches_oracle(eng, tiny_model):
    prompt = container.uniform_ints(9, 30, container.TINY.vocab)
    eng.reset()
    eng.eval(prompt)
    # a tree whose first branch follows the model's own argmax
    first = int(np.argmax(eng.eval([3], all_logits=False)))
    eng.rewind(30)
    tok = np.array([3, 11, first, 5, first, 6], dtype=np.int32)
    par = np.array([-1, 0, 0, 1, 2, 2], dtype=np.int32)
    path, final, lg = eng.verify_greedy(tok, par, want_logits=True)
    rc, opath, ofin = O.accept_tree(lg, tok, par)
    assert rc == 0 and path == opath and final == ofin
    assert path[:2] == [0, 2]


@pytest.mark.parametrize("which", ["tiny", "dsv3"])
def test_captured_forward_equals_direct_launches(tiny_model, variant_models, monkeypatch, which):
    """Calls of at most 128 tokens replay a captured graph of the forward (pos0 read from
    device memory, grids sized for a row bound); the same call sequence with capture off
    (HEARTH_GPU_GRAPH=0) launches every kernel directly. The graphs are replayed at
    several positions, for chains, a tree and single tokens, with eager work (prefill
    chunks above 128 tokens, rewinds, commits) between the replays: every logit is the
    same."""
    path = tiny_model if which == "tiny" else variant_models("dsv3")
    vocab = 4096
    toks = [int(t) for t in container.uniform_ints(61, 400, vocab)]
    parent = [-1, 0, 0, 1, 1, 2, 3]

    def run():
        out = []
        with Engine(path, max_seq=1024) as e:
            out.append(e.eval(toks[:200], all_logits=True))          # 200 > 128: direct launches
            for step in range(4):                                     # a 9-token chain, replayed at 4 positions
                out.append(e.eval(toks[200 + 9 * step:209 + 9 * step], all_logits=True))
                e.rewind(e.pos - 4)
            out.append(e.eval([toks[300]], all_logits=True))          # one token
            out.append(e.eval([toks[301]], all_logits=True))
            for step in range(3):                                     # a 7-node tree, committed each time
                lg = e.verify_tree(toks[310 + 7 * step:317 + 7 * step], parent)
                out.append(lg)
                e.commit_path([0, 1, 3])
            out.append(e.eval(toks[340:340 + 150], all_logits=True))  # direct again
            out.append(e.eval(toks[330:339], all_logits=True))        # the chain graph once more
        return out

    monkeypatch.setenv("HEARTH_GPU_GRAPH", "0")
    direct = run()
    monkeypatch.setenv("HEARTH_GPU_GRAPH", "1")
    graphed = run()
    assert len(direct) == len(graphed)
    for i, (a, b) in enumerate(zip(direct, graphed)):
        assert np.array_equal(_bits(a), _bits(b)), f"call {i}: replayed graph differs from direct launches"
