"""Sampled acceptance on the GPU (hearth_gpu_probs, hearth_gpu_accept_sample,
hearth_verify_sample) against the CPU restatement, which tests/test_sampling_oracle.py
pins to the reference's own Sampler / accept_point_mass outputs.

- the device distributions equal the restatement's float64 rows bit for bit, over
  temperature, top-k, top-p (including rows flat enough that the top-p candidates
  exceed the LDS sort and go through the global sort), min-p, the repetition penalty
  with a per-node context, ties, -inf entries, exp arguments down to -760 (subnormal
  and underflowing doubles) and vocabularies from 7 to 151936;
- acceptance (path and final token) equals the restatement's on random chains and
  trees, point-mass and general draft distributions, including uniforms placed exactly
  on the acceptance boundary (a 1-ulp difference in p[x] would flip the decision);
- the reference's own verify steps (tests/golden/sampling_ref.npz) are reproduced;
- on the engine, hearth_verify_sample accepts what the restatement accepts on the
  returned logits and commits the accepted path's KV.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle_py as O
from golden_io import GOLDEN
from hearth_amd import container
from hearth_amd import engine as E

pytestmark = pytest.mark.gpu

SETTINGS = [
    dict(temperature=1.0),
    dict(temperature=0.8, top_p=0.95),
    dict(temperature=0.7, top_k=40),
    dict(temperature=1.3, top_k=10, top_p=0.9, min_p=0.05),
    dict(temperature=0.0),
    dict(temperature=1.0, repetition_penalty=1.3),
    dict(temperature=0.5, min_p=0.1),
    dict(temperature=1e-4),
    dict(temperature=1.0, top_p=0.5),
    dict(temperature=0.9, top_p=1.0 - 1e-12),
]


def _rows(rng, kind, n, V):
    if kind == "normal1":
        return rng.normal(0, 1, (n, V)).astype(np.float32)
    if kind == "normal4":
        return rng.normal(0, 4, (n, V)).astype(np.float32)
    if kind == "ties":
        return rng.integers(-3, 4, (n, V)).astype(np.float32)
    if kind == "neginf":
        x = rng.normal(0, 2, (n, V)).astype(np.float32)
        x[rng.random((n, V)) < 0.3] = -np.inf
        x[:, 0] = 0.5
        return x
    if kind == "equal":
        return np.full((n, V), 0.25, dtype=np.float32)
    if kind == "flat":
        return rng.normal(0, 0.01, (n, V)).astype(np.float32)
    if kind == "wide":   # exp arguments down to -760: subnormal and underflowing doubles
        x = rng.uniform(-760.0, 0.0, (n, V)).astype(np.float32)
        x[:, 0] = 0.0
        edge = np.float32([-700, -708.5, -709.9, -720, -730, -744.4, -745.1, -745.3])[:V - 1]
        x[:, 1:1 + edge.size] = edge
        return x
    x = rng.normal(0, 1, (n, V)).astype(np.float32)
    x[:, V // 3] = 20.0
    return x


def _check_probs(rows, tokens, st, ctx):
    n, V = rows.shape
    s_gpu = E.make_sampler(context=ctx, **st)
    rc, p = E.gpu_probs(rows, tokens, None, s_gpu)
    assert rc == 0
    s_cpu = O.sampler(st.get("temperature", 1.0), st.get("top_k", 0), st.get("top_p", 1.0), st.get("min_p", 0.0),
                      st.get("repetition_penalty", 1.0), ctx)
    for v in range(n):
        orc, want = O.probs_s(rows[v], s_cpu, tokens[1:v + 1])
        assert orc == 0
        assert np.array_equal(p[v].view(np.uint64), want.view(np.uint64)), (v, V, st)


@pytest.mark.parametrize("V", [7, 300, 4096, 8193, 16384, 20000])
def test_gpu_probs_bit_exact(V):
    rng = np.random.default_rng(V)
    for kind in ["normal1", "normal4", "ties", "neginf", "equal", "flat", "peaked", "wide"]:
        for st in SETTINGS:
            rows = _rows(rng, kind, 3, V)
            tokens = rng.integers(0, V, 3).astype(np.int32)
            ctx = np.concatenate([rng.integers(0, V, 9), [-1, V + 3, 2, 2]]).astype(np.int32)
            _check_probs(rows, tokens, st, ctx)


@pytest.mark.parametrize("kind,st", [
    ("normal4", dict(temperature=0.8, top_p=0.95)),
    ("normal1", dict(temperature=1.3, top_k=50, top_p=0.9, min_p=0.02)),
    ("flat", dict(temperature=1.0, top_p=0.9)),       # ~137k candidates: global sort
    ("equal", dict(temperature=0.7, top_p=0.3)),      # every p equal: index order decides
    ("peaked", dict(temperature=1.0, repetition_penalty=1.2)),
    ("ties", dict(temperature=0.0, repetition_penalty=2.0)),
])
def test_gpu_probs_bit_exact_full_vocab(kind, st):
    V = 151936
    rng = np.random.default_rng(17)
    rows = _rows(rng, kind, 2, V)
    tokens = rng.integers(0, V, 2).astype(np.int32)
    ctx = rng.integers(0, V, 40).astype(np.int32)
    _check_probs(rows, tokens, st, ctx)


def _random_tree(rng, n, V, rows, st):
    parent = np.array([-1] + [int(rng.integers(0, i)) for i in range(1, n)], dtype=np.int32)
    tokens = rng.integers(0, V, n).astype(np.int32)
    s = O.sampler(**{k: v for k, v in st.items() if k != "ctx"})
    for c in range(1, n):   # many children are likely tokens of their parent
        if rng.random() < 0.6:
            _, p = O.probs_s(rows[parent[c]], s)
            tokens[c] = int(np.argmax(p)) if rng.random() < 0.5 else int(rng.choice(V, p=p / p.sum()))
    return tokens, parent


def test_gpu_accept_sample_equals_oracle():
    rng = np.random.default_rng(23)
    for trial in range(90):
        n, V = int(rng.integers(1, 12)), int(rng.integers(2, 3000))
        rows = rng.normal(0, float(rng.choice([0.5, 2.0, 6.0])), (n, V)).astype(np.float32)
        st = dict(SETTINGS[trial % len(SETTINGS)])
        tokens, parent = _random_tree(rng, n, V, rows, st)
        q = None
        if trial % 3 == 2:
            q = rng.random((n, V)) ** 3 + 1e-3
            q /= q.sum(1, keepdims=True)
        u = rng.random(2 * n)
        if trial % 4 == 1 and n > 1:
            # decide child 1 exactly on its boundary: u == p[x] / q[x] rejects, any larger p accepts
            _, p0 = O.probs_s(rows[parent[1]], O.sampler(**st))
            x = tokens[1]
            u[2] = p0[x] / (q[parent[1], x] if q is not None else 1.0)
            if u[2] >= 1.0:
                u[2] = np.nextafter(1.0, 0.0)
        want = O.accept_tree_s(rows, tokens, parent, O.sampler(**st), q=q, u=u)
        got = E.accept_sample(rows, tokens, parent, E.make_sampler(**st), q=q, u=u)
        assert got == want, (trial, n, V, st)


def test_gpu_accept_sample_reproduces_reference_steps():
    fix = np.load(GOLDEN / "sampling_ref.npz")
    C = fix["chains"]
    for j in range(len(C)):
        rows, draft, seq = fix[f"s{j}_rows"], fix[f"s{j}_draft"], fix[f"s{j}_seq"]
        k = draft.size
        T, tk, tp, mp, rp = (float(x) for x in C[j][:5])
        s = E.make_sampler(T, int(tk), tp, mp, rp, context=seq)
        tokens = np.concatenate([[seq[-1]], draft]).astype(np.int32)
        rc, path, fin = E.accept_sample(rows, tokens, None, s, u=E.chain_uniforms(fix[f"s{j}_stream"], k))
        assert rc == 0 and len(path) - 1 == int(C[j][5]) and fin == int(C[j][6]), j


def test_gpu_accept_sample_rejects_bad_logits_and_settings():
    rows = np.zeros((3, 100), dtype=np.float32)
    rows[1, 5] = np.nan
    s = E.make_sampler(0.0)
    u = np.zeros(6)
    assert E.accept_sample(rows, [0, 0, 0], None, s, u=u)[0] < 0          # row 1 reached
    assert E.accept_sample(rows, [0, 7, 0], None, s, u=u) == (0, [0], 0)   # rejected at row 0
    rows = np.full((2, 10), -np.inf, dtype=np.float32)
    assert E.accept_sample(rows, [0, 3], None, E.make_sampler(1.0), u=np.zeros(4))[0] < 0
    ok = np.zeros((2, 10), dtype=np.float32)
    for bad in [dict(temperature=-1.0), dict(top_p=0.0), dict(top_p=1.5), dict(min_p=2.0),
                dict(repetition_penalty=0.0), dict(top_k=-1)]:
        assert E.accept_sample(ok, [0, 3], None, E.make_sampler(**bad), u=np.zeros(4))[0] < 0


@pytest.fixture(scope="module")
def eng(tiny_model):
    e = E.Engine(tiny_model, max_seq=1024)
    yield e
    e.close()


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def test_verify_sample_matches_oracle_and_commits(eng):
    prompt = container.uniform_ints(21, 50, container.TINY.vocab)
    rng = np.random.default_rng(4)
    V = container.TINY.vocab
    for trial in range(6):
        eng.reset()
        eng.eval(prompt[:-1])
        first = int(np.argmax(eng.eval([prompt[-1]])))
        eng.rewind(49)
        tok = np.array([prompt[-1], first, 11, first, 5, 900, first], dtype=np.int32)
        par = np.array([-1, 0, 0, 1, 1, 2, 3], dtype=np.int32) if trial % 2 else None
        n = tok.size
        st = [dict(temperature=0.8, top_p=0.95), dict(temperature=1.0, top_k=20, repetition_penalty=1.1),
              dict(temperature=0.0)][trial % 3]
        q = None
        if trial >= 3:
            q = rng.random((n, V)) + 0.01
            q /= q.sum(1, keepdims=True)
        u = rng.random(2 * n)
        # trials 4 and 5 hand q over in the GPU's memory (hearth_gpu_verify_sample_dq)
        qa = eng.device_array(q) if trial >= 4 else q
        path, fin, lg = eng.verify_sample(tok, par, E.make_sampler(context=prompt, **st), q=qa, u=u, want_logits=True)
        if trial >= 4:
            qa.free()
        parent = par if par is not None else np.arange(-1, n - 1, dtype=np.int32)
        want = O.accept_tree_s(lg, tok, parent, O.sampler(context=prompt, **st), q=q, u=u)
        assert (0, path, fin) == want, trial
        assert eng.pos == 49 + len(path)
        # the committed KV is the accepted chain's
        nxt = eng.eval([fin])
        eng.rewind(49)
        eng.eval(tok[path])
        assert np.array_equal(_bits(nxt), _bits(eng.eval([fin])))


def test_verify_sample_chain_consumes_reference_uniforms(eng):
    prompt = container.uniform_ints(22, 40, container.TINY.vocab)
    eng.reset()
    eng.eval(prompt[:-1])
    draft = [int(t) for t in container.uniform_ints(23, 4, container.TINY.vocab)]
    rng = np.random.default_rng(99)
    n_acc, fin = eng.verify_sample_chain(int(prompt[-1]), draft, E.make_sampler(0.8, top_p=0.95), rng)
    used = n_acc + (1 if n_acc < len(draft) else 0) + 1
    ref = np.random.default_rng(99)
    ref.random(used)
    assert rng.random() == ref.random()
    assert eng.pos == 39 + n_acc + 1


def test_verify_sample_dq_rejects_host_q(eng):
    """hearth_gpu_verify_sample_dq returns -1, and commits nothing, for q in host memory."""
    import ctypes
    prompt = container.uniform_ints(24, 30, container.TINY.vocab)
    eng.reset()
    eng.eval(prompt[:-1])
    tok = np.array([prompt[-1], 3, 4], dtype=np.int32)
    q = np.full((3, container.TINY.vocab), 1.0 / container.TINY.vocab)
    u = np.full(6, 0.5)
    path, npath, fin = np.zeros(3, dtype=np.int32), ctypes.c_int(0), np.zeros(1, dtype=np.int32)
    smp = E.make_sampler(temperature=0.8)
    I32 = ctypes.POINTER(ctypes.c_int32)
    rc = eng._api.need("gpu_verify_sample_dq")(
        eng._handle(), tok.ctypes.data_as(I32), None, 3, ctypes.byref(smp), q.ctypes.data,
        u.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), path.ctypes.data_as(I32), ctypes.byref(npath),
        fin.ctypes.data_as(I32), None)
    assert rc == -1 and eng.pos == 29
    d = eng.device_array(q)
    with pytest.raises(ValueError):
        eng.verify_sample(tok[:2], None, smp, q=d, u=u)   # [3][V] rows for a 2-node call
    d.free()
    assert d.ptr is None
