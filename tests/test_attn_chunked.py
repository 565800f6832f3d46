"""The chunked attention order (an opt-in order of the GPU engine's GQA layers) in the
oracle.

It has no reference counterpart: the reference lets a GPU backend document its
tolerance (governance/decisions/ADR-0003-canonical-numerics.md:44-45). What pins the
restatement (oracle/hx_oracle.c chunked_head):
- an independent restatement here in exact rational arithmetic (every fmaf, add, multiply
  and divide rounded once to float32 from its exact value) must give the same bits;
- both orders must agree with attention computed in float64 to 1e-5, on contexts of
  one to several chunks (a dropped chunk, a wrong chunk weight or a transposed operand
  breaks that by orders of magnitude);
- closed forms: one row gives its V row exactly; equal scores give the mean of V;
- batch == sequential and tree == chain hold in the chunked order too.
Whole models: the chunked order's head outputs differ from the canonical ones by about
1e-6, and the int8 activation quantizer of these models turns such differences into
logit differences of up to a few 1e-2 on some rows and occasional routing changes; the
model test bounds that from below (a wrong fold would disagree on most rows).
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

import oracle_py as O
from hearth_amd import container

CH = 64


def _f32(x: Fraction) -> float:
    """x rounded to float32, ties to even (normal and subnormal range)"""
    if x == 0:
        return 0.0
    sgn, a = (-1.0, -x) if x < 0 else (1.0, x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)
    ulp = Fraction(2) ** (e - 23)
    m = a / ulp
    r = m.numerator // m.denominator
    rem = m - r
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and r % 2 == 1):
        r += 1
    return sgn * float(r * ulp)


def _fmaf(a, b, c) -> float:
    return _f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def _add(a, b) -> float:
    return _f32(Fraction(float(a)) + Fraction(float(b)))


def _expf(x) -> float:
    return float(O.lib().ho_exp_glibc_f(float(x)))


def _chunked_exact(q, K, V, rows, scale):
    """the chunked order of include/hearth_gpu.h, each operation rounded from its exact value"""
    n, nr = q.size, len(rows)
    s = []
    for i in range(nr):
        acc = 0.0
        for d in range(n):
            acc = _fmaf(q[d], K[rows[i], d], acc)
        s.append(_f32(Fraction(float(np.float32(scale))) * Fraction(acc)))
    nc = (nr + CH - 1) // CH
    mc = [max(s[c * CH:min(c * CH + CH, nr)]) for c in range(nc)]
    M = max(mc)
    L, O_ = 0.0, [0.0] * n
    for c in range(nc):
        i0, i1 = c * CH, min(c * CH + CH, nr)
        a = [_expf(_f32(Fraction(s[i]) - Fraction(mc[c]))) for i in range(i0, i1)] + [0.0] * (CH - (i1 - i0))
        oc = [0.0] * n
        for i in range(i0, i1):
            for d in range(n):
                oc[d] = _fmaf(a[i - i0], V[rows[i], d], oc[d])
        w = 1
        while w < CH:
            for k in range(0, CH, 2 * w):
                a[k] = _add(a[k], a[k + w])
            w *= 2
        wc = _expf(_f32(Fraction(mc[c]) - Fraction(M)))
        L = _fmaf(a[0], wc, L)
        for d in range(n):
            O_[d] = _fmaf(oc[d], wc, O_[d])
    return np.array([_f32(Fraction(O_[d]) / Fraction(L)) for d in range(n)], dtype=np.float32)


def _attn_f64(q, K, V, rows, scale):
    k, v = K[rows].astype(np.float64), V[rows].astype(np.float64)
    s = scale * (k @ q.astype(np.float64))
    p = np.exp(s - s.max())
    return (p / p.sum()) @ v


def _case(seed, nr, n, spread=1.0):
    rng = np.random.default_rng(seed)
    R = nr + 17
    K = (rng.standard_normal((R, n)) * spread).astype(np.float32)
    V = rng.standard_normal((R, n)).astype(np.float32)
    q = rng.standard_normal(n).astype(np.float32)
    rows = rng.permutation(R)[:nr].astype(np.int32)     # rows in any cache order
    return q, K, V, rows, float(np.float32(1.0 / np.sqrt(n)))


@pytest.fixture
def chunked():
    O.gpu_numerics(O.ATTN_CHUNKED)
    yield
    O.gpu_numerics()


@pytest.mark.parametrize("nr,n", [(1, 8), (5, 16), (63, 8), (64, 12), (65, 8), (130, 16), (200, 4)])
def test_chunked_head_equals_exact_restatement(chunked, nr, n):
    q, K, V, rows, scale = _case(1000 + nr, nr, n, spread=2.0)
    got = O.attn_head(q, K, V, rows, scale)
    want = _chunked_exact(q, K, V, rows, scale)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (got, want)


@pytest.mark.parametrize("mode", [O.ATTN_CANONICAL, O.ATTN_CHUNKED])
@pytest.mark.parametrize("nr", [1, 40, 64, 65, 127, 300, 1000])
def test_both_orders_match_float64_attention(mode, nr):
    O.gpu_numerics(mode)
    try:
        for seed in range(3):
            q, K, V, rows, scale = _case(seed * 7919 + nr, nr, 64, spread=3.0)
            got = O.attn_head(q, K, V, rows, scale).astype(np.float64)
            ref = _attn_f64(q, K, V, rows, scale)
            err = np.abs(got - ref).max() / np.abs(ref).max()
            assert err < 1e-5, (mode, nr, seed, err)
    finally:
        O.gpu_numerics()


def test_chunked_closed_forms(chunked):
    rng = np.random.default_rng(3)
    # one row: its V row exactly
    q, K, V, rows, scale = _case(5, 1, 32)
    assert np.array_equal(O.attn_head(q, K, V, rows, scale), V[rows[0]])
    # equal scores (q = 0): every e is 1, l_c counts the chunk's rows, the weights are 1, so
    # the result is the exact sum of V over the rows (small integers) divided by nr
    for nr in (64, 128, 100, 257):
        n = 24
        K = rng.standard_normal((nr, n)).astype(np.float32)
        V = rng.integers(-50, 50, (nr, n)).astype(np.float32)
        rows = np.arange(nr, dtype=np.int32)
        got = O.attn_head(np.zeros(n, np.float32), K, V, rows, 0.125)
        want = np.array([_f32(Fraction(int(V[:, d].sum()), nr)) for d in range(n)], dtype=np.float32)
        assert np.array_equal(got, want), nr


def _rel_err_rows(a, b):
    """per row: max |a - b| / max |b|"""
    return (np.abs(a.astype(np.float64) - b).max(1) / np.abs(b.astype(np.float64)).max(1))


@pytest.mark.parametrize("name", ["tiny", "qwen2", "olmoe"])
def test_model_chunked_close_to_canonical(tiny_model, variant_models, name):
    """Verify steps of 9 tokens from the same 100..460-token contexts, chunked against
    canonical: the argmax and the routes agree on at least 99% of the rows (measured on the
    tiny model: 99.8% and 99.9%), the median row is within 1e-3."""
    path = tiny_model if name == "tiny" else variant_models(name)
    toks = container.uniform_ints(11, 600, 4096)
    O.gpu_numerics(O.ATTN_CANONICAL)
    base = O.Model(path, cap=1024)
    base.eval(toks[:100], logits=False)
    errs, am, ra, n = [], 0, 0, 0
    try:
        for step in range(30):
            ctx = 100 + step * 12
            snap = base.kv_export(ctx)
            out = []
            for mode in (O.ATTN_CANONICAL, O.ATTN_CHUNKED):
                O.gpu_numerics(mode)
                m = O.Model(path, cap=1024)
                m.kv_import(snap, ctx)
                out.append(m.eval(toks[ctx:ctx + 9], routes=True))
            (lc, rc), (lk, rk) = out
            errs.append(_rel_err_rows(lk, lc))
            am += int((lk.argmax(1) == lc.argmax(1)).sum())
            ra += int((np.sort(rk, -1) == np.sort(rc, -1)).all(-1).sum())
            n += 9
            O.gpu_numerics(O.ATTN_CANONICAL)
            base.eval(toks[ctx:ctx + 12], logits=False)
    finally:
        O.gpu_numerics()
    err = np.concatenate(errs)
    assert np.median(err) < 1e-3, np.median(err)
    assert am / n >= 0.99, am / n
    assert ra / (n * rc.shape[1]) >= 0.99, ra / (n * rc.shape[1])


def test_chunked_tree_equals_chain_and_batch_equals_sequential(tiny_model, chunked):
    prompt = container.uniform_ints(5, 150, container.TINY.vocab)
    tok = np.array([17, 5, 9, 300, 4000, 12, 8], dtype=np.int32)
    par = np.array([-1, 0, 0, 1, 1, 2, 4], dtype=np.int32)
    t = O.Model(tiny_model)
    t.eval(prompt, logits=False)
    lt = t.eval_tree(tok, par)
    for node in range(len(tok)):
        path, v = [], node
        while v >= 0:
            path.append(v)
            v = par[v]
        c = O.Model(tiny_model)
        c.eval(prompt, logits=False)
        lc = c.eval(tok[path[::-1]])
        assert np.array_equal(lc[-1].view(np.uint32), lt[node].view(np.uint32)), node
    b = O.Model(tiny_model)
    batch = b.eval(prompt)
    s = O.Model(tiny_model)
    seq = np.concatenate([s.eval(prompt[i:i + 1]) for i in range(len(prompt))])
    assert np.array_equal(batch.view(np.uint32), seq.view(np.uint32))
