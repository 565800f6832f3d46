"""Sampled acceptance: the CPU restatement (oracle/hx_oracle.c ho_probs_s, ho_draw,
ho_accept_point_mass, ho_accept_tree_s) pinned against

- numpy itself: ho_np_sum is numpy's float64 pairwise sum, bit for bit, at every size;
- the reference's own sampling code (python/hearth/generate.py Sampler.probs, draw,
  accept_point_mass, generate() lines 376-392), through the vectors in
  tests/golden/sampling_ref.npz written by tests/golden/make_sampling_golden.py. The
  reference exponentiates with np.exp and the restatement with the portable exp, so the
  float64 distributions agree to a few ulps, with identical support; every draw and
  acceptance decision is identical;
- closed forms: temperature 0 gives greedy acceptance; recursive rejection sampling over
  a tree's children leaves the emitted token distributed as p (chi-square, with a
  negative control that must fail).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle_py as O
from golden_io import GOLDEN

FIX = GOLDEN / "sampling_ref.npz"


@pytest.fixture(scope="module")
def fix():
    return np.load(FIX)


def _s(row, ctx=()):
    T, tk, tp, mp, rp = row[:5]
    return O.sampler(float(T), int(tk), float(tp), float(mp), float(rp), ctx)


def test_np_sum_is_numpy_pairwise_sum():
    rng = np.random.default_rng(3)
    for n in list(range(0, 260)) + [511, 1000, 4096, 8191, 65537, 151936]:
        a = rng.random(n) * rng.choice([1.0, 1e-3, 1e6], n)
        assert O.np_sum(a) == np.sum(a), n


def test_probs_match_reference(fix):
    S = fix["settings"]
    assert len(S) >= 40
    for i in range(len(S)):
        rc, p = O.probs_s(fix[f"c{i}_logits"], _s(S[i], fix[f"c{i}_ctx"]))
        ref = fix[f"c{i}_p"]
        assert rc == 0
        assert np.array_equal(p == 0, ref == 0), i
        nz = ref > 0
        assert np.max(np.abs(p[nz] - ref[nz]) / ref[nz]) <= 4e-15, i


def test_draw_and_point_mass_match_reference(fix):
    S = fix["settings"]
    for i in range(len(S)):
        _, p = O.probs_s(fix[f"c{i}_logits"], _s(S[i], fix[f"c{i}_ctx"]))
        if S[i][0] > 0:
            for u, d in zip(fix[f"c{i}_draw_u"], fix[f"c{i}_draw"]):
                assert O.lib().ho_draw(p.ctypes.data_as(O._DP), p.size, float(u)) == d, (i, u)
        for d, u0, u1, ok, tok in fix[f"c{i}_acc"]:
            t = ctypes.c_int(0)
            r = O.lib().ho_accept_point_mass(p.ctypes.data_as(O._DP), p.size, int(d), float(u0), float(u1),
                                             ctypes.byref(t))
            assert (r, t.value) == (int(ok), int(tok)), (i, d)


def chain_uniforms(stream, k):
    """The reference draws one uniform per tried draft and one for the final token, in
    that order; in the restatement's layout u[2c] decides node c and u[2v + 1] draws at
    node v (after the child v + 1 was rejected, or the bonus at v = k)."""
    u = np.zeros(2 * (k + 1))
    for c in range(1, k + 1):
        u[2 * c] = stream[c - 1]
    for v in range(k):
        u[2 * v + 1] = stream[v + 1]
    u[2 * k + 1] = stream[k]
    return u


def test_chain_steps_match_reference(fix):
    C = fix["chains"]
    for j in range(len(C)):
        rows, draft, seq = fix[f"s{j}_rows"], fix[f"s{j}_draft"], fix[f"s{j}_seq"]
        k = draft.size
        s = _s(C[j], seq)
        tokens = np.concatenate([[seq[-1]], draft])
        rc, path, fin = O.accept_tree_s(rows, tokens, np.arange(-1, k), s, u=chain_uniforms(fix[f"s{j}_stream"], k))
        n_acc, final, used = int(C[j][5]), int(C[j][6]), int(C[j][7])
        assert rc == 0 and path == list(range(n_acc + 1)) and fin == final, j
        assert used == n_acc + (1 if n_acc < k else 0) + 1


def test_temperature_zero_is_greedy():
    rng = np.random.default_rng(5)
    for trial in range(150):
        n, V = int(rng.integers(1, 10)), int(rng.integers(2, 40))
        rows = rng.integers(-3, 4, size=(n, V)).astype(np.float32)
        parent = np.array([-1] + [int(rng.integers(0, i)) for i in range(1, n)], dtype=np.int32)
        tokens = rng.integers(0, V, n).astype(np.int32)
        for c in range(1, n):   # make some children the argmax of their parent
            if rng.random() < 0.6:
                tokens[c] = rows[parent[c]].argmax()
        u = rng.random(2 * n)
        g = O.accept_tree(rows, tokens, parent)
        assert O.accept_tree_s(rows, tokens, parent, O.sampler(0.0), u=u) == g
        q = rng.random((n, V)) + 0.1
        q /= q.sum(1, keepdims=True)
        assert O.accept_tree_s(rows, tokens, parent, O.sampler(0.0), q=q, u=u) == g


def _emitted(rows, tokens, parent, s, q, u):
    rc, path, fin = O.accept_tree_s(rows, tokens, parent, s, q=q, u=u)
    assert rc == 0
    return int(tokens[path[1]]) if len(path) > 1 else fin


def _chi2_first_token(rows, s, q_draw, q_claim, n_children, trials, rng, fixed=None):
    """Emitted token after the root, children drafted i.i.d. from q_draw (or fixed
    tokens with point-mass acceptance); returns (chi2, dof) against p."""
    V = rows.shape[1]
    _, p = O.probs_s(rows[0], s)
    n = 1 + n_children
    parent = np.array([-1] + [0] * n_children, dtype=np.int32)
    counts = np.zeros(V)
    q = None if q_claim is None else np.tile(q_claim, (n, 1))
    for _ in range(trials):
        if fixed is None:
            kids = rng.choice(V, size=n_children, p=q_draw)
        else:
            kids = fixed
        tokens = np.concatenate([[0], kids]).astype(np.int32)
        counts[_emitted(rows, tokens, parent, s, q, rng.random(2 * n))] += 1
    m = p > 0
    e = trials * p[m]
    return float(np.sum((counts[m] - e) ** 2 / e)), int(m.sum()) - 1, counts[~m].sum()


def test_tree_rejection_sampling_preserves_target():
    rng = np.random.default_rng(11)
    V = 8
    rows = rng.normal(0, 1.2, (4, V)).astype(np.float32)
    s = O.sampler(0.9, top_p=0.97)
    q = rng.random(V) + 0.05
    q /= q.sum()
    # chi-square 0.999 quantile for <= 7 dof is < 24.4
    chi2, dof, outside = _chi2_first_token(rows, s, q, q, 3, 6000, rng)
    assert outside == 0 and chi2 < 24.4, (chi2, dof)
    chi2, dof, outside = _chi2_first_token(rows, s, None, None, 3, 6000, rng, fixed=np.array([2, 5, 2]))
    assert outside == 0 and chi2 < 24.4, (chi2, dof)
    # negative control: claiming a draft distribution other than the one drafted from
    # breaks the guarantee, and the test must see it
    wrong = np.roll(q, 3)
    chi2, dof, _ = _chi2_first_token(rows, s, q, wrong, 3, 6000, rng)
    assert chi2 > 60.0, chi2
