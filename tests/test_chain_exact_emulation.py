"""The exact running sum of k_sample.hip (chain_exact), restated on the CPU.

chain_exact computes np.cumsum's float64 chain c_j = fl(c_{j-1} + x_j) a block at a
time: while c stays in one binade [2^e, 2^(e+1)) every c_j is a multiple of u = 2^(e-52),
so fl(c + x) = c + u RN(x / u) and integer prefix sums give every c_j of a block at once.
An entry whose x / u is halfway between two integers (a tie) rounds to even, which
depends on the parity of the units before it; with P_i the units before tie i counting
every earlier tie at its floor and a_i = (P_i + floor_i) mod 2, tie i adds floor_i +
(a_i xor a_(i-1)) (a_0 = 0): the parity of the adjustments so far is always a of the last
tie. An entry that takes the sum out of the binade, or is at least 2^53 u, is added on
its own and the block goes on from it in the new binade; where such entries are close
together the kernel adds 64 entries one after the other instead.

This file restates that procedure with Python integers (no thread partition: the sums
are exact, so the partition cannot change them) and checks it against np.cumsum on
inputs built to hit every case: ties in every position of a block (values of a few
significant bits), chains of ties, binade crossings, entries above the running sum,
subnormals and zeros. No GPU is used; the GPU path is checked against the oracle in
tests/test_gpu_sample.py.
"""
from __future__ import annotations

import math

import numpy as np
import pytest


def _ilogb(c: float) -> int:
    return math.frexp(c)[1] - 1


def chain_emulate(x: np.ndarray, block: int = 256, tie_rule: str = "xor") -> np.ndarray:
    """tie_rule "xor" is chain_exact's; "own" (a tie's adjustment from its own parity
    only) and "floor" (no adjustment) are planted mistakes for the negative control."""
    m = len(x)
    out = np.zeros(m)
    c, j0, in_order = 0.0, 0, True
    while j0 < m:
        if in_order:
            for j in range(j0, min(j0 + 64, m)):
                c = c + float(x[j])
                out[j] = c
            j0 = min(j0 + 64, m)
            in_order = c == 0.0
            continue
        jend = min(j0 + block, m)
        js = j0
        while js < jend:
            e = max(_ilogb(c), -1022)
            u = math.ldexp(1.0, e - 52)
            base = int(c / u)
            fb = jend
            vals = []
            for j in range(js, jend):
                q = math.ldexp(float(x[j]), 52 - e)   # x / u, exact
                if not q < 2.0 ** 53:
                    fb = j
                    break
                f = math.floor(q)
                r = q - f
                d = int(f) + (1 if r > 0.5 else 0)   # a tie at its floor
                vals.append((j, int(f), d, r == 0.5))
            # second pass: the tie parities use the units before each tie at the floor of
            # every earlier tie (P), the true units add the adjustments
            P, D, a_prev, done = base, base, 0, []
            for j, f, d, is_tie in vals:
                adj = 0
                if is_tie:
                    a = (P + f) & 1
                    adj = {"xor": a ^ a_prev, "own": a, "floor": 0}[tie_rule]
                    a_prev = a
                P += d
                D += d + adj
                if D >= 2 ** 53:
                    fb = j
                    break
                done.append((j, D))
            for j, Dj in done:
                out[j] = Dj * u
            if done:
                c = done[-1][1] * u
            if fb < jend:
                c = c + float(x[fb])
                out[fb] = c
                little = fb - js < 64
                js = fb + 1
                if little:
                    in_order = True
                    break
            else:
                js = jend
        j0 = js
    return out


def _check(x):
    want = np.cumsum(x)
    got = chain_emulate(x)
    assert np.array_equal(got.view(np.uint64), want.view(np.uint64))


def _tie_heavy(seed, n=3000, drift=0.0):
    """a running sum near 2^t after its first entry, then entries whose lowest bits sit at
    the sum's ulp or half of it (odd multiples of u / 2 are ties), plus a drift that
    takes the sum across binades"""
    rng = np.random.default_rng(seed)
    t = int(rng.integers(-30, 10))
    k = rng.integers(1, 64, n).astype(np.float64)
    sh = rng.integers(-54, -50, n).astype(np.float64)
    x = k * 2.0 ** (sh + t) + drift * 2.0 ** t
    return np.concatenate([[2.0 ** t], x])


@pytest.mark.parametrize("seed", range(6))
def test_ties_everywhere(seed):
    """x / u exactly halfway for a large share of the entries"""
    _check(_tie_heavy(seed))


@pytest.mark.parametrize("seed", range(4))
def test_ties_across_binades(seed):
    _check(_tie_heavy(seed, n=4000, drift=2.0 ** -10))


def test_ties_in_a_row():
    x = np.array([1.0] + [0.5 * 2.0 ** -52] * 300 + [1.5 * 2.0 ** -52] * 300 + [2.5 * 2.0 ** -52] * 300)
    _check(x)


@pytest.mark.parametrize("seed", range(4))
def test_probabilities(seed):
    """rows like the draw's: a normalized distribution in index order"""
    rng = np.random.default_rng(100 + seed)
    z = rng.normal(0, [0.5, 1.0, 2.0, 4.0][seed], 5000)
    p = np.exp(z - z.max())
    p /= p.sum()
    _check(p)


def test_crossings_huge_entries_subnormals_and_zeros():
    rng = np.random.default_rng(7)
    parts = [np.zeros(70), rng.uniform(0, 1, 500) * 2.0 ** -1074 * 64, rng.uniform(0, 1, 500) * 1e-300,
             np.zeros(3), 2.0 ** rng.integers(-60, 2, 800).astype(np.float64), rng.uniform(0, 1e-8, 900)]
    _check(np.concatenate(parts))


@pytest.mark.parametrize("rule", ["own", "floor"])
def test_catches_planted_mistakes(rule):
    """negative control: a tie adjusted from its own parity only (ignoring the earlier
    ties' adjustments), or never adjusted, differs from np.cumsum"""
    x = _tie_heavy(3)
    got = chain_emulate(x, tie_rule=rule)
    assert not np.array_equal(got.view(np.uint64), np.cumsum(x).view(np.uint64))
