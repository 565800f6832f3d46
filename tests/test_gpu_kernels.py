"""GPU kernels through the C ABI against the reference's known answers and the oracle.

- hearth_matmul on the GPU reproduces the reference's pinned kernel hashes
  (engine/tests/test_quant.c:923-931) for F32/F16/BF16/Q8/Q4, libm-free inputs;
- the int8-MFMA Q8/Q4 GEMM: T tokens in one call equal T single-token calls and the
  oracle bit for bit, across shapes with pad rows, odd block counts and the input kinds
  of the reference's tests (zero blocks, outliers, .5 ties, tiny values, NaN); T > 16
  takes the resident-weight kernel, with token tiles split over workgroups where the
  row tiles are few (T = 17, 23, 40, 85; K up to 4096);
- the greedy acceptance kernel equals the oracle's walk on tie-heavy random logits,
  chains and trees.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import kat
import oracle_py as O
from hearth_amd import _native

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [0, 1, 2, 3, 4])
def test_gpu_matmul_pinned_hashes(dtype):
    W, X = kat.pinned_inputs()
    q = _native.quantize(dtype, W)
    Y = _native.matmul(dtype, q, kat.R, kat.C, X)
    assert kat.fnv1a(Y.tobytes()) == kat.PIN_Y[dtype]


def _kind(rng, kind, rows, cols):
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    if kind == "zero_blocks":
        x.reshape(rows, -1, 64)[:, ::2] = 0.0
    elif kind == "outlier":
        x[rng.integers(rows), rng.integers(cols)] = 3e4
    elif kind == "ties":
        x = (rng.integers(-126, 127, (rows, cols)) + np.where(rng.random((rows, cols)) < 0.5, 0.5, -0.5)).astype(np.float32)
        x = np.clip(x, -127, 127)
        x[:, ::64] = 127.0
    elif kind == "tiny":
        x = x * np.where(rng.random((rows, cols)) < 0.5, 1e-30, 1e-41).astype(np.float32)
    elif kind == "nan":
        x[rng.random((rows, cols)) < 0.01] = np.nan
    return x


@pytest.mark.parametrize("dtype", [3, 4])
@pytest.mark.parametrize("rows,cols,T", [(16, 64, 1), (37, 192, 5), (250, 2048, 9), (96, 128, 40), (300, 768, 17),
                                         (48, 4096, 85), (33, 2112, 23)])
@pytest.mark.parametrize("kind", ["gauss", "zero_blocks", "outlier", "ties", "tiny", "nan"])
def test_gpu_gemm_equals_oracle_and_single_tokens(dtype, rows, cols, T, kind):
    rng = np.random.default_rng(rows * 31 + cols + T)
    W = rng.standard_normal((rows, cols)).astype(np.float32)
    X = _kind(rng, kind, T, cols)
    q = _native.quantize(dtype, W)
    Yg = _native.matmul(dtype, q, rows, cols, X)
    Yo = O.matmul(dtype, q, rows, cols, X)
    assert np.array_equal(Yg.view(np.uint32), Yo.view(np.uint32))
    for t in (0, T - 1):
        Y1 = _native.matmul(dtype, q, rows, cols, X[t:t + 1])
        assert np.array_equal(Y1[0].view(np.uint32), Yg[t].view(np.uint32))


def _accept_gpu(rows, tokens, parent):
    L = _native.lib()
    rows = np.ascontiguousarray(rows, dtype=np.float32)
    n, V = rows.shape
    t = np.ascontiguousarray(tokens, dtype=np.int32)
    p = np.ascontiguousarray(parent, dtype=np.int32)
    path = np.zeros(n, dtype=np.int32)
    npath, fin = ctypes.c_int(0), np.zeros(1, dtype=np.int32)
    I = ctypes.POINTER(ctypes.c_int32)
    rc = L.hearth_gpu_accept_greedy(rows.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), n, V, t.ctypes.data_as(I),
                                    p.ctypes.data_as(I), path.ctypes.data_as(I), ctypes.byref(npath), fin.ctypes.data_as(I))
    return rc, path[:npath.value].tolist(), int(fin[0])


def test_gpu_greedy_acceptance_equals_oracle():
    rng = np.random.default_rng(5)
    for trial in range(60):
        n, V = int(rng.integers(1, 30)), int(rng.integers(2, 3000))
        rows = rng.integers(-2, 3, size=(n, V)).astype(np.float32)   # heavy ties: first index must win
        parent = np.array([-1] + [int(rng.integers(0, i)) for i in range(1, n)], dtype=np.int32)
        am = rows.argmax(1)
        tokens = np.array([0] + [int(am[parent[i]]) if rng.random() < 0.5 else int(rng.integers(0, V))
                                 for i in range(1, n)], dtype=np.int32)
        assert _accept_gpu(rows, tokens, parent) == O.accept_tree(rows, tokens, parent)


def test_gpu_greedy_acceptance_rejects_bad_logits():
    """A row the walk reaches with NaN / +inf / all -inf logits fails the call, as the
    reference Sampler raises (generate.py:69-79); rows it never reaches do not matter."""
    rows = np.zeros((3, 100), dtype=np.float32)
    rows[1, 5] = np.nan
    assert _accept_gpu(rows, [0, 0, 0], [-1, 0, 1])[0] < 0       # draft 1 accepted -> row 1 read
    assert _accept_gpu(rows, [0, 7, 0], [-1, 0, 1]) == (0, [0], 0)  # draft 1 rejected at row 0
    rows = np.full((2, 10), -np.inf, dtype=np.float32)
    assert _accept_gpu(rows, [0, 3], [-1, 0])[0] < 0
    rows = np.zeros((2, 10), dtype=np.float32)
    rows[0, 4] = np.inf
    assert _accept_gpu(rows, [0, 3], [-1, 0])[0] < 0
