"""hearth_gpu_accept_greedy_noalloc (device buffers, scratch in a fixed library array)
against hearth_gpu_accept_greedy (host buffers, scratch from hipMalloc) on the same
logits: two calls in a row, the second smaller, then a tree, bad rows and the size
limit. The test allocates the caller's device buffers itself (through the HIP runtime);
the entry point under test allocates nothing."""
from __future__ import annotations

import ctypes
from ctypes import POINTER, byref, c_float, c_int, c_int32, c_size_t, c_void_p

import numpy as np
import pytest

from hearth_amd import _native
from hearth_amd.engine import accept_greedy

pytestmark = pytest.mark.gpu

H2D, D2H = 1, 2


class _Hip:
    def __init__(self):
        self.L = ctypes.CDLL("libamdhip64.so")
        self.bufs = []

    def ck(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed ({rc})")

    def put(self, a: np.ndarray) -> c_void_p:
        a = np.ascontiguousarray(a)
        p = c_void_p()
        self.ck(self.L.hipMalloc(byref(p), c_size_t(max(a.nbytes, 4))), "hipMalloc")
        self.bufs.append(p)
        if a.nbytes:
            self.ck(self.L.hipMemcpy(p, a.ctypes.data_as(c_void_p), c_size_t(a.nbytes), H2D), "hipMemcpy H2D")
        return p

    def get(self, p: c_void_p, like: np.ndarray) -> np.ndarray:
        out = np.empty_like(like)
        self.ck(self.L.hipMemcpy(out.ctypes.data_as(c_void_p), p, c_size_t(out.nbytes), D2H), "hipMemcpy D2H")
        return out

    def sync(self):
        self.ck(self.L.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def free(self):
        for p in self.bufs:
            self.L.hipFree(p)
        self.bufs.clear()


@pytest.fixture()
def hip():
    h = _Hip()
    yield h
    h.free()


def _noalloc():
    fn = _native.lib().hearth_gpu_accept_greedy_noalloc
    fn.restype = c_int
    fn.argtypes = [c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]
    return fn


def _run_noalloc(hip, rows, tokens, parent):
    n, V = rows.shape
    d_rows = hip.put(rows.astype(np.float32))
    d_tok = hip.put(np.asarray(tokens, dtype=np.int32))
    d_par = None if parent is None else hip.put(np.asarray(parent, dtype=np.int32))
    d_path = hip.put(np.full(n, -7, dtype=np.int32))
    d_res = hip.put(np.full(3, -7, dtype=np.int32))
    rc = _noalloc()(d_rows, n, V, d_tok, d_par, d_path, d_res, None)
    assert rc == 0, rc
    hip.sync()
    res = hip.get(d_res, np.zeros(3, dtype=np.int32))
    path = hip.get(d_path, np.zeros(n, dtype=np.int32))
    return int(res[2]), path[:max(int(res[0]), 0)].tolist(), int(res[1])


def _chain_case(seed, n, V, n_good):
    rng = np.random.default_rng(seed)
    rows = rng.standard_normal((n, V)).astype(np.float32)
    am = rows.argmax(1)
    tokens = rng.integers(0, V, n).astype(np.int32)
    for i in range(1, n_good + 1):           # node i accepted when it is the argmax of node i - 1
        tokens[i] = am[i - 1]
    return rows, tokens


def test_noalloc_matches_allocating_entry_two_calls(hip):
    for seed, n, V, good in ((1, 9, 151936, 4), (2, 5, 4096, 1)):    # second call smaller
        rows, tokens = _chain_case(seed, n, V, good)
        st, path, fin = _run_noalloc(hip, rows, tokens, None)
        rc, rpath, rfin = accept_greedy(rows, tokens)
        assert rc == 0 and st == 0
        assert path == rpath == list(range(good + 1)) and fin == rfin


def test_noalloc_tree_and_bad_rows(hip):
    rng = np.random.default_rng(5)
    V = 1000
    parent = np.array([-1, 0, 0, 1, 1, 2, 3], dtype=np.int32)
    rows = rng.standard_normal((len(parent), V)).astype(np.float32)
    am = rows.argmax(1)
    tokens = rng.integers(0, V, len(parent)).astype(np.int32)
    tokens[2] = am[0]                       # second child of the root is the argmax
    tokens[5] = am[2]
    st, path, fin = _run_noalloc(hip, rows, tokens, parent)
    rc, rpath, rfin = accept_greedy(rows, tokens, parent)
    assert st == rc == 0 and path == rpath == [0, 2, 5] and fin == rfin
    rows[0, 17] = np.nan                    # the reference raises on NaN logits
    st, _, _ = _run_noalloc(hip, rows, tokens, parent)
    rc, _, _ = accept_greedy(rows, tokens, parent)
    assert st == -1 and rc == -1


def test_noalloc_rejects_rows_past_its_scratch(hip):
    limit = 1024
    d = hip.put(np.zeros(8, dtype=np.int32))
    assert _noalloc()(d, limit + 1, 4, d, None, d, d, None) == -3
    assert _noalloc()(None, 4, 4, d, None, d, d, None) == -1


def test_noalloc_leaves_the_callers_pending_error(hip):
    """A HIP error the calling thread has not read yet is not cleared or taken for this
    call's own: the call returns -4 without launching, the error stays pending, and once
    the caller reads it the call works."""
    L = hip.L
    L.hipPeekAtLastError.restype = c_int
    L.hipGetLastError.restype = c_int
    rows, tokens = _chain_case(3, 4, 256, 1)
    d_rows, d_tok = hip.put(rows), hip.put(tokens)
    d_path, d_res = hip.put(np.zeros(4, dtype=np.int32)), hip.put(np.zeros(3, dtype=np.int32))
    L.hipGetLastError()
    assert L.hipSetDevice(c_int(4096)) != 0          # no such device: the thread now holds an error
    pending = L.hipPeekAtLastError()
    assert pending != 0
    assert _noalloc()(d_rows, 4, 256, d_tok, None, d_path, d_res, None) == -4
    assert L.hipPeekAtLastError() == pending
    assert L.hipGetLastError() == pending            # the caller reads (and clears) it
    st, path, fin = _run_noalloc(hip, rows, tokens, None)
    rc, rpath, rfin = accept_greedy(rows, tokens)
    assert st == rc == 0 and path == rpath == [0, 1] and fin == rfin
