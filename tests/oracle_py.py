"""ctypes wrapper of the CPU restatement (oracle/liboracle.so) for the tests.

Test infrastructure: the oracle is the checker, never the thing measured or shipped.
"""
from __future__ import annotations

import ctypes
import subprocess
from ctypes import POINTER, c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE = ROOT / "oracle" / "liboracle.so"
REF_LIB = ROOT / "oracle" / "_ref" / "libhearth_ref.so"

EXP_LIBM, EXP_PORTABLE, EXP_GLIBC = 0, 1, 2
ATTN_CANONICAL, ATTN_CHUNKED = 0, 1
_I32P, _FP, _DP = POINTER(c_int32), POINTER(c_float), POINTER(c_double)
_lib = None


class Sampler(ctypes.Structure):
    """ho_sampler (oracle/hx_oracle.h)."""
    _fields_ = [("temperature", c_double), ("top_k", c_int), ("top_p", c_double), ("min_p", c_double),
                ("repetition_penalty", c_double), ("context", _I32P), ("n_context", c_int)]


def sampler(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, repetition_penalty=1.0, context=()):
    ctx = np.ascontiguousarray(context, dtype=np.int32)
    s = Sampler(temperature, top_k, top_p, min_p, repetition_penalty,
                ctx.ctypes.data_as(_I32P) if ctx.size else None, int(ctx.size))
    s._keep = ctx
    return s


def lib():
    global _lib
    if _lib is None:
        if not ORACLE.is_file():
            subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "oracle"], check=True)
        L = ctypes.CDLL(str(ORACLE))
        L.ho_row_bytes.restype = c_size_t
        L.ho_row_bytes.argtypes = [c_int, c_int64]
        L.ho_quantize.argtypes = [c_int, _FP, c_int64, c_int64, c_void_p]
        L.ho_dequantize.argtypes = [c_int, c_void_p, c_int64, c_int64, _FP]
        L.ho_act_quant.argtypes = [_FP, c_int64, c_void_p]
        L.ho_matmul.argtypes = [c_int, c_void_p, c_int64, c_int64, _FP, c_int, _FP]
        L.ho_set_exp_mode.argtypes = [c_int]
        L.ho_set_attn_mode.argtypes = [c_int]
        L.ho_set_margins.argtypes = [c_void_p, _FP]
        L.ho_attn_head.argtypes = [_FP, _FP, _FP, c_size_t, _I32P, c_int, c_int, c_float, _FP]
        L.ho_expf.restype = c_float
        L.ho_expf.argtypes = [c_float]
        L.ho_exp_port_f.restype = c_float
        L.ho_exp_port_f.argtypes = [c_float]
        L.ho_exp_glibc_f.restype = c_float
        L.ho_exp_glibc_f.argtypes = [c_float]
        L.ho_exp_glibc_mismatches.restype = ctypes.c_uint64
        L.ho_exp_glibc_mismatches.argtypes = [ctypes.c_uint64, ctypes.c_uint64, c_int]
        L.ho_exp_port_d.restype = c_double
        L.ho_exp_port_d.argtypes = [c_double]
        L.ho_open.restype = c_void_p
        L.ho_open.argtypes = [ctypes.c_char_p, c_int, ctypes.c_char_p, c_size_t]
        L.ho_close.argtypes = [c_void_p]
        L.ho_info.argtypes = [c_void_p, POINTER(c_int)]
        L.ho_pos.argtypes = [c_void_p]
        L.ho_rewind.argtypes = [c_void_p, c_int]
        L.ho_eval.argtypes = [c_void_p, _I32P, c_int, _FP, _I32P]
        L.ho_eval_tree.argtypes = [c_void_p, _I32P, _I32P, c_int, _FP, _I32P]
        L.ho_commit_path.argtypes = [c_void_p, _I32P, c_int]
        L.ho_set_threads.argtypes = [c_void_p, c_int]
        L.ho_set_replay.argtypes = [c_void_p, POINTER(ctypes.c_uint16), c_int64]
        L.ho_kv_row_floats.restype = c_int64
        L.ho_kv_row_floats.argtypes = [c_void_p]
        L.ho_kv_export.argtypes = [c_void_p, c_int, _FP]
        L.ho_kv_import.argtypes = [c_void_p, c_int, _FP]
        L.ho_probs.argtypes = [_FP, c_int, c_double, c_int, c_double, c_double, _DP]
        L.ho_argmax.argtypes = [_FP, c_int]
        L.ho_draw.argtypes = [_DP, c_int, c_double]
        L.ho_accept_point_mass.argtypes = [_DP, c_int, c_int, c_double, c_double, POINTER(c_int)]
        L.ho_accept_general.argtypes = [_DP, _DP, c_int, c_int, c_double, c_double, POINTER(c_int)]
        L.ho_accept_tree.argtypes = [_FP, c_int, c_int, _I32P, _I32P, c_int, c_double, c_int, c_double, c_double,
                                     _DP, _DP, _I32P, POINTER(c_int), POINTER(c_int)]
        L.ho_np_sum.restype = c_double
        L.ho_np_sum.argtypes = [_DP, c_int64]
        L.ho_probs_s.argtypes = [_FP, c_int, POINTER(Sampler), _I32P, c_int, _DP]
        L.ho_accept_tree_s.argtypes = [_FP, c_int, c_int, _I32P, _I32P, POINTER(Sampler), _DP, _DP, _I32P,
                                       POINTER(c_int), POINTER(c_int)]
        _lib = L
    return _lib


def set_exp_mode(mode: int) -> None:
    lib().ho_set_exp_mode(mode)


def set_attn_mode(mode: int) -> None:
    lib().ho_set_attn_mode(mode)


def attn_head(q, K, V, rows, scale: float) -> np.ndarray:
    """ho_attn_head in the current modes: q [n], K and V [R][n] float32, rows [nr]"""
    q = np.ascontiguousarray(q, dtype=np.float32)
    K = np.ascontiguousarray(K, dtype=np.float32)
    V = np.ascontiguousarray(V, dtype=np.float32)
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    out = np.zeros(q.size, dtype=np.float32)
    rc = lib().ho_attn_head(q.ctypes.data_as(_FP), K.ctypes.data_as(_FP), V.ctypes.data_as(_FP), K.shape[1],
                            rows.ctypes.data_as(_I32P), rows.size, q.size, scale, out.ctypes.data_as(_FP))
    assert rc == 0, rc
    return out


def gpu_numerics(attn: int = ATTN_CANONICAL) -> None:
    """the oracle mode the GPU build matches bit for bit: its exp, and the attention order
    (the engine's default, canonical, unless given)"""
    set_exp_mode(EXP_GLIBC)
    set_attn_mode(attn)


def reference_numerics() -> None:
    """the oracle mode the reference engine matches bit for bit (the platform libm, the
    canonical attention order)"""
    set_exp_mode(EXP_LIBM)
    set_attn_mode(ATTN_CANONICAL)


def quantize(dtype: int, x) -> bytes:
    a = np.ascontiguousarray(x, dtype=np.float32)
    a = a.reshape(1, -1) if a.ndim == 1 else a
    rb = lib().ho_row_bytes(dtype, a.shape[1])
    out = np.empty(a.shape[0] * rb, dtype=np.uint8)
    assert lib().ho_quantize(dtype, a.ctypes.data_as(_FP), a.shape[0], a.shape[1], out.ctypes.data_as(c_void_p)) == 0
    return out.tobytes()


def matmul(dtype: int, W: bytes, rows: int, cols: int, X) -> np.ndarray:
    x = np.ascontiguousarray(X, dtype=np.float32).reshape(-1, cols)
    y = np.empty((x.shape[0], rows), dtype=np.float32)
    w = np.frombuffer(W, dtype=np.uint8)
    assert lib().ho_matmul(dtype, w.ctypes.data_as(c_void_p), rows, cols, x.ctypes.data_as(_FP), x.shape[0],
                           y.ctypes.data_as(_FP)) == 0
    return y


class Model:
    """The restatement's forward pass over a container (single-token loop)."""

    def __init__(self, path, cap: int = 0, threads: int = 1):
        err = ctypes.create_string_buffer(512)
        h = lib().ho_open(str(path).encode(), cap, err, len(err))
        if not h:
            raise RuntimeError(err.value.decode())
        self.h = c_void_p(h)
        info = (c_int * 12)()
        lib().ho_info(self.h, info)
        (self.n_layers, self.d_model, self.vocab, self.n_heads, self.n_kv_heads, self.head_dim, self.n_experts,
         self.top_k, self.expert_ffn, self.n_moe, self.cap, self.attn_kind) = list(info)
        lib().ho_set_threads(self.h, threads)

    def close(self):
        if self.h:
            lib().ho_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    @property
    def pos(self) -> int:
        return lib().ho_pos(self.h)

    def rewind(self, pos: int) -> None:
        assert lib().ho_rewind(self.h, pos) == 0

    def eval_margins(self, tokens):
        """logits, routes and the routing margins [n][n_moe] (ho_set_margins) of a chain eval"""
        t = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
        mg = np.empty((t.size, max(self.n_moe, 1)), dtype=np.float32)
        lib().ho_set_margins(self.h, mg.ctypes.data_as(_FP))
        lg, rt = self.eval(t, routes=True)
        return lg, rt, mg

    def eval(self, tokens, routes: bool = False, logits: bool = True):
        """logits [n][V] (None with logits=False: the head is skipped), and routes
        [n][n_moe][K] with routes=True"""
        t = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
        lg = np.empty((t.size, self.vocab), dtype=np.float32) if logits else None
        rt = np.empty((t.size, max(self.n_moe, 1), max(self.top_k, 1)), dtype=np.int32) if routes else None
        rc = lib().ho_eval(self.h, t.ctypes.data_as(_I32P), t.size, lg.ctypes.data_as(_FP) if logits else None,
                           rt.ctypes.data_as(_I32P) if routes else None)
        if rc != 0:
            raise RuntimeError(f"ho_eval {rc}")
        return (lg, rt) if routes else lg

    def eval_tree(self, tokens, parent, routes: bool = False):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        p = np.ascontiguousarray(parent, dtype=np.int32)
        lg = np.empty((t.size, self.vocab), dtype=np.float32)
        rt = np.empty((t.size, max(self.n_moe, 1), max(self.top_k, 1)), dtype=np.int32) if routes else None
        rc = lib().ho_eval_tree(self.h, t.ctypes.data_as(_I32P), p.ctypes.data_as(_I32P), t.size,
                                lg.ctypes.data_as(_FP), rt.ctypes.data_as(_I32P) if routes else None)
        if rc != 0:
            raise RuntimeError(f"ho_eval_tree {rc}")
        return (lg, rt) if routes else lg

    def commit_path(self, path) -> None:
        p = np.ascontiguousarray(path, dtype=np.int32)
        assert lib().ho_commit_path(self.h, p.ctypes.data_as(_I32P), p.size) == 0

    def kv_export(self, n: int | None = None) -> np.ndarray:
        """KV rows of positions [0, n) in the layout of hearth_gpu_kv_export"""
        n = self.pos if n is None else int(n)
        w = lib().ho_kv_row_floats(self.h)
        out = np.empty((self.n_layers, n * w), dtype=np.float32)
        assert lib().ho_kv_export(self.h, n, out.ctypes.data_as(_FP)) == 0
        return out

    def kv_import(self, snap, n: int) -> None:
        a = np.ascontiguousarray(snap, dtype=np.float32)
        assert a.size >= self.n_layers * n * lib().ho_kv_row_floats(self.h)
        assert lib().ho_kv_import(self.h, int(n), a.ctypes.data_as(_FP)) == 0

    def set_replay(self, ids) -> None:
        """route replay: ids [rows][n_moe][K] (uint16), or None for routing"""
        if ids is None:
            assert lib().ho_set_replay(self.h, None, 0) == 0
            return
        a = np.ascontiguousarray(ids, dtype=np.uint16)
        assert lib().ho_set_replay(self.h, a.ctypes.data_as(POINTER(ctypes.c_uint16)), a.shape[0]) == 0


def write_trace(path, ids, n_layers: int, n_experts: int) -> None:
    """a routing trace file (FORMAT.md §9), written by the package's writer"""
    from hearth_amd import container
    container.write_route_trace(path, ids, n_layers, n_experts)


def synthetic_routes(seed: int, rows: int, n_moe: int, n_experts: int, k: int) -> np.ndarray:
    """rows of K distinct experts per MoE layer"""
    rng = np.random.default_rng(seed)
    out = np.empty((rows, n_moe, k), dtype=np.uint16)
    for r in range(rows):
        for m in range(n_moe):
            out[r, m] = rng.choice(n_experts, size=k, replace=False)
    return out


def accept_tree(rows, tokens, parent, mode=0, temperature=0.0, top_k=0, top_p=1.0, min_p=0.0, q=None, u=None):
    rows = np.ascontiguousarray(rows, dtype=np.float32)
    n, V = rows.shape
    t = np.ascontiguousarray(tokens, dtype=np.int32)
    p = np.ascontiguousarray(parent, dtype=np.int32)
    qq = None if q is None else np.ascontiguousarray(q, dtype=np.float64)
    uu = np.zeros(2 * n + 2) if u is None else np.ascontiguousarray(u, dtype=np.float64)
    path = np.zeros(n, dtype=np.int32)
    npath, fin = c_int(0), c_int(0)
    rc = lib().ho_accept_tree(rows.ctypes.data_as(_FP), n, V, t.ctypes.data_as(_I32P), p.ctypes.data_as(_I32P), mode,
                              temperature, top_k, top_p, min_p, None if qq is None else qq.ctypes.data_as(_DP),
                              uu.ctypes.data_as(_DP), path.ctypes.data_as(_I32P), ctypes.byref(npath), ctypes.byref(fin))
    return rc, path[:npath.value].tolist(), fin.value


def probs(logits, temperature, top_k=0, top_p=1.0, min_p=0.0):
    x = np.ascontiguousarray(logits, dtype=np.float32)
    out = np.empty(x.size, dtype=np.float64)
    rc = lib().ho_probs(x.ctypes.data_as(_FP), x.size, temperature, top_k, top_p, min_p, out.ctypes.data_as(_DP))
    return rc, out


def np_sum(a) -> float:
    x = np.ascontiguousarray(a, dtype=np.float64)
    return lib().ho_np_sum(x.ctypes.data_as(_DP), x.size)


def probs_s(logits, s: Sampler, extra=()):
    x = np.ascontiguousarray(logits, dtype=np.float32)
    e = np.ascontiguousarray(extra, dtype=np.int32)
    out = np.empty(x.size, dtype=np.float64)
    rc = lib().ho_probs_s(x.ctypes.data_as(_FP), x.size, ctypes.byref(s), e.ctypes.data_as(_I32P) if e.size else None,
                          int(e.size), out.ctypes.data_as(_DP))
    return rc, out


def accept_tree_s(rows, tokens, parent, s: Sampler, q=None, u=None):
    """Sampled tree acceptance with a sampler: point-mass when q is None, general q
    otherwise. Returns (rc, path, final token)."""
    rows = np.ascontiguousarray(rows, dtype=np.float32)
    n, V = rows.shape
    t = np.ascontiguousarray(tokens, dtype=np.int32)
    p = np.ascontiguousarray(parent, dtype=np.int32)
    qq = None if q is None else np.ascontiguousarray(q, dtype=np.float64)
    uu = np.zeros(2 * n) if u is None else np.ascontiguousarray(u, dtype=np.float64)
    path = np.zeros(n, dtype=np.int32)
    npath, fin = c_int(0), c_int(0)
    rc = lib().ho_accept_tree_s(rows.ctypes.data_as(_FP), n, V, t.ctypes.data_as(_I32P), p.ctypes.data_as(_I32P),
                                ctypes.byref(s), None if qq is None else qq.ctypes.data_as(_DP), uu.ctypes.data_as(_DP),
                                path.ctypes.data_as(_I32P), ctypes.byref(npath), ctypes.byref(fin))
    return rc, path[:npath.value].tolist(), fin.value
