"""Loads libhearth.so, the MI355X verify engine behind the hearth.h C ABI.

Search order: $HEARTH_LIB (a file or a directory holding libhearth.so), then the
library built in-tree next to this file (python -m hearth_amd.build). There is no CPU
fallback: without the library every engine call raises HearthLibNotFound.
Reference counterpart: python/hearth/_native.py:1-153.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

__all__ = ["HearthLibNotFound", "lib", "lib_path", "quantize", "dequantize", "row_bytes", "matmul"]

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_path: Path | None = None


class HearthLibNotFound(RuntimeError):
    """libhearth.so could not be found or loaded."""


def _candidates() -> list[Path]:
    env = os.environ.get("HEARTH_LIB")
    if env:
        p = Path(env)
        p = p / "libhearth.so" if p.is_dir() else p
        if not p.is_file():
            raise HearthLibNotFound(f"HEARTH_LIB={env!r} does not name libhearth.so")
        return [p]
    return [Path(__file__).resolve().parent / "libhearth.so"]


def _declare(L: ctypes.CDLL) -> None:
    c_int, c_i64, c_vp, c_fp = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.POINTER(ctypes.c_float)
    sigs = {
        "hearth_version": (ctypes.c_char_p, []),
        "hearth_row_bytes": (ctypes.c_size_t, [c_int, c_i64]),
        "hearth_quantize": (c_int, [c_int, c_fp, c_i64, c_i64, c_vp, c_int]),
        "hearth_dequantize": (c_int, [c_int, c_vp, c_i64, c_i64, c_fp]),
        "hearth_matmul": (c_int, [c_int, c_vp, c_i64, c_i64, c_fp, c_int, c_fp, c_int]),
        "hearth_cpu_isa": (c_int, []),
        "hearth_gpu_device": (c_int, [ctypes.c_char_p, ctypes.c_size_t]),
        "hearth_gpu_accept_greedy": (c_int, [c_fp, c_int, c_int, ctypes.POINTER(ctypes.c_int32),
                                             ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32),
                                             ctypes.POINTER(c_int), ctypes.POINTER(ctypes.c_int32)]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name, None)
        if fn is not None:
            fn.restype, fn.argtypes = res, args


def lib() -> ctypes.CDLL:
    global _lib, _path
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        errs = []
        for p in _candidates():
            if not p.is_file():
                errs.append(f"{p}: missing (build it with python -m hearth_amd.build)")
                continue
            try:
                L = ctypes.CDLL(str(p))
            except OSError as e:
                errs.append(f"{p}: {e}")
                continue
            _declare(L)
            _lib, _path = L, p
            return L
        raise HearthLibNotFound("libhearth.so not loadable: " + "; ".join(errs))


def lib_path() -> Path | None:
    try:
        lib()
    except HearthLibNotFound:
        return None
    return _path


def row_bytes(dtype: int, n_cols: int) -> int:
    return int(lib().hearth_row_bytes(int(dtype), int(n_cols)))


def quantize(dtype: int, x, n_threads: int = 0) -> bytes:
    """float32 [rows, cols] -> FORMAT.md §6 bytes via hearth_quantize."""
    import numpy as np
    a = np.ascontiguousarray(x, dtype=np.float32)
    if a.ndim == 1:
        a = a.reshape(1, -1)
    rows, cols = a.shape
    rb = row_bytes(dtype, cols)
    if rb == 0:
        raise ValueError(f"{cols} columns invalid for dtype {dtype}")
    out = np.empty(rows * rb, dtype=np.uint8)
    rc = lib().hearth_quantize(int(dtype), a.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), rows, cols,
                               out.ctypes.data_as(ctypes.c_void_p), int(n_threads))
    if rc != 0:
        raise ValueError(f"hearth_quantize failed ({rc})")
    return out.tobytes()


def dequantize(dtype: int, data: bytes, rows: int, cols: int):
    import numpy as np
    src = np.frombuffer(data, dtype=np.uint8)
    out = np.empty((rows, cols), dtype=np.float32)
    rc = lib().hearth_dequantize(int(dtype), src.ctypes.data_as(ctypes.c_void_p), rows, cols,
                                 out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    if rc != 0:
        raise ValueError(f"hearth_dequantize failed ({rc})")
    return out


def matmul(dtype: int, W: bytes, rows: int, cols: int, X, isa: int = 0):
    """Y [T, rows] = W . X[t] through hearth_matmul (runs on the GPU)."""
    import numpy as np
    x = np.ascontiguousarray(X, dtype=np.float32).reshape(-1, cols)
    T = x.shape[0]
    y = np.empty((T, rows), dtype=np.float32)
    w = np.frombuffer(W, dtype=np.uint8)
    rc = lib().hearth_matmul(int(dtype), w.ctypes.data_as(ctypes.c_void_p), rows, cols,
                             x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), T,
                             y.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), int(isa))
    if rc != 0:
        raise RuntimeError(f"hearth_matmul failed ({rc})")
    return y
