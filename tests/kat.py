"""Known-answer inputs and hashes of the reference's kernel tests
(engine/tests/test_quant.c:55-62 pinned constants, 862-935 det_fill / det_fill_tails /
test_pinned), rewritten in numpy. The inputs come from an integer LCG with exact
conversions, so the hashes hold on every machine and on the GPU."""
from __future__ import annotations

import numpy as np

PIN_Q8 = 0xda285a267ed1fb09
PIN_Q4 = 0x5ed717f72d36fb0c
PIN_Q4_TAILS = 0xb020847e5d2b0807
PIN_Y = {0: 0x78ee7e5c72e238a0, 1: 0xacbfba9fb13b1207, 2: 0xaa0b6460cbd8ad23, 3: 0x532a2d32570c08dc,
         4: 0xa8a0369ab6f0ed22}
R, C, T = 24, 512, 3
_M = (1 << 64) - 1
_A, _B = 6364136223846793005, 1442695040888963407


def fnv1a(data: bytes, h: int = 0xcbf29ce484222325) -> int:
    for x in data:
        h = ((h ^ x) * 0x100000001b3) & _M
    return h


def _lcg_stream(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int64)
    s = seed
    for i in range(n):
        s = (s * _A + _B) & _M
        out[i] = (s >> 40) - (1 << 23)
    return out


def det_fill(n: int, seed: int) -> np.ndarray:
    v = _lcg_stream(seed, 4 * n).reshape(n, 4).astype(np.float64) * 2.0 ** -23
    x = v[:, 0] + v[:, 1] + v[:, 2] + v[:, 3]   # exact in double, summed in the C order
    i = np.arange(n)
    blk = i // 64
    x = x * np.ldexp(1.0, (blk % 7) - 3)
    x = np.where((blk % 13 == 5) & (i % 64 == 17), x * 40.0, x)
    x = np.where(blk % 11 == 3, 0.0, x)
    return x.astype(np.float32)


def det_fill_tails(n: int, seed: int) -> np.ndarray:
    v = _lcg_stream(seed, 6 * n).reshape(n, 6).astype(np.float64) * 2.0 ** -23
    num = ((v[:, 0] + v[:, 1]) + v[:, 2]) + v[:, 3]
    den = v[:, 4] + v[:, 5]
    return (num / (0.125 + np.abs(den))).astype(np.float32)


def pinned_inputs():
    return det_fill(R * C, 1).reshape(R, C), det_fill(T * C, 2).reshape(T, C)
