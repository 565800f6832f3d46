"""Access to the committed golden fixtures (tests/golden/*.npz)."""
from __future__ import annotations

from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"


def tiny_ref():
    p = GOLDEN / "tiny_ref.npz"
    return np.load(p, allow_pickle=False) if p.is_file() else None


def tiny_sha256():
    g = tiny_ref()
    return None if g is None else str(g["sha256"])
