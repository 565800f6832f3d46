"""Index ranges of the attention kernels, enumerated on the CPU.

Every ancestor-table index and KV-cache slot that k_attn_chunk and the two value kernels
(k_attn_values, k_attn_values_w) compute is enumerated from the kernels' own index
arithmetic, restated here workgroup by workgroup and lane by lane, for the chain, tree and
prefill geometries the GPU tests run, and must stay in range:

- hearth_amd/csrc/k_attn.hip k_attn_chunk: the launcher (attention_chunked: items per
  token, tokens per block, chunks), the early exit, kshared, and the tree branch that maps
  row r0 + lane >= pos0 through anc[t][r0 + lane - pos0] (score loop) and the tail of the
  value loop (rows jl .. nk - 1);
- k_attn_values / k_attn_values_w: the tree loads (row v clamped to nr - 1, anc_s index
  v - pos0 when v > pos0, the source row pos0 + anc or v itself) of every tile the
  three-deep load pipeline issues, and anc_s's size.

A geometry is what hearth_engine::run_geometry uploads: depth[t] (t for a chain, the
parent's depth + 1 for a tree) and anc[t][0..depth[t]] (the path from node 0 to t). The
GPU never runs here: no test in this file needs one.
"""
from __future__ import annotations

import numpy as np
import pytest

from hearth_amd import container

# k_attn.hip constants
AC_CH, AC_WAVES, AC_IPW, AC_QMAX = 64, 8, 4, 12288
TV_ROWS, TV_SUM, TV_LOAD = 128, 4, 8
MAX_ANC = 4096


def geometry(n, parent=None):
    """depth and anc as run_geometry builds them (parent None: a chain)."""
    depth = np.zeros(n, dtype=np.int64)
    anc = np.full((n, n), -1, dtype=np.int64)
    for i in range(n):
        depth[i] = i if parent is None else (0 if i == 0 else depth[parent[i]] + 1)
        v, j = i, depth[i]
        while v >= 0 and j >= 0:
            anc[i, j] = v
            v = (v - 1) if parent is None else parent[v]
            j -= 1
    return depth, anc


def tree_4x4x4():
    parent, level = [-1], [0]
    for _ in range(3):
        nxt = []
        for p in level:
            for _ in range(4):
                parent.append(p)
                nxt.append(len(parent) - 1)
        level = nxt
    return np.array(parent)


def chunked_ok(hd, grp):
    """attention_chunked_ok (k_attn.hip)"""
    rw = 4 if grp % 4 == 0 else 2 if grp % 2 == 0 else 1
    return hd in (64, 128) and 1 <= grp <= 128 and grp * hd <= AC_QMAX and grp // rw <= AC_WAVES * AC_IPW


def check_chunk(pos0, depth, anc, chain, H, Hkv, hd, cap, kshared_of=None):
    """k_attn_chunk's launch and the indices of every workgroup (k_attn.hip
    attention_chunked and k_attn_chunk). kshared_of replaces the kernel's kshared (for the
    negative control)."""
    T = len(depth)
    grp = H // Hkv
    rw = 4 if grp % 4 == 0 else 2 if grp % 2 == 0 else 1
    ipt = grp // rw
    ntb_max = max(1, min(AC_WAVES * AC_IPW // ipt, AC_QMAX // (grp * hd)))
    nblk = (T + ntb_max - 1) // ntb_max
    ntb = (T + nblk - 1) // nblk
    ncg = (pos0 + T + AC_CH - 1) // AC_CH   # nr_max = pos + T
    nd = hd // 64
    seen = 0
    for c in range(ncg):
        r0 = c * AC_CH
        for tb in range(nblk):
            t0 = tb * ntb
            nt = min(ntb, T - t0)
            if nt <= 0:
                continue
            # every item of the block has a wave: it = wave + k AC_WAVES, k < AC_IPW
            assert nt * ipt <= AC_WAVES * AC_IPW
            # the block's queries fit the staging buffer
            assert (nt - 1) * grp * hd + 64 * (grp * nd - 1) + 63 < AC_QMAX
            dmax = int(depth[t0:t0 + nt].max())
            if pos0 + dmax + 1 <= r0:
                continue
            kshared = min(max((pos0 + T if chain else pos0) - r0, 0), AC_CH)
            if kshared_of is not None:
                kshared = kshared_of(r0)
            for tl in range(nt):
                t = t0 + tl
                nk = min(pos0 + int(depth[t]) + 1 - r0, AC_CH)
                if nk <= 0:
                    continue
                seen += 1
                jl = min(nk, kshared)
                # rows read from the slot of the same index: written rows of the cache
                for j in range(jl):
                    row = r0 + j
                    assert 0 <= row < cap and (row < pos0 or (chain and row < pos0 + T))
                # the tree branch (scores: lanes kshared .. nk - 1; values: rows jl .. nk - 1)
                for j in range(jl, nk):
                    ai = r0 + j - pos0
                    assert 0 <= ai <= depth[t], (pos0, t, r0, j)
                    slot = pos0 + int(anc[t, ai])
                    assert pos0 <= slot < pos0 + T <= cap
    return seen


def check_values(pos0, depth, anc, chain, cap, rows_per_tile, loaders, clamp=True):
    """The loads of k_attn_values (rows_per_tile 128, 8 loader waves) or
    k_attn_values_w (ROWS = 16 NL) for every token: tiles 0 .. ntiles + 2 of the load
    pipeline (three loads ahead; the last steps load nothing, the main loop stops at
    i + 3 <= ntiles, so the highest tile loaded is ntiles + 2)."""
    for t in range(len(depth)):
        dep = int(depth[t])
        nr = pos0 + dep + 1
        assert dep < MAX_ANC   # anc_s[MAX_ANC]
        ntiles = (nr + rows_per_tile - 1) // rows_per_tile
        hi_tile = ntiles + 2 if ntiles >= 3 else 2
        lw = np.arange(loaders)[:, None]
        r = np.arange(16)[None, :]
        for i in range(hi_tile + 1):
            v = i * rows_per_tile + 16 * lw + r
            if chain:
                # rows past the cache read zeros (the buffer's range is cap rows); rows
                # of the token's chain are written rows
                used = v[v < nr]
                assert used.size == 0 or (used.max() < cap and used.min() >= 0)
                continue
            if clamp:
                v = np.minimum(v, nr - 1)
            idx = np.where(v > pos0, v - pos0, 0)
            assert idx.min() >= 0 and idx.max() <= dep
            an = pos0 + anc[t, idx]
            assert (anc[t, idx] >= 0).all()
            srow = np.where(v < pos0, v, an)
            assert srow.min() >= 0 and srow.max() < min(cap, pos0 + len(depth))
            # p rows (LDS-direct, clamped to nr - 1 in the tree branch) stay in the S row
            vp = np.minimum(i * rows_per_tile + np.arange(rows_per_tile), nr - 1)
            assert vp.max() < nr


MODELS = {
    "qwen3": (container.QWEN3_30B_A3B.n_heads, container.QWEN3_30B_A3B.n_kv_heads, container.QWEN3_30B_A3B.head_dim),
    "tiny": (container.TINY.n_heads, container.TINY.n_kv_heads, container.TINY.head_dim),
    "qwen2": (container.TINY_QWEN2.n_heads, container.TINY_QWEN2.n_kv_heads, container.TINY_QWEN2.head_dim),
    "olmoe": (container.TINY_OLMOE.n_heads, container.TINY_OLMOE.n_kv_heads, container.TINY_OLMOE.head_dim),
}

# (name, pos0, parent or None, T, cap): the geometries of the GPU tests
GEOMETRIES = [
    ("chain k=8 at ctx 4095", 4087, None, 9, 4104),
    ("chain k=8 at the cache's end", 4087, None, 9, 4096),
    ("tree 4x4x4 at ctx 2047", 2047, "4x4x4", 85, 2200),
    ("small tree", 49, [-1, 0, 0, 1, 1, 2, 3], 7, 1024),
    ("prefill 160", 0, None, 160, 1024),
    ("prefill 512", 0, None, 512, 4104),
    ("prefill 88 after 512", 512, None, 88, 4104),
    ("chain 9 after 600", 600, None, 9, 4104),
    ("long context chain", 9000, None, 9, 9216),
    ("long context tree", 9000, [-1, 0, 0, 1, 1, 2, 3, 4, 5], 9, 9216),
    ("device loop chain k=16", 300, None, 17, 1024),
    ("single token", 0, None, 1, 64),
]


@pytest.mark.parametrize("model", sorted(MODELS))
@pytest.mark.parametrize("geo", GEOMETRIES, ids=[g[0] for g in GEOMETRIES])
def test_attention_indices_in_range(model, geo):
    name, pos0, parent, T, cap = geo
    H, Hkv, hd = MODELS[model]
    if parent == "4x4x4":
        parent = tree_4x4x4()
    elif parent is not None:
        parent = np.array(parent)
    assert parent is None or len(parent) == T
    depth, anc = geometry(T, None if parent is None else list(parent))
    chain = parent is None or all(parent[i] == i - 1 for i in range(T))
    if chunked_ok(hd, H // Hkv):
        assert check_chunk(pos0, depth, anc, chain, H, Hkv, hd, cap) > 0
    check_values(pos0, depth, anc, chain, cap, TV_ROWS, TV_LOAD)
    check_values(pos0, depth, anc, chain, cap, 64, 4)   # k_attn_values_w<., 4, ., 64>


def test_checks_catch_planted_mistakes():
    """Negative controls, planted in the restatement: (1) the mistake that once faulted a
    probe copy of k_attn_chunk -- every lane sent into the tree branch (kshared 0), so rows
    of the prompt's cache look up anc[t][r0 + lane - pos0] with a negative index; (2) the
    value kernels' tree loads without the clamp of row v to nr - 1, which index anc_s past
    the token's depth in the pipeline's look-ahead tiles."""
    pos0, T = 4087, 9
    depth, anc = geometry(T)
    with pytest.raises(AssertionError):
        check_chunk(pos0, depth, anc, True, 32, 4, 128, 4104, kshared_of=lambda r0: 0)
    parent = [-1, 0, 0, 1, 1, 2, 3]
    depth, anc = geometry(7, parent)
    check_values(49, depth, anc, False, 1024, TV_ROWS, TV_LOAD)
    with pytest.raises(AssertionError):
        check_values(49, depth, anc, False, 1024, TV_ROWS, TV_LOAD, clamp=False)


def test_chunked_ok_bounds_items():
    """Every KV-group size the chunked order accepts fits its items in one block of waves."""
    for hd in (64, 128):
        for grp in range(1, 200):
            if chunked_ok(hd, grp):
                rw = 4 if grp % 4 == 0 else 2 if grp % 2 == 0 else 1
                assert grp // rw <= AC_WAVES * AC_IPW
