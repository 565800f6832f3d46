"""Writer and reader of the .hearth container (the reference's docs/FORMAT.md v1), and the
synthetic models the verify benchmarks and parity tests run on.

The writer follows FORMAT.md §1-6 (the reference's writers: python/hearth/format.py:417,
engine/tests/test_model.c:267-324): preamble, typed metadata, 128-byte tensor entries,
32-byte expert entries, 64-byte aligned tensors, 4096-byte aligned expert slabs
(gate [F,D], up [F,D], down [D,F] at 64-byte aligned offsets). Aliased slabs
(flag bit 0) let synthetic benchmark containers point many experts at a few physical
slabs; the engine still gives every (layer, expert) its own HBM copy.

Random weights come from splitmix64 and Irwin-Hall sums of 12 uniforms (the recipe of
engine/tests/test_model.c:90-102), computed exactly in float64, so a model built from a
seed is byte-identical on every machine.
"""
from __future__ import annotations

import math
import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

F32, F16, BF16, Q8, Q4, I32, U8 = range(7)
QK = 64
MAGIC = 0x48545248

# FORMAT.md §3.1 key types: 1 u32, 2 f32, 3 u64, 4 str, 5 u32[], 6 f32[], 7 u8[]
_KEY_TYPES = {
    "arch": 4, "n_layers": 1, "d_model": 1, "vocab_size": 1, "max_seq": 1, "norm_eps": 2, "attn_kind": 1,
    "n_heads": 1, "n_kv_heads": 1, "head_dim": 1, "qk_norm": 1, "qkv_bias": 1, "q_lora_rank": 1,
    "kv_lora_rank": 1, "qk_nope_dim": 1, "qk_rope_dim": 1, "v_head_dim": 1, "rope_dim": 1, "rope_style": 1,
    "rope_attn_factor": 2, "attn_scale": 2, "dense_ffn_dim": 1, "n_experts": 1, "top_k": 1, "expert_ffn_dim": 1,
    "shared_ffn_dim": 1, "shared_gate": 1, "score_fn": 1, "score_bias": 1, "n_group": 1, "topk_group": 1,
    "norm_topk_prob": 1, "routed_scale": 2, "emb_scale": 2, "residual_scale": 2, "logit_scale": 2,
    "tie_embeddings": 1, "layer_kind": 7, "bos_id": 1, "eos_ids": 5, "tokenizer": 4, "chat_template": 4,
    "source": 4, "expert_dtype": 1,
}


def row_bytes(dtype: int, n: int) -> int:
    if dtype in (F32, I32):
        return 4 * n
    if dtype in (F16, BF16):
        return 2 * n
    if dtype == U8:
        return n
    if n % QK:
        raise ValueError(f"{n} columns is not a multiple of {QK}")
    return (n // QK) * (66 if dtype == Q8 else 34)


def _al(x: int, a: int) -> int:
    return (x + a - 1) // a * a


def slab_layout(dtype: int, D: int, F: int) -> tuple[int, int, int, int]:
    """(nbytes, off_gate, off_up, off_down) of one expert slab (FORMAT.md §5)."""
    og = 0
    ou = _al(F * row_bytes(dtype, D), 64)
    od = _al(ou + F * row_bytes(dtype, D), 64)
    return _al(od + D * row_bytes(dtype, F), 4096), og, ou, od


def _meta_bytes(meta: dict) -> bytes:
    out = bytearray()
    for k, v in meta.items():
        t = _KEY_TYPES.get(k)
        if t is None:
            raise KeyError(f"unknown metadata key {k!r}")
        kb = k.encode("ascii")
        out += struct.pack("<H", len(kb)) + kb + bytes([t])
        if t == 1:
            out += struct.pack("<I", int(v) & 0xFFFFFFFF)
        elif t == 2:
            out += struct.pack("<f", float(v))
        elif t == 4:
            b = str(v).encode("utf-8")
            out += struct.pack("<I", len(b)) + b
        elif t == 5:
            out += struct.pack("<I", len(v)) + b"".join(struct.pack("<I", int(x)) for x in v)
        elif t == 7:
            out += struct.pack("<I", len(v)) + bytes(int(x) for x in v)
    return bytes(out)


@dataclass
class _T:
    name: str
    dtype: int
    shape: tuple
    data: bytes


@dataclass
class ContainerWriter:
    """Collects tensors and expert slabs, then writes one FORMAT.md v1 file."""
    meta: dict
    tensors: list = field(default_factory=list)
    experts: dict = field(default_factory=dict)        # (layer, e) -> (dtype, slab bytes) or ("alias", (l, e))

    def add(self, name: str, dtype: int, shape, data: bytes) -> None:
        shape = tuple(int(s) for s in shape)
        rows = 1
        for s in shape[:-1]:
            rows *= s
        if len(data) != rows * row_bytes(dtype, shape[-1]):
            raise ValueError(f"{name}: {len(data)} bytes for shape {shape} dtype {dtype}")
        self.tensors.append(_T(name, dtype, shape, bytes(data)))

    def add_expert(self, layer: int, e: int, dtype: int, slab: bytes) -> None:
        self.experts[(layer, e)] = (dtype, slab)

    def alias_expert(self, layer: int, e: int, src: tuple) -> None:
        """(layer, e) shares the physical slab of expert src (flag bit 0)."""
        self.experts[(layer, e)] = ("alias", src)

    def write(self, path) -> Path:
        path = Path(path)
        L = int(self.meta["n_layers"])
        E = int(self.meta.get("n_experts", 0))
        lk = list(self.meta.get("layer_kind", [1 if E else 0] * L))
        ne = L * E if E and any(lk) else 0
        meta = _meta_bytes(self.meta)
        meta_off = 64
        tdir = _al(meta_off + len(meta), 64)
        edir = tdir + 128 * len(self.tensors)
        off = _al(edir + 32 * ne, 64)
        toff = []
        for t in self.tensors:
            toff.append(off)
            off = _al(off + len(t.data), 64)
        off = _al(off, 4096)
        phys = {}   # (layer, e) of a real slab -> offset
        entries = [(0, 0, 0, 0)] * ne
        for (l, e), v in sorted(self.experts.items()):
            if v[0] == "alias":
                continue
            dt, slab = v
            phys[(l, e)] = off
            entries[l * E + e] = (off, len(slab), dt, 0)
            off += len(slab)
        for (l, e), v in sorted(self.experts.items()):
            if v[0] != "alias":
                continue
            o, nb, dt, _ = entries[v[1][0] * E + v[1][1]]
            entries[l * E + e] = (o, nb, dt, 1)
        with open(path, "wb") as f:
            f.write(struct.pack("<IIQQQQQQII", MAGIC, 1, meta_off, len(meta), tdir, len(self.tensors), edir, ne, 4096, 0))
            f.seek(meta_off)
            f.write(meta)
            f.seek(tdir)
            for t, o in zip(self.tensors, toff):
                nm = t.name.encode("ascii")
                if len(nm) > 79:
                    raise ValueError(f"tensor name too long: {t.name}")
                shape = list(t.shape) + [1] * (4 - len(t.shape))
                f.write(nm + b"\0" * (80 - len(nm)) + struct.pack("<II4IQQQ", t.dtype, len(t.shape), *shape, o, len(t.data), 0))
            f.seek(edir)
            for (o, nb, dt, fl) in entries:
                f.write(struct.pack("<QQIIQ", o, nb, dt, fl, 0))
            for t, o in zip(self.tensors, toff):
                f.seek(o)
                f.write(t.data)
            for (l, e), v in sorted(self.experts.items()):
                if v[0] != "alias":
                    f.seek(phys[(l, e)])
                    f.write(v[1])
            f.truncate(off)
        return path


# ---------------------------------------------------------------- seeded weights

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _splitmix(state: int, n: int) -> np.ndarray:
    """n outputs of splitmix64 starting from state (vectorised, wraps mod 2^64)."""
    with np.errstate(over="ignore"):
        z = np.uint64(state) + (np.arange(1, n + 1, dtype=np.uint64) * np.uint64(0x9E3779B97F4A7C15))
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def normal(seed: int, n: int, std: float) -> np.ndarray:
    """n float32 draws of N(0, std^2) by Irwin-Hall (12 uniforms k/2^24), exact in
    float64 up to the final scaling, so identical on every machine."""
    s = np.zeros(n, dtype=np.float64)
    base = (int(seed) * 0x632BE59BD9B4E019) & 0xFFFFFFFFFFFFFFFF
    for k in range(12):
        u = (_splitmix((base + k * 0x7F4A7C159E3779B9) & 0xFFFFFFFFFFFFFFFF, n) >> np.uint64(40)).astype(np.float64)
        s += u * (1.0 / 16777216.0)
    return ((s - 6.0) * std).astype(np.float32)


def uniform_ints(seed: int, n: int, hi: int) -> np.ndarray:
    """n integers in [0, hi) from splitmix64 (multiply-shift, bias < 2^-32)."""
    z = _splitmix((int(seed) * 0xD1B54A32D192ED03) & 0xFFFFFFFFFFFFFFFF, n) >> np.uint64(32)
    return ((z * np.uint64(hi)) >> np.uint64(32)).astype(np.int64)


def uniforms(seed: int, n: int) -> np.ndarray:
    """n float64 uniforms in [0, 1) with 53 random bits."""
    z = _splitmix((int(seed) * 0x9FB21C651E98DF25) & 0xFFFFFFFFFFFFFFFF, n) >> np.uint64(11)
    return z.astype(np.float64) * (1.0 / 9007199254740992.0)


# ---------------------------------------------------------------- synthetic models

@dataclass
class Shape:
    """Hyper-parameters of a synthetic MoE model. The defaults are Qwen3-MoE (GQA,
    per-head qk-norm, NEOX RoPE, softmax top-k with norm_topk_prob); the other fields
    select the FORMAT.md variants of the other supported families (q/k/v biases and a
    gated shared expert as Qwen2-MoE, full-width qk-norm as OLMoE, sigmoid scores with a
    selection bias, group-limited routing, routed scale, leading dense layers and a
    shared expert as DeepSeek-V3, partial and interleaved RoPE, tied embeddings,
    embedding/residual/logit scales)."""
    n_layers: int
    d_model: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    n_experts: int
    top_k: int
    expert_ffn: int
    vocab: int
    max_seq: int = 4096
    rope_theta: float = 1e6
    arch: str = "qwen3_moe"
    qk_norm: int = 1
    qkv_bias: int = 0
    rope_dim: int = 0            # 0: head_dim
    rope_style: int = 0
    shared_ffn: int = 0
    shared_gate: int = 0
    score_fn: int = 0
    score_bias: int = 0
    n_group: int = 1
    topk_group: int = 1
    norm_topk: int = 1
    routed_scale: float = 1.0
    n_dense: int = 0             # leading dense (layer_kind 0) layers
    dense_ffn: int = 0
    tie: int = 0
    emb_scale: float = 1.0
    resid_scale: float = 1.0
    logit_scale: float = 1.0
    # multi-head latent attention (attn_kind 1): q_lora 0 = uncompressed q
    attn_kind: int = 0
    q_lora: int = 0
    kv_lora: int = 0
    nope: int = 0
    rope_qk: int = 0
    v_head: int = 0


TINY = Shape(n_layers=4, d_model=512, n_heads=8, n_kv_heads=2, head_dim=64, n_experts=16, top_k=4,
             expert_ffn=256, vocab=4096, max_seq=1024)
# Small models of the other families, for parity tests of the FORMAT.md variants.
TINY_DSV3_GQA = Shape(n_layers=4, d_model=512, n_heads=8, n_kv_heads=2, head_dim=64, n_experts=16, top_k=4,
                      expert_ffn=256, vocab=4096, max_seq=1024, arch="deepseek_v3", qk_norm=0, rope_style=1,
                      shared_ffn=256, score_fn=1, score_bias=1, n_group=4, topk_group=2, norm_topk=1,
                      routed_scale=2.5, n_dense=1, dense_ffn=512)
TINY_QWEN2 = Shape(n_layers=3, d_model=512, n_heads=8, n_kv_heads=4, head_dim=64, n_experts=16, top_k=4,
                   expert_ffn=192, vocab=4096, max_seq=1024, arch="qwen2_moe", qk_norm=0, qkv_bias=1,
                   shared_ffn=384, shared_gate=1, norm_topk=0)
TINY_OLMOE = Shape(n_layers=3, d_model=512, n_heads=8, n_kv_heads=8, head_dim=64, n_experts=16, top_k=4,
                   expert_ffn=256, vocab=4096, max_seq=1024, arch="olmoe", qk_norm=2, norm_topk=0, rope_dim=32,
                   tie=1, emb_scale=1.5, resid_scale=0.75, logit_scale=0.5)
TINY_DSV3 = Shape(n_layers=4, d_model=512, n_heads=4, n_kv_heads=4, head_dim=128, n_experts=16, top_k=4,
                  expert_ffn=256, vocab=4096, max_seq=1024, arch="deepseek_v3", qk_norm=0, rope_style=1,
                  shared_ffn=256, score_fn=1, score_bias=1, n_group=4, topk_group=2, norm_topk=1,
                  routed_scale=2.5, n_dense=1, dense_ffn=512, attn_kind=1, q_lora=192, kv_lora=128, nope=64,
                  rope_qk=64, v_head=64)
TINY_MLA_NOQ = Shape(n_layers=2, d_model=512, n_heads=8, n_kv_heads=8, head_dim=96, n_experts=16, top_k=4,
                     expert_ffn=256, vocab=4096, max_seq=1024, arch="deepseek_v2_lite", qk_norm=0,
                     attn_kind=1, q_lora=0, kv_lora=256, nope=64, rope_qk=32, v_head=128)
TINY_VARIANTS = {"dsv3_gqa": TINY_DSV3_GQA, "qwen2": TINY_QWEN2, "olmoe": TINY_OLMOE, "dsv3": TINY_DSV3,
                 "mla_noq": TINY_MLA_NOQ}

QWEN3_30B_A3B = Shape(n_layers=48, d_model=2048, n_heads=32, n_kv_heads=4, head_dim=128, n_experts=128, top_k=8,
                      expert_ffn=768, vocab=151936, max_seq=8192)
# DeepSeek-V3 widths (multi-head latent attention, 256 routed experts top-8 + a shared
# expert, sigmoid scores with a selection bias, 8 groups top-4, routed scale 2.5),
# depth cut to 3 dense + 20 MoE layers.
DEEPSEEK_V3 = Shape(n_layers=23, d_model=7168, n_heads=128, n_kv_heads=128, head_dim=192, n_experts=256, top_k=8,
                    expert_ffn=2048, vocab=129280, max_seq=8192, arch="deepseek_v3", qk_norm=0, rope_style=1,
                    shared_ffn=2048, score_fn=1, score_bias=1, n_group=8, topk_group=4, norm_topk=1,
                    routed_scale=2.5, n_dense=3, dense_ffn=18432, attn_kind=1, q_lora=1536, kv_lora=512, nope=128,
                    rope_qk=64, v_head=128)


def _rope_dim(s: Shape) -> int:
    return s.rope_dim or (s.rope_qk if s.attn_kind == 1 else s.head_dim)


def _meta(s: Shape, source: str) -> dict:
    m = dict(arch=s.arch, n_layers=s.n_layers, d_model=s.d_model, vocab_size=s.vocab, max_seq=s.max_seq,
             norm_eps=1e-6, n_heads=s.n_heads, n_kv_heads=s.n_kv_heads, head_dim=s.head_dim, qk_norm=s.qk_norm,
             rope_dim=_rope_dim(s), attn_scale=float(np.float32(1.0 / math.sqrt(s.head_dim))),
             n_experts=s.n_experts, top_k=s.top_k, expert_ffn_dim=s.expert_ffn, norm_topk_prob=s.norm_topk,
             layer_kind=[0] * s.n_dense + [1] * (s.n_layers - s.n_dense), bos_id=1, eos_ids=[2], source=source)
    # keys written only where they differ from the FORMAT.md default
    extra = dict(qkv_bias=(s.qkv_bias, 0), rope_style=(s.rope_style, 0), shared_ffn_dim=(s.shared_ffn, 0),
                 shared_gate=(s.shared_gate, 0), score_fn=(s.score_fn, 0), score_bias=(s.score_bias, 0),
                 n_group=(s.n_group, 1), topk_group=(s.topk_group, 1), dense_ffn_dim=(s.dense_ffn, 0),
                 tie_embeddings=(s.tie, 0), routed_scale=(float(s.routed_scale), 1.0),
                 emb_scale=(float(s.emb_scale), 1.0), residual_scale=(float(s.resid_scale), 1.0),
                 logit_scale=(float(s.logit_scale), 1.0))
    for k, (v, default) in extra.items():
        if v != default:
            m[k] = v
    if s.attn_kind == 1:
        m.update(attn_kind=1, q_lora_rank=s.q_lora, kv_lora_rank=s.kv_lora, qk_nope_dim=s.nope, qk_rope_dim=s.rope_qk,
                 v_head_dim=s.v_head, attn_scale=float(np.float32(1.0 / math.sqrt(s.nope + s.rope_qk))))
    return m


def rope_inv_freq(s: Shape) -> np.ndarray:
    """1 / theta^(2j / rope_dim) in float32, computed with the platform libm's pow."""
    d = _rope_dim(s)
    return np.array([1.0 / math.pow(s.rope_theta, (2 * j) / d) for j in range(d // 2)], dtype=np.float32)


def make_tiny(path, quantize, seed: int = 1, shape: Shape = TINY, std: float = 0.02) -> Path:
    """A small model with N(0, std^2) weights from `seed`: Q4 experts, Q8 attention,
    embedding and lm_head, F32 router and norms (norms = 1.0), the quantization done by
    the authoritative quantizer `quantize(dtype, float32 [rows, cols]) -> bytes`."""
    s = shape
    D, H, Hkv, hd, E, F, V, L = s.d_model, s.n_heads, s.n_kv_heads, s.head_dim, s.n_experts, s.expert_ffn, s.vocab, s.n_layers
    w = ContainerWriter(_meta(s, f"synthetic:tiny:seed{seed}"))
    k = [seed * 1000003]

    def rnd(rows, cols):
        k[0] += 1
        return normal(k[0], rows * cols, std).reshape(rows, cols)

    def q(name, dtype, rows, cols):
        w.add(name, dtype, (rows, cols), quantize(dtype, rnd(rows, cols)))

    def vec(name, n, base=0.0, sd=0.02):
        k[0] += 1
        w.add(name, F32, (n,), (base + normal(k[0], n, sd)).astype(np.float32).tobytes())

    ones = np.ones(D, dtype=np.float32).tobytes()
    q("tok_embd", Q8, V, D)
    if not s.tie:
        q("lm_head", Q8, V, D)
    w.add("out_norm", F32, (D,), ones)
    w.add("rope_inv_freq", F32, (_rope_dim(s) // 2,), rope_inv_freq(s).tobytes())
    for l in range(L):
        p = f"blk.{l}."
        w.add(p + "attn_norm", F32, (D,), ones)
        w.add(p + "ffn_norm", F32, (D,), ones)
        if s.attn_kind == 1:
            qh = s.nope + s.rope_qk
            if s.q_lora:
                q(p + "attn_q_a", Q8, s.q_lora, D)
                vec(p + "attn_q_a_norm", s.q_lora, 1.0, 0.1)
                q(p + "attn_q_b", Q8, H * qh, s.q_lora)
            else:
                q(p + "attn_q", Q8, H * qh, D)
            q(p + "attn_kv_a", Q8, s.kv_lora + s.rope_qk, D)
            vec(p + "attn_kv_a_norm", s.kv_lora, 1.0, 0.1)
            q(p + "attn_kv_b", Q8, H * (s.nope + s.v_head), s.kv_lora)
            q(p + "attn_o", Q8, D, H * s.v_head)
        else:
            q(p + "attn_q", Q8, H * hd, D)
            q(p + "attn_k", Q8, Hkv * hd, D)
            q(p + "attn_v", Q8, Hkv * hd, D)
            q(p + "attn_o", Q8, D, H * hd)
        if s.qkv_bias:
            vec(p + "attn_q_bias", H * hd)
            vec(p + "attn_k_bias", Hkv * hd)
            vec(p + "attn_v_bias", Hkv * hd)
        if s.qk_norm == 1:
            w.add(p + "attn_q_norm", F32, (hd,), np.ones(hd, np.float32).tobytes())
            w.add(p + "attn_k_norm", F32, (hd,), np.ones(hd, np.float32).tobytes())
        elif s.qk_norm == 2:
            vec(p + "attn_q_norm", H * hd, 1.0, 0.1)
            vec(p + "attn_k_norm", Hkv * hd, 1.0, 0.1)
        if l < s.n_dense:
            q(p + "ffn_gate", Q8, s.dense_ffn, D)
            q(p + "ffn_up", Q8, s.dense_ffn, D)
            q(p + "ffn_down", Q8, D, s.dense_ffn)
            continue
        w.add(p + "moe_router", F32, (E, D), rnd(E, D).tobytes())
        if s.score_bias:
            vec(p + "moe_router_bias", E, 0.0, 0.05)
        if s.shared_ffn:
            q(p + "shexp_gate", Q8, s.shared_ffn, D)
            q(p + "shexp_up", Q8, s.shared_ffn, D)
            q(p + "shexp_down", Q8, D, s.shared_ffn)
            if s.shared_gate:
                w.add(p + "shexp_gate_inp", F32, (1, D), (rnd(1, D) * 10.0).astype(np.float32).tobytes())
        nb, og, ou, od = slab_layout(Q4, D, F)
        for e in range(E):
            slab = bytearray(nb)
            for off, (rows, cols) in ((og, (F, D)), (ou, (F, D)), (od, (D, F))):
                b = quantize(Q4, rnd(rows, cols))
                slab[off:off + len(b)] = b
            w.add_expert(l, e, Q4, bytes(slab))
    return w.write(path)


def _random_blocks(rng: np.random.Generator, dtype: int, rows: int, cols: int) -> bytes:
    """rows x cols of valid random Q8/Q4 blocks, std ~ 1/sqrt(cols) (the reference's
    synthetic recipe, python/hearth/synth.py:287-305)."""
    nb = cols // QK
    sd = 1.0 / math.sqrt(cols)
    if dtype == Q8:
        blk = np.zeros((rows, nb), dtype=[("d", "<f2"), ("q", "i1", (QK,))])
        blk["d"] = np.float16(3.0 * sd / 127.0)
        blk["q"] = np.clip(np.rint(rng.standard_normal((rows, nb, QK), dtype=np.float32) * 42.0), -127, 127).astype(np.int8)
    else:
        blk = np.zeros((rows, nb), dtype=[("d", "<f2"), ("qs", "u1", (32,))])
        blk["d"] = np.float16(3.0 * sd / 7.0)
        qv = (np.clip(np.rint(rng.standard_normal((rows, nb, QK), dtype=np.float32) * 2.5), -8, 7) + 8).astype(np.uint8)
        blk["qs"] = qv[..., :32] | (qv[..., 32:] << 4)
    return blk.tobytes()


class _RowPool:
    """Dense rows drawn from a pool of random encoded rows (the reference's synthetic
    recipe, python/hearth/synth.py:328-338): row r of a matrix with salt s is pool row
    (r * 31 + s) mod n. Throughput runs only need valid blocks of the right shape."""

    def __init__(self, rng: np.random.Generator, n: int = 1021):
        self.rng, self.n, self.p = rng, n, {}

    def rows(self, dtype: int, rows: int, cols: int, salt: int) -> bytes:
        key = (dtype, cols)
        if key not in self.p:
            self.p[key] = np.frombuffer(_random_blocks(self.rng, dtype, self.n, cols), dtype=np.uint8).reshape(self.n, -1)
        idx = (np.arange(rows, dtype=np.int64) * 31 + salt) % self.n
        return self.p[key][idx].tobytes()


def make_shaped(path, shape: Shape = QWEN3_30B_A3B, seed: int = 0, n_unique_slabs: int = 32,
                n_layers: int | None = None) -> Path:
    """A real-shaped model with random weights for throughput runs: Q4 experts, Q8
    attention / dense FFN / shared expert / embedding / lm_head, F32 routers (N(0,
    2.5^2/D), distinct per layer), unit norms (norms before a low-rank projection drawn
    near 1). GQA with per-head qk-norm, or multi-head latent attention (attn_kind 1);
    leading dense layers, a shared expert and the routing settings follow the shape.
    Expert slabs cycle over n_unique_slabs physical slabs (aliased entries); the engine
    still gives every (layer, expert) its own copy."""
    s = shape if n_layers is None else Shape(**{**shape.__dict__, "n_layers": n_layers})
    rng = np.random.default_rng(seed)
    D, H, Hkv, hd, E, F, V, L = s.d_model, s.n_heads, s.n_kv_heads, s.head_dim, s.n_experts, s.expert_ffn, s.vocab, s.n_layers
    w = ContainerWriter(_meta(s, f"synthetic:{s.arch}:seed{seed}"))
    ones = np.ones(D, dtype=np.float32).tobytes()
    pool = _RowPool(rng)

    def q8(name, rows, cols, salt):
        w.add(name, Q8, (rows, cols), pool.rows(Q8, rows, cols, salt))

    def near_one(name, n):
        w.add(name, F32, (n,), (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32).tobytes())

    q8("tok_embd", V, D, 1)
    q8("lm_head", V, D, 2)
    w.add("out_norm", F32, (D,), ones)
    w.add("rope_inv_freq", F32, (_rope_dim(s) // 2,), rope_inv_freq(s).tobytes())
    n_moe = sum(1 for l in range(L) if l >= s.n_dense)
    nb, og, ou, od = slab_layout(Q4, D, F)
    slabs = []
    for i in range(min(n_unique_slabs, max(1, n_moe * E))):
        slab = bytearray(nb)
        for j, (off, (rows, cols)) in enumerate(((og, (F, D)), (ou, (F, D)), (od, (D, F)))):
            b = pool.rows(Q4, rows, cols, 7919 + 3 * i + j)
            slab[off:off + len(b)] = b
        slabs.append(bytes(slab))
    first, n_seen = {}, 0      # unique slab -> (layer, expert) holding it; MoE entries so far
    for l in range(L):
        p = f"blk.{l}."
        w.add(p + "attn_norm", F32, (D,), ones)
        w.add(p + "ffn_norm", F32, (D,), ones)
        if s.attn_kind == 1:
            qh = s.nope + s.rope_qk
            if s.q_lora:
                q8(p + "attn_q_a", s.q_lora, D, 10 * l + 3)
                near_one(p + "attn_q_a_norm", s.q_lora)
                q8(p + "attn_q_b", H * qh, s.q_lora, 10 * l + 4)
            else:
                q8(p + "attn_q", H * qh, D, 10 * l + 3)
            q8(p + "attn_kv_a", s.kv_lora + s.rope_qk, D, 10 * l + 5)
            near_one(p + "attn_kv_a_norm", s.kv_lora)
            q8(p + "attn_kv_b", H * (s.nope + s.v_head), s.kv_lora, 10 * l + 6)
            q8(p + "attn_o", D, H * s.v_head, 10 * l + 7)
        else:
            q8(p + "attn_q", H * hd, D, 10 * l + 3)
            q8(p + "attn_k", Hkv * hd, D, 10 * l + 4)
            q8(p + "attn_v", Hkv * hd, D, 10 * l + 5)
            q8(p + "attn_o", D, H * hd, 10 * l + 6)
            if s.qk_norm == 1:
                w.add(p + "attn_q_norm", F32, (hd,), np.ones(hd, np.float32).tobytes())
                w.add(p + "attn_k_norm", F32, (hd,), np.ones(hd, np.float32).tobytes())
        if l < s.n_dense:
            q8(p + "ffn_gate", s.dense_ffn, D, 10 * l + 8)
            q8(p + "ffn_up", s.dense_ffn, D, 10 * l + 9)
            q8(p + "ffn_down", D, s.dense_ffn, 10 * l + 10)
            continue
        router = (rng.standard_normal((E, D), dtype=np.float32) * np.float32(2.5 / math.sqrt(D))).astype(np.float32)
        w.add(p + "moe_router", F32, (E, D), router.tobytes())
        if s.score_bias:
            w.add(p + "moe_router_bias", F32, (E,), (0.05 * rng.standard_normal(E)).astype(np.float32).tobytes())
        if s.shared_ffn:
            q8(p + "shexp_gate", s.shared_ffn, D, 10 * l + 8)
            q8(p + "shexp_up", s.shared_ffn, D, 10 * l + 9)
            q8(p + "shexp_down", D, s.shared_ffn, 10 * l + 10)
        for e in range(E):
            i = n_seen % len(slabs)
            if n_seen < len(slabs):
                w.add_expert(l, e, Q4, slabs[i])
                first[i] = (l, e)
            else:
                w.alias_expert(l, e, first[i])
            n_seen += 1
    return w.write(path)


def zipf_routes(seed: int, rows: int, n_moe: int, n_experts: int, k: int, s: float = 1.1) -> np.ndarray:
    """Routing-trace rows [rows][n_moe][k] (uint16) with Zipf expert popularity: in each
    MoE layer the experts are ranked by a seeded random permutation and a token takes k
    distinct experts, drawn without replacement with p(rank r) proportional to
    (r + 1)^-s (the reference simulator's skewed routing, docs/SIMULATOR.md:172-182).
    Sampling without replacement is done as the top k of log p + Gumbel noise, which
    has the same distribution as k successive renormalised draws."""
    rng = np.random.default_rng(seed)
    logp = -s * np.log(np.arange(1, n_experts + 1, dtype=np.float64))
    perm = np.stack([rng.permutation(n_experts) for _ in range(n_moe)])      # rank -> expert
    keys = logp[None, None, :] + rng.gumbel(size=(rows, n_moe, n_experts))
    top = np.argsort(-keys, axis=-1, kind="stable")[..., :k]                   # ranks
    return np.take_along_axis(np.broadcast_to(perm[None], (rows, n_moe, n_experts)), top, -1).astype(np.uint16)


def write_route_trace(path, ids, n_layers: int, n_experts: int) -> Path:
    """A routing-trace file (FORMAT.md §9) of ids [rows][n_moe][k]: 'HRTR', version 1,
    n_layers, E, K, n_moe as little-endian uint32, then the rows as uint16 expert ids
    (what hearth_trace_start writes and hearth_route_replay reads)."""
    a = np.ascontiguousarray(ids, dtype="<u2")
    rows, n_moe, k = a.shape
    hdr = np.array([0x52545248, 1, n_layers, n_experts, k, n_moe], dtype="<u4")
    path = Path(path)
    with open(path, "wb") as f:
        f.write(hdr.tobytes())
        f.write(a.tobytes())
    return path


def sha256(path, chunk: int = 1 << 24) -> str:
    """sha256 hex digest of a file (fingerprint of a generated container)."""
    import hashlib
    h = hashlib.sha256()
    with open(path, "rb") as f:
        while True:
            b = f.read(chunk)
            if not b:
                break
            h.update(b)
    return h.hexdigest()
