"""The CPU restatement (oracle/) against the reference's own known answers.

- pinned FNV-1a hashes of the reference's quantizers and kernels
  (engine/tests/test_quant.c:55-62, 901-935), for the oracle and for the product
  library's host quantizer;
- whole forward passes: bit-exact with the reference engine built from its sources
  (oracle/_ref) and with the committed golden outputs of that engine;
- the portable exponential against the platform libm and closed forms, and the glibc
  expf restatement (the device exp) against the libm on every float input;
- tree evaluation against the chain evaluation of every root path.
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest

import golden_io
import kat
import oracle_py as O
from hearth_amd import _native, container


@pytest.mark.parametrize("dtype", [3, 4])
def test_oracle_quantizer_pins(dtype):
    W, _ = kat.pinned_inputs()
    assert kat.fnv1a(O.quantize(dtype, W)) == {3: kat.PIN_Q8, 4: kat.PIN_Q4}[dtype]


def test_oracle_q4_heavy_tail_pin():
    x = kat.det_fill_tails(64 * 1024, 3).reshape(64, 1024)
    assert kat.fnv1a(O.quantize(4, x)) == kat.PIN_Q4_TAILS


@pytest.mark.parametrize("dtype", [0, 1, 2, 3, 4])
def test_oracle_matmul_pins(dtype):
    W, X = kat.pinned_inputs()
    Y = O.matmul(dtype, O.quantize(dtype, W), kat.R, kat.C, X)
    assert kat.fnv1a(Y.tobytes()) == kat.PIN_Y[dtype]


@pytest.mark.parametrize("dtype", [3, 4])
def test_library_quantizer_pins(dtype):
    """hearth_quantize of libhearth.so (host code) writes reference-identical bytes."""
    W, _ = kat.pinned_inputs()
    assert kat.fnv1a(_native.quantize(dtype, W)) == {3: kat.PIN_Q8, 4: kat.PIN_Q4}[dtype]
    x = kat.det_fill_tails(64 * 1024, 3).reshape(64, 1024)
    assert kat.fnv1a(_native.quantize(4, x)) == kat.PIN_Q4_TAILS


def test_act_quant_ties_and_degenerate_blocks():
    """NUMERICS §2 closed forms: x*id on exact .5 ties rounds half to even; zero and
    NaN inputs give q = 0; inf saturates the scale."""
    x = np.zeros(256, np.float32)
    x[:64] = np.arange(64) - 31.5          # amax 32 -> id = 127/32, products on k + .5 grid
    x[0] = 127.0
    x[64:128] = 0.0
    x[128:192] = np.nan
    x[192] = np.inf
    out = np.zeros(4 * 72, np.uint8)
    O.lib().ho_act_quant(x.ctypes.data_as(O._FP), 256, out.ctypes.data_as(O.c_void_p))
    blk = out.reshape(4, 72)
    d = blk[:, :4].copy().view(np.float32)[:, 0]
    q = blk[:, 8:].view(np.int8)
    assert d[0] == np.float32(127.0) / np.float32(127.0)
    ref = np.array([np.round(np.float32(v)) for v in x[:64]], dtype=np.int64)   # id = 1: ties to even
    assert np.array_equal(q[0].astype(np.int64), np.clip(ref, -127, 127))
    assert d[1] == 0.0 and not q[1].any()
    assert not q[2].any()
    assert np.isinf(d[3]) and not q[3].any()


def test_portable_exp_matches_libm_and_closed_forms():
    """The portable exp is within one ulp of glibc's expf and equal in > 99.9% of
    cases; exact special values; monotone on a dense grid."""
    L = O.lib()
    xs = np.linspace(-103.0, 88.5, 200001, dtype=np.float32)
    port = np.array([L.ho_exp_port_f(float(v)) for v in xs[::10]], dtype=np.float32)
    libm = np.exp(xs[::10].astype(np.float64)).astype(np.float32)   # correctly rounded reference
    ulp = np.abs(port.view(np.int32).astype(np.int64) - libm.view(np.int32).astype(np.int64))
    assert ulp.max() <= 1 and (ulp == 0).mean() > 0.999
    assert L.ho_exp_port_f(0.0) == 1.0
    assert L.ho_exp_port_f(float("-inf")) == 0.0
    assert math.isinf(L.ho_exp_port_f(89.0)) and math.isnan(L.ho_exp_port_f(float("nan")))
    assert np.all(np.diff(port) >= 0)
    for v in (-745.0, -700.0, -1.0, 1e-10, 0.5, 300.0, 709.0):
        assert L.ho_exp_port_d(v) == pytest.approx(math.exp(v), rel=3e-16, abs=5e-324)


def test_oracle_matches_reference_golden():
    """The restatement (libm exp) reproduces the reference engine's committed outputs bit
    for bit: prompt logits, every argmax, the verify logits and the routing."""
    g = golden_io.tiny_ref()
    if g is None:
        pytest.skip("no golden fixture")
    import tempfile
    from pathlib import Path
    path = container.make_tiny(Path(tempfile.mkdtemp()) / "t.hearth", _native.quantize, seed=1)
    assert container.sha256(path) == str(g["sha256"])
    O.reference_numerics()
    m = O.Model(path)
    lp, rp = m.eval(g["prompt"], routes=True)
    assert np.array_equal(lp[-8:].view(np.uint32), g["prompt_last8"].view(np.uint32))
    assert np.array_equal(lp.argmax(1), g["prompt_argmax"])
    # the reference's greedy continuation: one single-token eval per step
    cont = [int(c) for c in g["continuation"]]
    assert cont[0] == int(lp[-1].argmax())
    for i in range(len(cont) - 1):
        assert int(m.eval([cont[i]])[0].argmax()) == cont[i + 1], i
    m.rewind(128)
    lv, rv = m.eval(g["verify_tokens"], routes=True)
    assert np.array_equal(lv.view(np.uint32), g["verify_logits"].view(np.uint32))
    assert np.array_equal(rp, g["routes"][:128])
    assert np.array_equal(rv, g["routes"][-5:])


@pytest.mark.skipif(not O.REF_LIB.is_file(), reason="reference engine not built (make -C oracle)")
def test_oracle_matches_reference_engine(tiny_model):
    """Bit-exact with the reference engine compiled from source, batch of 64 tokens."""
    from hearth_amd.engine import Engine
    toks = container.uniform_ints(3, 64, container.TINY.vocab)
    ref = Engine(tiny_model, lib=str(O.REF_LIB), threads=4, prefetch="off")
    lr = ref.eval(toks, all_logits=True)
    ref.close()
    O.reference_numerics()
    lo = O.Model(tiny_model).eval(toks)
    assert np.array_equal(lr.view(np.uint32), lo.view(np.uint32))


@pytest.mark.skipif(not O.REF_LIB.is_file(), reason="reference engine not built (make -C oracle)")
@pytest.mark.parametrize("variant", sorted(container.TINY_VARIANTS))
def test_oracle_matches_reference_engine_variants(variant_models, variant):
    """The restatement of the other families' features (q/k/v biases, full-width qk-norm,
    partial and interleaved RoPE, sigmoid scores with selection bias, group-limited
    routing, routed scale, shared experts with and without gate, dense layers, tied
    embeddings, embedding/residual/logit scales) is bit-exact with the reference engine
    compiled from source, with routes."""
    from hearth_amd.engine import Engine
    path = variant_models(variant)
    toks = container.uniform_ints(31, 40, 4096)
    ref = Engine(path, lib=str(O.REF_LIB), threads=4, prefetch="off")
    lr = ref.eval(toks, all_logits=True)
    lr2 = ref.eval(toks[:5], all_logits=True)
    ref.close()
    O.reference_numerics()
    m = O.Model(path)
    lo = m.eval(toks)
    lo2 = m.eval(toks[:5])
    assert np.array_equal(lr.view(np.uint32), lo.view(np.uint32))
    assert np.array_equal(lr2.view(np.uint32), lo2.view(np.uint32))


@pytest.mark.skipif(not O.REF_LIB.is_file(), reason="reference engine not built (make -C oracle)")
@pytest.mark.parametrize("name", ["tiny", "dsv3"])
def test_oracle_route_replay_matches_reference_engine(tiny_model, variant_models, tmp_path, name):
    """Route replay (model.c:1004-1012, 1885-1960): the token at position p takes the
    experts of trace row p % rows for every MoE layer, weights from the router's scores
    (no selection bias, no group limit). The restatement is bit-exact with the reference
    engine replaying the same synthetic trace, rows wrapping, and reports the replayed
    routes."""
    from hearth_amd.engine import Engine
    path = tiny_model if name == "tiny" else variant_models(name)
    O.reference_numerics()
    m = O.Model(path)
    ids = O.synthetic_routes(7, 37, m.n_moe, m.n_experts, m.top_k)
    tr = tmp_path / "routes.hrtr"
    O.write_trace(tr, ids, m.n_layers, m.n_experts)
    vocab = container.TINY.vocab if name == "tiny" else 4096
    toks = container.uniform_ints(41, 64, vocab)
    ref = Engine(path, lib=str(O.REF_LIB), threads=4, prefetch="off")
    ref.route_replay(tr)
    lr = ref.eval(toks, all_logits=True)
    lr2 = ref.eval(toks[:5], all_logits=True)
    ref.close()
    m.set_replay(ids)
    lo, ro = m.eval(toks, routes=True)
    lo2 = m.eval(toks[:5])
    assert np.array_equal(lr.view(np.uint32), lo.view(np.uint32))
    assert np.array_equal(lr2.view(np.uint32), lo2.view(np.uint32))
    assert np.array_equal(ro, ids[np.arange(64) % 37].astype(np.int32))


def test_tree_equals_chain(tiny_model):
    """Every tree node's logits equal the chain evaluation of its root path (bit for bit),
    and committing a path leaves the same KV as evaluating the chain."""
    O.gpu_numerics()
    prompt = container.uniform_ints(5, 40, container.TINY.vocab)
    tok = np.array([17, 5, 9, 300, 4000, 12, 8], dtype=np.int32)
    par = np.array([-1, 0, 0, 1, 1, 2, 4], dtype=np.int32)
    t = O.Model(tiny_model)
    t.eval(prompt)
    lt = t.eval_tree(tok, par)
    for node in range(len(tok)):
        path = []
        v = node
        while v >= 0:
            path.append(v)
            v = par[v]
        path = path[::-1]
        c = O.Model(tiny_model)
        c.eval(prompt)
        lc = c.eval(tok[path])
        assert np.array_equal(lc[-1].view(np.uint32), lt[node].view(np.uint32)), node
    t.commit_path([0, 1, 4, 6])
    after_tree = t.eval([77])
    c = O.Model(tiny_model)
    c.eval(prompt)
    c.eval(tok[[0, 1, 4, 6]])
    assert np.array_equal(c.eval([77]).view(np.uint32), after_tree.view(np.uint32))


def test_greedy_acceptance_closed_form():
    """Greedy chain acceptance = longest prefix with argmax(rows[i]) == d_i, final =
    argmax at the first mismatch (first index wins ties), generate.py:365-392."""
    rng = np.random.default_rng(0)
    for trial in range(200):
        k, V = int(rng.integers(1, 9)), int(rng.integers(2, 50))
        rows = rng.integers(-3, 4, size=(k + 1, V)).astype(np.float32)   # many ties
        am = rows.argmax(1)
        drafts = np.where(rng.random(k) < 0.6, am[:k], rng.integers(0, V, k)).astype(np.int32)
        n_acc = 0
        while n_acc < k and drafts[n_acc] == am[n_acc]:
            n_acc += 1
        rc, path, fin = O.accept_tree(rows, np.concatenate([[0], drafts]), np.arange(-1, k))
        assert rc == 0 and path == list(range(n_acc + 1)) and fin == am[n_acc]


def test_kv_snapshot_round_trip(tiny_model):
    """ho_kv_export -> ho_kv_import into a fresh model continues exactly like the model
    that computed the context (the layout is plumbing; the rows must arrive intact)"""
    O.gpu_numerics()
    toks = container.uniform_ints(31, 24, container.TINY.vocab)
    a = O.Model(tiny_model, cap=64)
    a.eval(toks[:20], logits=False)
    snap = a.kv_export()
    assert snap.shape == (container.TINY.n_layers, 20 * 2 * container.TINY.n_kv_heads * container.TINY.head_dim)
    b = O.Model(tiny_model, cap=64)
    b.kv_import(snap, 20)
    assert b.pos == 20
    la, lb = a.eval(toks[20:]), b.eval(toks[20:])
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    assert np.array_equal(a.kv_export(), b.kv_export())



def test_glibc_expf_restatement_equals_libm_on_every_float():
    """The device exp (ho_exp_glibc_f restates it) is this image's libm expf, which the
    reference engine calls: equal on all 2^32 inputs (NaN results compared as NaN)."""
    bad = O.lib().ho_exp_glibc_mismatches(0, 1 << 32, min(16, os.cpu_count() or 1))
    assert bad == 0, f"{bad} inputs differ from libm expf"


def test_glibc_expf_table_is_2_to_the_i_over_32():
    """The 32 table entries are the correctly rounded doubles of 2^(i/32) (80 significant
    digits, then one rounding), stored minus i << 47 as the algorithm expects; and the
    special values."""
    import struct
    from decimal import Decimal, getcontext
    from fractions import Fraction
    getcontext().prec = 80
    ln2 = Decimal(2).ln()
    want = []
    for i in range(32):
        f = Fraction((Decimal(i) / 32 * ln2).exp())
        b = struct.unpack("<Q", struct.pack("<d", f.numerator / f.denominator))[0]
        want.append((b - (i << 47)) & 0xFFFFFFFFFFFFFFFF)
    src = (O.ROOT / "oracle" / "hx_oracle.c").read_text()
    body = src[src.index("EXP2F_TAB[32] = {"):]
    body = body[:body.index("};")]
    import re
    got = [int(h, 16) for h in re.findall(r"0x([0-9a-f]{16})ull", body)]
    assert got == want
    O.set_exp_mode(O.EXP_GLIBC)
    assert O.lib().ho_expf(0.0) == 1.0 and O.lib().ho_expf(1.0) == np.float32(math.e)
    assert O.lib().ho_expf(89.0) == float("inf") and O.lib().ho_expf(-104.0) == 0.0
    assert O.lib().ho_expf(float("-inf")) == 0.0 and math.isnan(O.lib().ho_expf(float("nan")))
    O.set_exp_mode(O.EXP_LIBM)
