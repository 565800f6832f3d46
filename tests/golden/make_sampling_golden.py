"""Writes tests/golden/sampling_ref.npz: outputs of the reference's own sampling code
(python/hearth/generate.py: Sampler.probs, Sampler.draw, accept_point_mass and the
verify block of generate() at lines 365-392) on seeded logits, for the parity tests of
the sampled-acceptance restatement. Run in the build container, where the reference
tree is present:

    python tests/golden/make_sampling_golden.py

The reference functions are imported from the reference tree and called as they are;
their random draws come from a stand-in generator whose random() returns preset
uniforms, so each output is a function of the stored inputs. Stored per case: the
logits (f32), the sampler settings and penalty context, the float64 distribution,
draws for preset uniforms, and point-mass acceptance results; per chain step: the
rows, drafts, uniform stream, accepted count, final token and uniforms consumed.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

REF_PY = Path("/root/reference/python")
OUT = Path(__file__).resolve().parent / "sampling_ref.npz"


class PresetRng:
    """Stands in for np.random.Generator: random() returns the preset values in order."""

    def __init__(self, values):
        self.values = list(values)
        self.used = 0

    def random(self):
        v = self.values[self.used]
        self.used += 1
        return v


def logits_kinds(rng):
    f = np.float32
    yield "normal1", rng.normal(0, 1, 1000).astype(f)
    yield "normal4", rng.normal(0, 4, 4096).astype(f)
    yield "ties", rng.integers(-3, 4, 257).astype(f)
    x = rng.normal(0, 2, 500).astype(f)
    x[rng.random(500) < 0.3] = -np.inf
    yield "neginf", x
    x = np.full(64, -np.inf, dtype=f)
    x[17] = 1.5
    yield "single", x
    yield "tiny_v", rng.normal(0, 1, 7).astype(f)
    x = rng.normal(0, 1, 1000).astype(f)
    x[321] = 20.0
    yield "peaked", x
    yield "equal", np.full(300, 0.25, dtype=f)


SETTINGS = [
    dict(temperature=1.0),
    dict(temperature=0.8, top_p=0.95),
    dict(temperature=0.7, top_k=40),
    dict(temperature=1.3, top_k=10, top_p=0.9, min_p=0.05),
    dict(temperature=0.0),
    dict(temperature=1.0, repetition_penalty=1.3, ctx=True),
    dict(temperature=0.5, min_p=0.1),
    dict(temperature=1e-4),
    dict(temperature=1.0, top_p=0.5),
]


def main():
    sys.path.insert(0, str(REF_PY))
    from hearth.generate import Sampler, accept_point_mass  # the reference's own code

    rng = np.random.default_rng(2026)
    out = {}
    cases = []
    for kind, x in logits_kinds(rng):
        V = x.size
        for si, st in enumerate(SETTINGS):
            if (si + len(cases)) % 3 and kind not in ("ties", "single", "tiny_v"):
                continue   # a spread of settings per kind keeps the fixture small
            ctx = np.array([], dtype=np.int64)
            if st.get("ctx"):
                ctx = np.concatenate([rng.integers(0, V, 12), [-1, V + 5, 3, 3]]).astype(np.int64)
            s = Sampler(temperature=st.get("temperature", 1.0), top_k=st.get("top_k", 0), top_p=st.get("top_p", 1.0),
                        min_p=st.get("min_p", 0.0), repetition_penalty=st.get("repetition_penalty", 1.0))
            p = s.probs(x, list(ctx) if ctx.size else None)
            us = rng.random(4)
            draws = []
            for u in us:
                s.rng = PresetRng([u])
                draws.append(s.draw(p) if s.temperature > 0 else int(np.argmax(p)))
            nz = np.flatnonzero(p)
            ds = [int(np.argmax(p)), int(rng.integers(0, V)), int(nz[-1]), int(np.argmin(p))]
            acc = []
            for d in ds:
                u2 = rng.random(2)
                ok, tok = accept_point_mass(p, d, PresetRng(u2))
                acc.append([d, u2[0], u2[1], int(ok), tok])
            i = len(cases)
            out[f"c{i}_logits"] = x
            out[f"c{i}_ctx"] = ctx.astype(np.int32)
            out[f"c{i}_p"] = p
            out[f"c{i}_draw_u"] = us
            out[f"c{i}_draw"] = np.array(draws, dtype=np.int32)
            out[f"c{i}_acc"] = np.array(acc, dtype=np.float64)
            cases.append([st.get("temperature", 1.0), st.get("top_k", 0), st.get("top_p", 1.0), st.get("min_p", 0.0),
                          st.get("repetition_penalty", 1.0)])
    out["settings"] = np.array(cases, dtype=np.float64)

    # verify steps through generate()'s acceptance block (generate.py:376-392)
    chains = []
    for j in range(8):
        k, V = 4, 300
        rows = rng.normal(0, 3 if j % 2 else 1.5, (k + 1, V)).astype(np.float32)
        am = rows.argmax(1)
        draft = [int(am[i]) if rng.random() < 0.7 else int(rng.integers(0, V)) for i in range(k)]
        seq = [int(t) for t in rng.integers(0, V, 20)]
        st = SETTINGS[1] if j < 4 else dict(temperature=0.9, top_k=50, repetition_penalty=1.2)
        s = Sampler(temperature=st["temperature"], top_k=st.get("top_k", 0), top_p=st.get("top_p", 1.0),
                    repetition_penalty=st.get("repetition_penalty", 1.0))
        stream = rng.random(2 * k + 2)
        s.rng = PresetRng(stream)
        use_ctx = s.uses_context
        full = seq + draft if use_ctx else seq
        n_acc, final = 0, None
        for i, d in enumerate(draft):
            ctx = full[: len(seq) + i] if use_ctx else None
            ok, t = accept_point_mass(s.probs(rows[i], ctx), d, s.rng)
            if not ok:
                final = t
                break
            n_acc += 1
        if final is None:
            ctx = full[: len(seq) + len(draft)] if use_ctx else None
            final = s.sample(rows[len(draft)], ctx)
        out[f"s{j}_rows"] = rows
        out[f"s{j}_draft"] = np.array(draft, dtype=np.int32)
        out[f"s{j}_seq"] = np.array(seq, dtype=np.int32)
        out[f"s{j}_stream"] = stream
        chains.append([st["temperature"], st.get("top_k", 0), st.get("top_p", 1.0), 0.0,
                       st.get("repetition_penalty", 1.0), n_acc, final, s.rng.used])
    out["chains"] = np.array(chains, dtype=np.float64)
    np.savez_compressed(OUT, **out)
    print(f"{len(cases)} distribution cases, {len(chains)} verify steps -> {OUT} ({OUT.stat().st_size} B)")


if __name__ == "__main__":
    main()
