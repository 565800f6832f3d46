"""Writes tests/golden/tiny_ref.npz: outputs of the reference engine itself (compiled
from /root/reference sources by oracle/Makefile into oracle/_ref/libhearth_ref.so) on
the tiny Qwen3-MoE-shaped model, for the parity tests. Run in the build container:

    make -C oracle && python tests/golden/make_golden.py

Scenario (config 1): a 128-token uniform-random prompt (seed 7) evaluated in one call;
the greedy continuation (8 tokens, one call each); then a k=4 greedy speculative verify
at position 128 of [last] + drafts, the drafts being the continuation with each
position replaced by a uniform token with probability 0.3 (seed 15), exactly as
generate.py:365-392 does (eval all_logits, accept, rewind). The routing trace of every
call is kept. Stored: the sha256 of the container, the tokens, the prompt's last-8
logit rows and the argmax of all 128 rows, the verify logits [5][4096], the accepted
count and final token, and the routes.
"""
from __future__ import annotations

import sys
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

from hearth_amd import _native, container  # noqa: E402
from hearth_amd.engine import Engine  # noqa: E402

REF = ROOT / "oracle" / "_ref" / "libhearth_ref.so"


def scenario():
    prompt = container.uniform_ints(7, 128, container.TINY.vocab).astype(np.int32)
    corrupt = container.uniforms(15, 8) < 0.3
    rand_tok = container.uniform_ints(12, 8, container.TINY.vocab).astype(np.int32)
    return prompt, corrupt, rand_tok


def read_trace(path, n_moe, K):
    b = Path(path).read_bytes()[24:]
    return np.frombuffer(b, dtype="<u2").reshape(-1, n_moe, K).astype(np.int32)


def main():
    tmp = Path(tempfile.mkdtemp())
    path = container.make_tiny(tmp / "tiny.hearth", _native.quantize, seed=1)
    prompt, corrupt, rand_tok = scenario()
    e = Engine(path, lib=str(REF), threads=4, prefetch="off")
    e.trace_start(tmp / "t.hrtr")
    lp = e.eval(prompt, all_logits=True)
    cont = [int(np.argmax(lp[-1]))]
    for _ in range(7):
        cont.append(int(np.argmax(e.eval([cont[-1]]))))
    e.rewind(128)
    drafts = np.where(corrupt[:4], rand_tok[:4], np.array(cont[1:5], dtype=np.int32)).astype(np.int32)
    verify_in = np.concatenate([[cont[0]], drafts]).astype(np.int32)
    lv = e.eval(verify_in, all_logits=True)
    n_acc, final = 0, None
    for i, d in enumerate(drafts):
        t = int(np.argmax(lv[i]))
        if t != int(d):
            final = t
            break
        n_acc += 1
    if final is None:
        final = int(np.argmax(lv[4]))
    e.trace_stop()
    routes = read_trace(tmp / "t.hrtr", 4, 4)
    info = e.info
    e.close()
    out = Path(__file__).resolve().parent / "tiny_ref.npz"
    np.savez_compressed(out, sha256=np.array(container.sha256(path)), prompt=prompt,
                        prompt_last8=lp[-8:], prompt_argmax=lp.argmax(1).astype(np.int32),
                        continuation=np.array(cont, dtype=np.int32), verify_tokens=verify_in, verify_logits=lv,
                        n_acc=np.int32(n_acc), final=np.int32(final), routes=routes)
    print(f"wrote {out} ({out.stat().st_size} bytes); n_acc={n_acc} final={final} arch={info['arch']}")


if __name__ == "__main__":
    main()
