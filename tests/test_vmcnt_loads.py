"""The value kernels' load counts in this build's own AMD assembly.

k_attn_values and k_attn_values_w (hearth_amd/csrc/k_attn.hip) keep three V tiles in
flight and publish tile i + 1 after `s_waitcnt vmcnt(WV)` with WV = 2 * (4 + PL): the
wait is right only if every tile issues exactly WV / 2 vector-memory loads (4 16-byte V
loads and PL LDS-direct p loads), so that the WV loads still outstanding are exactly
those of the two tiles after it. A compiler that dropped or merged a load would make the
wait release a tile whose loads are still in flight, with no build error. This test
compiles k_attn.hip to gfx950 assembly with the library's flags and checks, along each
kernel's code, that the first vmcnt(WV) of a pipeline follows 3 WV / 2 loads (the three
tiles of the prologue) and every later one WV / 2 loads (the tile each step issues).
Waits for fewer loads (vmcnt(0), the geometry's own loads) start a new pipeline; waits
for more loads than WV are weaker than the pipeline's and are skipped.
"""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

from hearth_amd import build

SRC = build.CSRC / "k_attn.hip"


def _asm(tmp_path: Path) -> str:
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc is not available")
    out = tmp_path / "k_attn.s"
    flags = [f for f in build.COMMON if f != "-fPIC"]
    r = subprocess.run([hipcc, "-x", "hip", *flags, "--cuda-device-only", "-S", str(SRC), "-o", str(out)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return out.read_text()


def _functions(asm: str):
    for m in re.finditer(r"^(_ZN\S*k_attn_values\S*):", asm, re.M):
        end = asm.find(".Lfunc_end", m.end())
        yield m.group(1), asm[m.end():end]


def _wv(name: str) -> int:
    """WV of the kernel: 2 (4 + PL), PL = 1 for k_attn_values, NS R ROWS / (NL 64) for
    k_attn_values_w<NS, NL, R, ROWS>."""
    if "k_attn_values_w" not in name:
        return 2 * (4 + 1)
    ns, nl, r, rows = (int(x) for x in re.search(r"ILi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)E", name).groups())
    return 2 * (4 + ns * r * rows // (nl * 64))


def _check(body: str, wv: int) -> int:
    """Asserts the load counts; returns how many vmcnt(WV) waits were checked."""
    count, first, checked = 0, True, 0
    for line in body.splitlines():
        t = line.strip()
        if t.startswith("buffer_load") or t.startswith("global_load"):
            count += 1
        elif t.startswith("s_waitcnt") and "vmcnt(" in t:
            n = int(re.search(r"vmcnt\((\d+)\)", t).group(1))
            if n == wv:
                want = 3 * wv // 2 if first else wv // 2
                assert count == want, f"{count} loads before vmcnt({wv}), expected {want}"
                first, count, checked = False, 0, checked + 1
            elif n < wv:
                first, count = True, 0
    return checked


def test_value_kernels_issue_the_loads_their_waits_count(tmp_path):
    asm = _asm(tmp_path)
    names = []
    for name, body in _functions(asm):
        names.append(name)
        # the chain and tree pipelines each: a prologue wait and the loop's three steps
        assert _check(body, _wv(name)) >= 8, name
    assert any("k_attn_values_w" in n for n in names) and any("k_attn_valuesEN" in n for n in names)


def test_check_catches_a_dropped_load():
    """Negative control: one load fewer in a step (the compiler dropping one) fails."""
    good = "\n".join(["buffer_load_dwordx4 v[0:3]"] * 15 + ["s_waitcnt vmcnt(10)"] +
                     ["buffer_load_dwordx4 v[0:3]"] * 5 + ["s_waitcnt vmcnt(10)"])
    assert _check(good, 10) == 2
    bad = "\n".join(["buffer_load_dwordx4 v[0:3]"] * 15 + ["s_waitcnt vmcnt(10)"] +
                    ["buffer_load_dwordx4 v[0:3]"] * 4 + ["s_waitcnt vmcnt(10)"])
    with pytest.raises(AssertionError):
        _check(bad, 10)
