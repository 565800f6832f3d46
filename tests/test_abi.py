"""C-ABI checks (CPU only, no device calls).

- libhearth.so exports every function that include/hearth.h and include/hearth_gpu.h
  declare (HEARTH_API);
- the ctypes mirrors in hearth_amd/engine.py have the layout the headers give: sizes and
  field offsets are computed by gcc from the headers themselves;
- where the reference tree is present (this container), include/hearth.h declares the
  same structs (sizes, offsets) and enum values as the reference's
  engine/include/hearth.h:40-112 and the same function names as its lines 119-159.
"""
from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
import tempfile
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
INC = ROOT / "include"
REF_H = Path("/root/reference/engine/include/hearth.h")

from hearth_amd import _native  # noqa: E402
from hearth_amd import engine as E  # noqa: E402

ENUMS = ["HEARTH_F32", "HEARTH_F16", "HEARTH_BF16", "HEARTH_Q8", "HEARTH_Q4", "HEARTH_I32", "HEARTH_U8",
         "HEARTH_POLICY_LRU", "HEARTH_POLICY_LFU", "HEARTH_PREFETCH_OFF", "HEARTH_PREFETCH_NEXT",
         "HEARTH_PREFETCH_SHARED", "HEARTH_ISA_AUTO", "HEARTH_ISA_SCALAR", "HEARTH_ISA_AVX2", "HEARTH_ISA_AVX512"]

MIRRORS = {
    "hearth_options": E.HearthOptions,
    "hearth_model_info": E.HearthModelInfo,
    "hearth_stats": E.HearthStats,
}


def _declared(header: Path) -> list[str]:
    text = header.read_text()
    return re.findall(r"HEARTH_API\s+[^;(]*?\**\s*\b(hearth_\w+)\s*\(", text)


def _layout_program(header: Path, structs: dict) -> str:
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{header}"', "int main(void) {"]
    for cname, mirror in structs.items():
        lines.append(f'    printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, *_ in mirror._fields_:
            lines.append(f'    printf("{cname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
    for en in ENUMS:
        lines.append(f'    printf("{en} %d\\n", (int){en});')
    lines += ["    return 0;", "}"]
    return "\n".join(lines) + "\n"


def _run_layout(header: Path, structs: dict) -> dict:
    if not shutil.which("gcc"):
        pytest.skip("gcc not available")
    with tempfile.TemporaryDirectory() as d:
        src, exe = Path(d) / "layout.c", Path(d) / "layout"
        src.write_text(_layout_program(header, structs))
        subprocess.run(["gcc", "-std=c11", "-I", str(header.parent), str(src), "-o", str(exe)], check=True)
        out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    vals = {}
    for line in out.splitlines():
        key, _, num = line.rpartition(" ")
        vals[key] = int(num)
    return vals


def test_library_exports_every_declared_function():
    lib = ctypes.CDLL(str(_native.lib_path()))
    names = _declared(INC / "hearth.h") + _declared(INC / "hearth_gpu.h")
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_ctypes_mirrors_match_headers():
    structs = dict(MIRRORS)
    structs["hearth_gpu_kstats"] = E.KStats
    structs["hearth_gpu_store_info"] = E.StoreInfo
    structs["hearth_sampler"] = E.HearthSampler
    vals = _run_layout(INC / "hearth_gpu.h", structs)
    for cname, mirror in structs.items():
        assert vals[f"{cname} size"] == ctypes.sizeof(mirror), cname
        for fname, *_ in mirror._fields_:
            assert vals[f"{cname}.{fname}"] == getattr(mirror, fname).offset, f"{cname}.{fname}"


def test_enum_values():
    vals = _run_layout(INC / "hearth.h", {})
    want = dict(HEARTH_F32=0, HEARTH_F16=1, HEARTH_BF16=2, HEARTH_Q8=3, HEARTH_Q4=4, HEARTH_I32=5, HEARTH_U8=6,
                HEARTH_POLICY_LRU=0, HEARTH_POLICY_LFU=1, HEARTH_PREFETCH_OFF=0, HEARTH_PREFETCH_NEXT=1,
                HEARTH_PREFETCH_SHARED=2, HEARTH_ISA_AUTO=0, HEARTH_ISA_SCALAR=1, HEARTH_ISA_AVX2=2,
                HEARTH_ISA_AVX512=3)
    assert {k: vals[k] for k in want} == want
    assert E.POLICIES == {"lru": 0, "lfu": 1}
    assert E.ISAS == {"auto": 0, "scalar": 1, "avx2": 2, "avx512": 3}


@pytest.mark.skipif(not REF_H.is_file(), reason="reference tree not present")
def test_header_matches_reference_header():
    ours = _run_layout(INC / "hearth.h", MIRRORS)
    ref = _run_layout(REF_H, MIRRORS)
    assert ours == ref
    assert set(_declared(REF_H)) <= set(_declared(INC / "hearth.h"))


def test_library_reports_version():
    lib = ctypes.CDLL(str(_native.lib_path()))
    lib.hearth_version.restype = ctypes.c_char_p
    assert lib.hearth_version().decode().startswith("0.1.")
