"""Malformed and truncated containers fail cleanly (the reference's INV-FMT / INV-SAFE,
tests/golden/test_golden_invariants.py:165-180): hearth_open returns NULL with a message
that names the problem, before any device is touched, for every corruption below of
the tiny model's container. The reader is hearth_amd/csrc/modelfile.cpp (FORMAT.md
§2-6 and the canonical-tensor check of engine/src/modelfile.c:621).

These run without a GPU: a well-formed container gets as far as the device step and
fails there ("no HIP device"), so a malformed one must fail earlier, with its own
message."""
from __future__ import annotations

import struct

import pytest

from hearth_amd import _native, container
from hearth_amd.engine import Engine, HearthError

HDR = struct.Struct("<IIQQQQQQII")   # magic, version, meta off/len, tensor dir/count, expert dir/count, align, pad


@pytest.fixture(scope="module")
def tiny_bytes(tmp_path_factory):
    p = tmp_path_factory.mktemp("reader") / "tiny.hearth"
    container.make_tiny(p, _native.quantize, seed=1)
    return p.read_bytes()


def _fields(data):
    return dict(zip(("magic", "version", "meta_off", "meta_len", "tdir", "nt", "edir", "ne", "align", "pad"),
                    HDR.unpack_from(data, 0)))


def _patch(data, off, fmt, value):
    b = bytearray(data)
    struct.pack_into(fmt, b, off, value)
    return bytes(b)


def _tensor_entry(data, name):
    h = _fields(data)
    for i in range(h["nt"]):
        o = h["tdir"] + 128 * i
        if data[o:o + 80].split(b"\0", 1)[0] == name.encode():
            return o
    raise KeyError(name)


def _cases(data):
    h = _fields(data)
    out_norm = _tensor_entry(data, "out_norm")
    emb = _tensor_entry(data, "tok_embd")
    e0 = h["edir"]
    return {
        "empty": (b"", "too small"),
        "magic": (b"XXXX" + data[4:], "not a .hearth container"),
        "version": (_patch(data, 4, "<I", 2), "version"),
        "truncated_half": (data[:len(data) // 2], "outside the file"),
        "truncated_dirs": (data[:100], None),
        "truncated_last_slab": (data[:len(data) - 4096], "outside the file"),
        "flipped_counts": (_patch(data, 32, "<Q", 1 << 40), None),
        "meta_past_end": (_patch(data, 16, "<Q", len(data)), None),
        "tensor_outside": (_patch(data, emb + 104, "<Q", len(data) + 64), "outside the file"),
        "tensor_unaligned": (_patch(data, emb + 104, "<Q", 65), "aligned"),
        "tensor_bad_dtype": (_patch(data, emb + 80, "<I", 99), "dtype"),
        "tensor_nbytes": (_patch(data, emb + 112, "<Q", 1234), "nbytes"),
        "tensor_missing": (data[:out_norm] + b"out_nxrm" + data[out_norm + 8:], "out_norm"),
        "tensor_shape": (_patch(data, out_norm + 88, "<I", 7), None),
        "expert_outside": (_patch(data, e0, "<Q", len(data) + 4096), "outside the file"),
        "expert_short": (_patch(data, e0 + 8, "<Q", 4096), "needed"),
        "expert_dtype": (_patch(data, e0 + 16, "<I", 9), "dtype"),
        "expert_count": (_patch(data, 48, "<Q", h["ne"] - 1), "expert entries"),
    }


CASES = ["empty", "magic", "version", "truncated_half", "truncated_dirs", "truncated_last_slab", "flipped_counts",
         "meta_past_end", "tensor_outside", "tensor_unaligned", "tensor_bad_dtype", "tensor_nbytes", "tensor_missing",
         "tensor_shape", "expert_outside", "expert_short", "expert_dtype", "expert_count"]


@pytest.mark.parametrize("name", CASES)
def test_malformed_container_fails_cleanly(tiny_bytes, tmp_path, name):
    blob, want = _cases(tiny_bytes)[name]
    p = tmp_path / f"{name}.hearth"
    p.write_bytes(blob)
    with pytest.raises(HearthError) as ex:
        Engine(p).close()
    msg = str(ex.value)
    assert "HIP device" not in msg and "no device" not in msg, f"{name}: the reader accepted it ({msg})"
    if want is not None:
        assert want in msg, f"{name}: {msg}"


def test_well_formed_container_passes_the_reader(tiny_bytes, tmp_path):
    """the unmodified container gets past every check (to the device step on a host
    without a GPU, or opens where there is one)"""
    p = tmp_path / "ok.hearth"
    p.write_bytes(tiny_bytes)
    try:
        Engine(p).close()
    except HearthError as ex:
        assert "HIP device" in str(ex) or "device" in str(ex), str(ex)
