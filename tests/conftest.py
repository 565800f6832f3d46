"""pytest configuration: the `gpu` marker and shared fixtures.

GPU tests (marked gpu) need an MI355X and the in-tree libhearth.so; everything else runs
on the CPU. The tiny model container is generated from its seed once per session.
"""
from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(Path(__file__).resolve().parent))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (MI355X) and the built libhearth.so")


@pytest.fixture(scope="session")
def tiny_model(tmp_path_factory):
    """The tiny Qwen3-MoE-shaped model (4 layers, hidden 512, GQA 8/2, 16 experts top-4,
    F 256, vocab 4096), N(0, 0.02) weights from seed 1, Q4 experts / Q8 dense."""
    from hearth_amd import _native, container
    import golden_io
    path = tmp_path_factory.mktemp("models") / "tiny.hearth"
    container.make_tiny(path, _native.quantize, seed=1)
    want = golden_io.tiny_sha256()
    if want is not None:
        assert container.sha256(path) == want, "tiny model bytes differ from the ones the golden fixtures were made on"
    return path


@pytest.fixture(scope="session")
def variant_models(tmp_path_factory):
    """Builds (once per session) the small models of the other families (DeepSeek-V3
    routing with a GQA attention, Qwen2-MoE, OLMoE; hearth_amd.container.TINY_VARIANTS)
    and returns name -> path."""
    from hearth_amd import _native, container
    d = tmp_path_factory.mktemp("variants")
    cache = {}

    def get(name):
        if name not in cache:
            cache[name] = container.make_tiny(d / f"{name}.hearth", _native.quantize, seed=2,
                                              shape=container.TINY_VARIANTS[name])
        return cache[name]
    return get
