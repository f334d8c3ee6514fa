"""Shared test setup: import paths, the `gpu` marker and common helpers."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "s-salaad_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X / gfx950)")


@pytest.fixture(scope="session")
def gpu_device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no ROCm device is visible")
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _device_checks_record_nothing(request):
    """Under the library's checked build (SSALAAD_AMD_LIB pointing at
    libssalaad_amd_checked.so), every GPU test must leave no device
    bounds-check record behind: neither in the devices' status words nor in the
    library's own word for calls that pass none."""
    yield
    if request.node.get_closest_marker("gpu") is None:
        return
    from ssalaad_amd import _lib, _runtime

    lib = _lib.load()
    if not lib.ssl_device_checks():
        return
    import torch

    torch.cuda.synchronize()
    bad = {idx: hex(w.read()) for idx, w in _runtime._STATUS.items() if w.read() >> 8}
    word = lib.ssl_debug_check_word()
    assert not bad and word == 0, f"device bounds checks failed: status {bad}, op word {word:#x}"
