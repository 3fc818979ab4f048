"""Shared pytest setup: markers, import paths, GPU detection, poisoned allocations."""

from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(ROOT, "gemma4-fa4-kernels_amd")
for path in (ROOT, PKG_ROOT):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long CPU test")


def pytest_collection_modifyitems(config, items):
    # GPU tests are skipped (not failed) when no GPU is visible, so that
    # `-m "not gpu"` and plain runs both work in the CPU-only container.
    try:
        import torch

        have_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        have_gpu = False
    if have_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def _poisoned_device_allocations(request, monkeypatch):
    """GPU tests see ``torch.empty`` / ``torch.empty_like`` on the GPU return
    memory already filled: NaN in floating dtypes, all-ones bits in integer
    dtypes (0xFF bytes in the library's uint8 workspaces), True in bool.
    The library's outputs, workspaces and scratch are allocated that way, so
    a kernel that reads an element before writing it, or leaves an output
    element unwritten, fails the comparison instead of passing on whatever
    the caching allocator last held.  G4_TEST_POISON=0 turns it off."""
    if request.node.get_closest_marker("gpu") is None or os.environ.get("G4_TEST_POISON") == "0":
        yield
        return
    import torch

    # `with torch.device(...)` recognises factory functions by identity from a
    # set it builds once: build it from the real functions before wrapping them.
    from torch.utils._device import _device_constructors

    _device_constructors()
    real_empty, real_empty_like = torch.empty, torch.empty_like

    def poison(t):
        if isinstance(t, torch.Tensor) and t.is_cuda and t.numel():
            if t.dtype.is_floating_point:
                t.fill_(float("nan"))
            elif t.dtype == torch.bool:
                t.fill_(True)
            elif not t.dtype.is_complex:
                info = torch.iinfo(t.dtype)
                t.fill_(info.max if info.min == 0 else -1)
        return t

    monkeypatch.setattr(torch, "empty", lambda *a, **k: poison(real_empty(*a, **k)))
    monkeypatch.setattr(torch, "empty_like", lambda *a, **k: poison(real_empty_like(*a, **k)))
    yield
