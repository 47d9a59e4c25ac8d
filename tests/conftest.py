"""Shared pytest setup.

* registers the ``gpu`` marker: tests that launch HIP kernels on an MI355X;
* puts the repository root (for ``oracle``) and the package directory (for
  ``trianglemix``) on ``sys.path``.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_ROOT = ROOT / "sparse-attention-op-for-ascend-npu-_amd"
for p in (ROOT, PKG_ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; fails (does not skip) when the HIP path cannot run."""
    import torch

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    from trianglemix import native

    native.load_hip_library()
    native.load_triangle_mix_adapter()
    name = torch.cuda.get_device_properties(0).gcnArchName
    assert name.startswith("gfx950"), f"expected gfx950, got {name}"
    return torch.device("cuda:0")
