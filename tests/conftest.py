from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "moe-offload-lab_amd"
for p in (str(ROOT), str(PKG_DIR)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built libmoehip.so")


def gpu_ready() -> bool:
    try:
        import torch

        if not torch.cuda.is_available():
            return False
        from moelab_hip import _lib

        _lib.check_device(0)
        return True
    except Exception:  # noqa: BLE001
        return False


@pytest.fixture(scope="session")
def dev():
    """The GPU device for gpu-marked tests; the library must load (no skipping on a GPU box)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from moelab_hip import _lib

    _lib.check_device(0)  # raises if libmoehip.so is missing or the GPU is not gfx950
    return torch.device("cuda:0")
