"""Test configuration: import paths and the ``gpu`` marker.

``-m "not gpu"`` runs everywhere (oracle vs golden vectors, host logic, ABI
exports); ``-m gpu`` needs a ROCm device and the built libtrmoe.so and
compares the HIP kernels with the CPU oracle.
"""

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "complexity-framework_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """The ROCm device; GPU tests fail (not skip) if it or the library is missing."""
    import torch

    if not _gpu_available():
        pytest.fail("GPU test selected but no ROCm device is visible")
    from complexity_amd import _native

    _native.load()  # raises with the load error if libtrmoe.so is missing
    if os.environ.get("TRMOE_SKIP_ARCH_CHECK") != "1":
        assert _native.load().trmoe_device_supported() == 1, "device is not gfx950"
    return torch.device("cuda:0")
