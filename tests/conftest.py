"""Shared test setup: import paths, the `gpu` marker and GPU fixtures."""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PACKAGE = ROOT / "elastic-kv-vmm_amd"
for entry in (str(PACKAGE), str(ROOT)):
    if entry not in sys.path:
        sys.path.insert(0, entry)

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU and the built libelastic_vmm.so (HIP path)")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; fails loudly (no skip) when the HIP path cannot run."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    from elastic_kv import _native

    _native.kernel_library()  # raises if libelastic_vmm.so is missing or stale
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def coracle():
    from oracle.oracle import COracle, build

    build(force=False)
    return COracle()
