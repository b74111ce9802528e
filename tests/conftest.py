"""Shared pytest setup: the `gpu` marker, import paths and fixtures.

`-m "not gpu"` tests run on any host (oracle, host logic, C-ABI loading and
error paths); `-m gpu` tests need an MI355X and call the HIP library through
its C ABI."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "hip-kernels_amd"), os.path.dirname(__file__)):
    if p not in sys.path:
        sys.path.insert(0, p)
# GPTOSS_PYBIND_DIR: another build of the `gptoss` module (the sanitizer
# build of tests/sanitize), imported ahead of the in-tree one
if os.environ.get("GPTOSS_PYBIND_DIR"):
    sys.path.insert(0, os.environ["GPTOSS_PYBIND_DIR"])


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; calls the HIP library")


@pytest.fixture(scope="session")
def orc():
    import moe_oracle as _orc  # oracle/moe_oracle.py
    _orc.lib()
    return _orc


@pytest.fixture(scope="session")
def gpu():
    """The HIP library binding; only for tests marked gpu."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a host without a GPU (run with -m 'not gpu')")
    import gptoss_moe
    return gptoss_moe
