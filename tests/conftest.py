"""Shared test setup: import paths, the `gpu` marker and device helpers."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("mini-serve-rs_amd", "oracle", ""):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)

# RLSE_KV_LIB (read by rlse_kv) swaps in another build of the library, such
# as a sanitized one (mini-serve-rs_amd/csrc: make sanitize; sanitize_tests.sh
# runs the CPU tests against it).


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def kv():
    import rlse_kv
    rlse_kv.load()
    return rlse_kv


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.load()
    return oracle
