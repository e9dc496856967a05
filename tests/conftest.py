"""Shared test setup: import paths, the `gpu` marker, device helpers."""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (REPO, os.path.join(REPO, "oracle"), os.path.join(REPO, "tiny-llm_amd"),
          os.path.join(REPO, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def tl():
    """The HIP library (GPU tests only).  torch is imported first so that the
    process has a single HIP runtime."""
    import torch  # noqa: F401  (loads the HIP runtime first)
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    import tinyllm_kv
    tinyllm_kv.load()
    return tinyllm_kv
