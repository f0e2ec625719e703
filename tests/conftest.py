"""Shared test set-up: the `gpu` marker, the built library, seeded generators."""

import sys
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through libmi_paged.so)")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def native_lib():
    """libmi_paged.so, built first if it is missing."""
    from mini_infra_qwen3_amd import _native, build

    if not _native.LIBRARY_PATH.exists():
        build.build(verbose=False)
    return _native.load()


@pytest.fixture(scope="session")
def device():
    return torch.device("cuda:0")
