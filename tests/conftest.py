"""Test configuration: import paths, the `gpu` marker and shared builders."""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PACKAGE_ROOT = ROOT / "neurosim-gpu_amd"
for path in (str(ROOT), str(PACKAGE_ROOT)):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def pytest_collection_modifyitems(config, items):
    # GPU tests run after the CPU ones so a slow first GPU init does not hide CPU failures.
    items.sort(key=lambda item: 1 if item.get_closest_marker("gpu") else 0)


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("a GPU test ran without a visible GPU")
    from neurosim_gpu.native import load_library

    load_library()  # a missing library fails the GPU tests loudly
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def large_case(gpu):
    """The headline graph: random_topology(166000, 25M candidates, seed 0), built once."""
    from cases import make_case

    print("building N=166000 M=25000000 graph", flush=True)
    return make_case(166_000, 25_000_000, 0, gpu)
