"""Shared test set-up.

Markers: `gpu` tests need a real gfx950 GPU and call the HIP kernels through
the C ABI; everything else runs on the CPU (oracle, host logic, library
loading).  The package directory is put on sys.path so the modules import by
their plain names, as the reference's bin/ modules do.
"""
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "drama3-offloading_amd"
GOLDEN = Path(__file__).resolve().parent / "golden"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the HIP library")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this process")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def lib():
    import hipfetch
    lib = hipfetch.load()
    if lib is None:
        pytest.fail(f"libmoeoffload not loadable: {hipfetch.last_error()}")
    return lib


@pytest.fixture(scope="session")
def dev():
    import torch
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def traces():
    with np.load(GOLDEN / "route_traces.npz") as z:
        return {k: z[k] for k in z.files}


def say(msg: str) -> None:
    """Progress line that names the case, flushed before a GPU step."""
    print(msg, flush=True)
    sys.stdout.flush()
