"""Shared fixtures.  Tests marked `gpu` need an MI355X; the rest run on CPU."""
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (str(ROOT), str(ROOT / "ssla-rt_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (run with -m gpu)")


@pytest.fixture(scope="session")
def stub_dir(tmp_path_factory):
    """Stub weight directory at 80x64, seed 1, tdrop 4 (the CPU-reference config)."""
    from ssla_hip import stub
    d = tmp_path_factory.mktemp("stub_80x64")
    stub.write_stub(str(d), height=64, width=80, seed=1, tdrop=4)
    return str(d)


@pytest.fixture(scope="session")
def stub_npz(stub_dir):
    from oracle import oracle
    return oracle.load_npz(stub_dir)
