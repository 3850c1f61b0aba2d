"""pytest configuration: the `gpu` marker and shared fixtures.

`-m "not gpu"` runs the CPU tier (oracle pins, golden vectors, host logic, C-ABI exports);
`-m gpu` runs the parity tests through the C ABI on an MI355X.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from quanta_amd import _lib

    _lib.load()
    return torch.device("cuda", 0)


def pytest_runtest_logstart(nodeid, location):
    # Name the case before a GPU step starts, so a run that dies still says where it was.
    if os.environ.get("QMOE_TRACE_TESTS"):
        print(f"\n[start] {nodeid}", flush=True)
