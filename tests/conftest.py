import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libdefer_gpu.so)")


def pytest_collection_modifyitems(session, config, items):
    """The C program (test_gpu_00_c_abi.py) runs in a process of its own and
    makes cooperative launches, which the device grants to one process at a
    time: it goes first, before this process has launched anything."""
    first = [it for it in items if it.path.name == "test_gpu_00_c_abi.py"]
    if first:
        items[:] = first + [it for it in items if it not in first]
