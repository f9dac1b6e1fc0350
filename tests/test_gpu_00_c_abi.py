"""GPU: the C ABI driven from C through the static library.

tests/c_abi/abi_test (built by defer_amd/build.py from abi_test.c, linked
against libdefer_gpu.a and the CPU oracle) creates a model, forwards a prompt,
samples, generates and replays through include/defer_gpu.h, and checks every
result against the oracle; it exits 0 only when all checks hold.

The program is a separate process, and the cooperative launch of the
persistent kernel uses the device's global wave synchronisation, which the
driver grants one process at a time: tests/conftest.py runs this test before
every other one, while the test process itself has not yet launched a
cooperative kernel. (Were the launch refused, the library would run the same
ops as per-phase kernels, with the same bits.)
"""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_c_program_on_the_static_library():
    exe = os.path.join(ROOT, "tests", "c_abi", "abi_test")
    assert os.path.exists(exe), "build it first: python defer_amd/build.py c_abi"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stderr
    assert "ok" in r.stdout
