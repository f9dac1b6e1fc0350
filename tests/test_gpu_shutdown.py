"""GPU: defer_gpu_shutdown, the library's process teardown.

It refuses while a model or cache is live, then synchronises and resets the
devices the library used (hipDeviceReset, which frees every allocation of the
process there), after which the library works again. The reset would free the
tensors of this test process too, so the calls run in a child process of
their own; the child prints what it saw and exits 0 only when every check
held.
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r"""
import sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from defer_amd import gpu as G, synthetic

cfg = synthetic.CONFIGS["tiny"]
w = synthetic.make_weights(cfg, 1234)
prompt = synthetic.make_prompt(cfg["vocab_size"], 8, seed=3)

def run():
    m = G.GpuModel(G.Config.from_dict(cfg), w)
    c = G.GpuCache(m, 64)
    m.prompt(c, prompt[:-1])
    out = m.forward(int(prompt[-1]), c)
    return m, c, out

m, c, first = run()
try:
    G.shutdown()
    print("shutdown with live handles: not refused", flush=True)
    sys.exit(1)
except G.DeferGpuError as e:
    print("refused while live:", e, flush=True)
c.close()
m.close()
G.shutdown()
print("shutdown ok", flush=True)
m, c, again = run()
assert np.array_equal(first.view(np.uint32), again.view(np.uint32)), "logits differ after the reset"
print("after the reset: logits bit-identical", flush=True)
c.close()
m.close()
G.shutdown()
print("ok", flush=True)
"""


def test_shutdown_refuses_live_handles_then_resets_and_library_works_again():
    print("child: tiny model, shutdown with live handles, after close, reuse", flush=True)
    r = subprocess.run([sys.executable, "-c", CHILD, ROOT], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stderr
    assert "refused while live" in r.stdout and r.stdout.rstrip().endswith("ok")
