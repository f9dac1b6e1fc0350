"""Build recipe for the native libraries (run from any directory).

* libdefer_gpu.so   -- the HIP kernels and the C ABI of include/defer_gpu.h,
                       compiled by hipcc for gfx950 only.
* libdefer_host.so  -- the C++ host side (session, WAL, checkpoint, ChaCha8,
                       SHA-256, safetensors) of include/defer_host.h.

Device code is built with -ffp-contract=off so that every fused multiply-add
in the kernels is an explicit fmaf() and the arithmetic is identical wherever
a device function is inlined, and with packed-FP32 instructions disabled.
"""
from __future__ import annotations

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "defer_amd")
CSRC = os.path.join(PKG, "csrc")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
GPU_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def _run(cmd, cwd=ROOT):
    print("+", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if out.strip():
        print(out, flush=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}")


def build_gpu() -> str:
    out = os.path.join(PKG, "libdefer_gpu.so")
    tmp = out + ".tmp"
    srcs = [os.path.join(CSRC, "defer_gpu.hip")] + sorted(
        os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.startswith("kernels_") and f.endswith(".hip"))
    _run([HIPCC, *GPU_FLAGS, "-o", tmp, *srcs])
    os.replace(tmp, out)
    return out


def build_host() -> str:
    out = os.path.join(PKG, "libdefer_host.so")
    srcs = sorted(
        os.path.join(CSRC, "host", f) for f in os.listdir(os.path.join(CSRC, "host")) if f.endswith(".cpp")
    )
    tmp = out + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra",
          "-I", os.path.join(ROOT, "include"), "-o", tmp, *srcs,
          "-L", PKG, "-ldefer_gpu", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, out)
    return out


def build_all() -> None:
    build_gpu()
    if os.path.isdir(os.path.join(CSRC, "host")):
        build_host()


if __name__ == "__main__":
    which = sys.argv[1:] or ["all"]
    for w in which:
        {"gpu": build_gpu, "host": build_host, "all": build_all}[w]()
