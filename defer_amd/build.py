"""Build recipe for the native libraries (run from any directory).

* libdefer_gpu.so   -- the HIP kernels and the C ABI of include/defer_gpu.h,
                       compiled by hipcc for gfx950 only;
* libdefer_gpu.a    -- the same objects as a static archive (what a Rust
                       build.rs links: static=defer_gpu plus the HIP runtime);
* tests/c_abi/abi_test -- a C program linking the archive (and the oracle, as
                       its checker) that the GPU tests run.
* tests/probe/libexact_probe.so -- test-only entry points into the exact
                       sampler's device code (tests/test_exact.py).
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


BUILD = os.path.join(ROOT, "_build")


def build_gpu() -> str:
    """Objects compiled once, linked into the shared library and archived
    into the static one."""
    out = os.path.join(PKG, "libdefer_gpu.so")
    arc = os.path.join(PKG, "libdefer_gpu.a")
    os.makedirs(BUILD, exist_ok=True)
    srcs = [os.path.join(CSRC, "defer_gpu.hip")] + sorted(
        os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.startswith("kernels_") and f.endswith(".hip"))
    flags = [f for f in GPU_FLAGS if f != "-shared"]
    objs = [os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o")) for src in srcs]
    # the translation units compile independently: one hipcc each, at once
    from concurrent.futures import ThreadPoolExecutor

    with ThreadPoolExecutor(max_workers=min(len(srcs), 6)) as ex:
        for f in [ex.submit(_run, [HIPCC, *flags, "-c", "-o", obj, src]) for src, obj in zip(srcs, objs)]:
            f.result()
    tmp = out + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, out)
    if os.path.exists(arc):
        os.remove(arc)
    _run(["ar", "rcs", arc, *objs])
    return out


def build_c_abi_test() -> str:
    """tests/c_abi/abi_test: C, linked against libdefer_gpu.a and the oracle."""
    d = os.path.join(ROOT, "tests", "c_abi")
    out = os.path.join(d, "abi_test")
    os.makedirs(BUILD, exist_ok=True)
    cflags = ["-O2", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-Wall"]
    t_obj = os.path.join(BUILD, "abi_test.o")
    o_obj = os.path.join(BUILD, "oracle.o")
    _run(["gcc", *cflags, "-c", "-o", t_obj, os.path.join(d, "abi_test.c")])
    _run(["gcc", *cflags, "-Wno-unused-parameter", "-c", "-o", o_obj,
          os.path.join(ROOT, "oracle", "oracle.c")])
    _run(["g++", "-o", out, t_obj, o_obj, os.path.join(PKG, "libdefer_gpu.a"),
          "-L/opt/rocm/lib", "-lamdhip64", "-lm", "-Wl,-rpath,/opt/rocm/lib"])
    return out


def build_probe() -> str:
    """tests/probe/libexact_probe.so: test-only entry points into the exact
    sampler's device code (expf_ref, the wave scan, the walker)."""
    d = os.path.join(ROOT, "tests", "probe")
    out = os.path.join(d, "libexact_probe.so")
    tmp = out + ".tmp"
    _run([HIPCC, *GPU_FLAGS, "-o", tmp, os.path.join(d, "exact_probe.hip")])
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
    build_c_abi_test()
    build_probe()


if __name__ == "__main__":
    which = sys.argv[1:] or ["all"]
    for w in which:
        {"gpu": build_gpu, "host": build_host, "c_abi": build_c_abi_test, "probe": build_probe,
         "all": build_all}[w]()
