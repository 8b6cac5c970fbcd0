"""Builds the gfx950 library llm-inference-diy_amd/lib/libqdiy.so with hipcc.

Usage: python llm-inference-diy_amd/build.py [--verbose]
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB_DIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIB_DIR, "libqdiy.so")
BENCH_LIB = os.path.join(LIB_DIR, "libqdiy_bench.so")
ENGINE_EXE = os.path.join(LIB_DIR, "qdiy_engine")

SOURCES = ["qd_capi.cpp", "qd_engine.cpp", "qd_attention.hip", "qd_rope_cache.hip", "qd_decode_ops.hip", "qd_prefill.hip",
           "qd_flash_prefill.hip"]
ARCH = "gfx950"

# Packed-fp32 VALU forms are disabled for all device code: plain float code is
# compiled to scalar v_fma/v_mul/v_add only.  No floating-point contraction:
# every a*b+c in the sources rounds twice unless written as fmaf, which keeps
# the kernels' arithmetic restatable bit for bit on the host.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-ffp-contract=off"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    raise RuntimeError("hipcc not found")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that is harmless
    noise = "is not a recognized feature for this target"
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if noise not in ln]
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs))


def build(verbose: bool = False) -> str:
    """Builds libqdiy.so (kernels + C ABI), libqdiy_bench.so (bench loops and the
    read-ceiling kernel) and the qdiy_engine executable (stdin/stdout protocol)."""
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB + ".tmp"
    _run([hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
          "-Wall", "-Wno-unused-result", *DEVICE_FLAGS, "-I", INCLUDE, "-I", CSRC,
          "-Wl,-soname,libqdiy.so", "-o", tmp, *[os.path.join(CSRC, s) for s in SOURCES]], verbose)
    os.replace(tmp, LIB)
    tmp = BENCH_LIB + ".tmp"
    _run([hipcc(), f"--offload-arch={ARCH}", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
          *DEVICE_FLAGS, "-I", INCLUDE, "-o", tmp, os.path.join(CSRC, "qd_bench.cpp"),
          os.path.join(CSRC, "qd_bench_read.hip"), "-L", LIB_DIR, "-lqdiy", "-Wl,-rpath,$ORIGIN"],
         verbose)
    os.replace(tmp, BENCH_LIB)
    tmp = ENGINE_EXE + ".tmp"
    _run([hipcc(), "-O2", "-std=c++17", "-Wall", "-I", INCLUDE, "-o", tmp,
          os.path.join(CSRC, "qd_engine_main.cpp"), "-L", LIB_DIR, "-lqdiy", "-Wl,-rpath,$ORIGIN"],
         verbose)
    os.replace(tmp, ENGINE_EXE)
    return LIB


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
