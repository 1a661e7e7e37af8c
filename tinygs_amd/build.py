"""Builds libtinygs_amd.so (the C-ABI library) in-tree with hipcc for gfx950.

Numerics flags are part of the contract: no FP contraction (explicit fma only),
IEEE division / sqrt, denormals preserved, no packed-FP32 instruction
selection. Usage: ``python -m tinygs_amd.build [-j N]``.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libtinygs_amd.so")
SOURCES = ["preprocess.hip", "binning.hip", "blend_forward.hip", "blend_backward.hip", "fgs16.hip",
           "preprocess_backward.hip", "loss.hip", "adam.hip", "strategy.hip", "morton.hip", "formats.hip", "selftest.hip", "capi.hip"]
ARCH = os.environ.get("TGS_OFFLOAD_ARCH", "gfx950")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src: str, extra: list[str]) -> str:
    obj = os.path.join(OUT_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    if r.stderr.strip():
        # surface warnings other than the host pass's note about packed-fp32-ops
        lines = [ln for ln in r.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
        if lines:
            sys.stderr.write("\n".join(lines) + "\n")
    return obj


def build(jobs: int = 8, extra: list[str] | None = None, verbose: bool = True) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    extra = extra or []
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(lambda s: _compile(s, extra), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
           "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


ROOT = os.path.dirname(HERE)
CPP_TESTS = ("train_step", "densify_step")   # tests/cpp/<name>.cpp -> tests/cpp/_build/<name>
CPP_TEST_BIN = os.path.join(ROOT, "tests", "cpp", "_build", "train_step")


def cpp_test_bin(name: str) -> str:
    return os.path.join(ROOT, "tests", "cpp", "_build", name)


def build_cpp_test(verbose: bool = True) -> str:
    """Compiles the C++ consumers of include/tinygs_amd/tinygs.hpp (host code
    only) against the built library."""
    for name in CPP_TESTS:
        out = cpp_test_bin(name)
        os.makedirs(os.path.dirname(out), exist_ok=True)
        cmd = [hipcc(), "-std=c++17", "-O2", "-Wall", "-I", os.path.join(ROOT, "include"),
               os.path.join(ROOT, "tests", "cpp", name + ".cpp"),
               "-o", out + ".tmp", "-L", HERE, "-ltinygs_amd", f"-Wl,-rpath,{HERE}",
               "-Wl,-rpath,$ORIGIN/../../../tinygs_amd", "-Wl,-rpath,/opt/rocm/lib"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
        os.replace(out + ".tmp", out)
        if verbose:
            print(f"built {out}")
    return CPP_TEST_BIN


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=8)
    a = ap.parse_args()
    build(a.j)
    build_cpp_test()
