"""Builds the native libraries in-tree.

* ``emberlm_amd/lib/libember_hip.so``  -- the gfx950 kernels + C ABI (include/ember_hip.h),
  compiled with hipcc for gfx950 only.
* ``emberlm_amd/lib/libctd.so``        -- the C++ Tensor/autograd/Module/optim layer
  (include/ctd/...), host-only C++ that calls nothing but the C ABI.
* ``emberlm_amd/lib/ctd_tests``        -- the C++ test binary (tests/cpp/*.cpp).

Usage: ``python -m emberlm_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
INC = os.path.join(ROOT, "include")
KDIR = os.path.join(HERE, "csrc", "kernels")
HDIR = os.path.join(HERE, "csrc", "host")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "lib")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIP_FLAGS = [
    "-O3", "--offload-arch=gfx950", "-std=c++17", "-fPIC", "-I" + INC, "-I" + KDIR,
    # Packed-FP32 VALU forms are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]
CXX_FLAGS = ["-O2", "-std=c++20", "-fPIC", "-I" + INC, "-Wall", "-Wextra"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in l and "is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _jobs():
    return int(os.environ.get("MAX_JOBS", min(8, os.cpu_count() or 4)))


def build_hip(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIB, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(KDIR, "*.hip")))
    hipcc = os.path.join(ROCM, "bin", "hipcc")

    def compile_one(src):
        obj = os.path.join(BUILD, os.path.basename(src) + ".o")
        _run([hipcc, *HIP_FLAGS, "-c", src, "-o", obj])
        return obj

    with cf.ThreadPoolExecutor(_jobs()) as ex:
        objs = list(ex.map(compile_one, srcs))
    out = os.path.join(LIB, "libember_hip.so")
    tmp = out + ".tmp"
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, out)
    if verbose:
        print("built", out)
    return out


def build_host(verbose=False):
    """C++ host layer (no HIP headers): links against libember_hip.so."""
    srcs = sorted(glob.glob(os.path.join(HDIR, "*.cpp")))
    if not srcs:
        return None
    os.makedirs(BUILD, exist_ok=True)
    cxx = shutil.which("g++") or "g++"

    def compile_one(src):
        obj = os.path.join(BUILD, "host_" + os.path.basename(src) + ".o")
        _run([cxx, *CXX_FLAGS, "-c", src, "-o", obj])
        return obj

    with cf.ThreadPoolExecutor(_jobs()) as ex:
        objs = list(ex.map(compile_one, srcs))
    out = os.path.join(LIB, "libctd.so")
    tmp = out + ".tmp"
    _run([cxx, "-shared", "-o", tmp, *objs, "-L" + LIB, "-lember_hip",
          "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, out)
    if verbose:
        print("built", out)
    return out


def build_cpp_tests(verbose=False):
    srcs = sorted(glob.glob(os.path.join(ROOT, "tests", "cpp", "*.cpp")))
    if not srcs or not os.path.exists(os.path.join(LIB, "libctd.so")):
        return None
    cxx = shutil.which("g++") or "g++"
    out = os.path.join(LIB, "ctd_tests")
    oracle_inc = os.path.join(ROOT, "oracle")
    oracle_lib = os.path.join(ROOT, "oracle", "_build")
    _run([cxx, *CXX_FLAGS, "-I" + oracle_inc, "-o", out + ".tmp", *srcs, "-L" + LIB, "-lctd",
          "-lember_hip", "-L" + oracle_lib, "-lember_oracle",
          "-Wl,-rpath,$ORIGIN", "-Wl,-rpath,$ORIGIN/../../oracle/_build", "-lm"])
    os.replace(out + ".tmp", out)
    if verbose:
        print("built", out)
    return out


def build_tools(verbose=False):
    """Command-line tools (emberlm_amd/csrc/tools/*.cpp), one executable each in lib/."""
    srcs = sorted(glob.glob(os.path.join(ROOT, "emberlm_amd", "csrc", "tools", "*.cpp")))
    if not srcs or not os.path.exists(os.path.join(LIB, "libctd.so")):
        return []
    cxx = shutil.which("g++") or "g++"
    outs = []
    for src in srcs:
        out = os.path.join(LIB, os.path.splitext(os.path.basename(src))[0])
        _run([cxx, *CXX_FLAGS, "-o", out + ".tmp", src, "-L" + LIB, "-lctd", "-lember_hip",
              "-Wl,-rpath,$ORIGIN"])
        os.replace(out + ".tmp", out)
        outs.append(out)
        if verbose:
            print("built", out)
    return outs


def build_oracle():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)


def build_all(verbose=False):
    build_oracle()
    build_hip(verbose)
    build_host(verbose)
    build_tools(verbose)
    build_cpp_tests(verbose)


if __name__ == "__main__":
    build_all(verbose=True)
    sys.exit(0)
