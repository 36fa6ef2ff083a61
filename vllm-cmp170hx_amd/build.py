"""Builds libvllm_mi355x.so (the C-ABI library of hand-written gfx950 HIP
kernels) in-tree, next to the Python package that loads it.

    python vllm-cmp170hx_amd/build.py [--jobs N]

Every source is compiled for gfx950 only, with packed-FP32 instructions
disabled, then linked into one shared library with no dependency on torch.
"""

from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
PACKAGE = os.path.join(HERE, "vllm_mi355x")
LIBRARY = os.path.join(PACKAGE, "libvllm_mi355x.so")
OBJDIR = os.path.join(HERE, "_build")

SOURCES = ["common.cpp", "exl3_linear.hip", "exl3_gemm.hip", "exl3_moe.hip", "marlin_moe.hip"]

ARCH = "gfx950"
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    # no packed FP32 (v_pk_*_f32) anywhere in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    if os.path.exists(path):
        return path
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (ROCm is required to build libvllm_mi355x.so)")
    return found


def _compile(src: str) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    obj = os.path.join(OBJDIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd.insert(1, "-x")
        cmd.insert(2, "hip")
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compiling {src} failed:\n{res.stdout}\n{res.stderr}")
    return obj


def _check_undefined(library: str) -> None:
    """A shared library links with undefined symbols, which only fail when it
    is loaded: reject a kernel launch stub the host compilation did not emit
    (clang can drop one silently) or any other symbol of this project."""
    nm = shutil.which("nm")
    if not nm:
        return
    res = subprocess.run([nm, "-u", "-C", library], capture_output=True, text=True)
    bad = [line.strip() for line in res.stdout.splitlines()
           if "__device_stub__" in line or any(ns in line for ns in ("exl3::", "marlin::", "vq::"))]
    if bad:
        os.remove(library)
        raise RuntimeError("linked library has undefined project symbols:\n  " + "\n  ".join(bad[:10]))


def build(jobs: int | None = None, verbose: bool = False) -> str:
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, SOURCES))
    tmp = LIBRARY + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"linking failed:\n{res.stdout}\n{res.stderr}")
    _check_undefined(tmp)
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}")
    return LIBRARY


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--jobs", type=int, default=None)
    args = parser.parse_args()
    build(args.jobs, verbose=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
