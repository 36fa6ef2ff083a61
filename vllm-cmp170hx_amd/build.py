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

# (source, object name, extra flags).  The small-M GEMV instantiations are
# one source compiled once per part of the format list, so they build in
# parallel (exl3_gemv.h); the tile GEMM's likewise.
GEMV_PARTS = 8
TILE_PARTS = 4  # the tile GEMM's instantiations likewise (exl3_tile.h)
# The slowest sources first.
SOURCES = [("exl3_gemv_part.hip", f"exl3_gemv_part{p}", [f"-DVQ_GEMV_PART={p}"]) for p in range(GEMV_PARTS)] + \
          [("exl3_tile_part.hip", f"exl3_tile_part{p}", [f"-DVQ_TILE_PART={p}"]) for p in range(TILE_PARTS)] + \
          [("marlin_moe.hip", "marlin_moe", []), ("exl3_gemm.hip", "exl3_gemm", []),
           ("exl3_linear.hip", "exl3_linear", []), ("exl3_moe.hip", "exl3_moe", []),
           ("exl3_ple.hip", "exl3_ple", []),
           ("common.cpp", "common", [])]

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


def _compile(entry) -> str:
    src, name, flags = entry
    os.makedirs(OBJDIR, exist_ok=True)
    obj = os.path.join(OBJDIR, name + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *flags, *_format_flags(), "-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd.insert(1, "-x")
        cmd.insert(2, "hip")
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compiling {src} failed:\n{res.stdout}\n{res.stderr}")
    return obj


def _format_flags() -> list:
    """VQ_BUILD_FORMATS="8,2 3,2" restricts the EXL3 formats compiled (a
    development build; the library then refuses the others)."""
    spec = os.environ.get("VQ_BUILD_FORMATS", "").strip()
    if not spec:
        return []
    pairs = [tuple(int(v) for v in item.split(",")) for item in spec.split()]
    return ["-DVQ_EXL3_FORMATS(X)=" + " ".join(f"X({b}, {c})" for b, c in pairs)]


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


TORCH_LIBRARY_PATH = os.path.join(PACKAGE, "libvllm_mi355x_torch.so")


def build_torch_classes(verbose: bool = False) -> str:
    """libvllm_mi355x_torch.so: the host-only torch custom classes the
    reference's loader requires (csrc/torch_classes.cpp), built with g++
    against the installed torch."""
    import torch
    from torch.utils import cpp_extension

    cxx = shutil.which("g++") or shutil.which("c++")
    if not cxx:
        raise RuntimeError("g++ not found (needed for libvllm_mi355x_torch.so)")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [cxx, "-O2", "-fPIC", "-shared", "-std=c++17", "-w", f"-D_GLIBCXX_USE_CXX11_ABI={abi}"]
    cmd += [f"-I{p}" for p in cpp_extension.include_paths()]
    cmd += [os.path.join(CSRC, "torch_classes.cpp"), "-o", TORCH_LIBRARY_PATH + ".tmp"]
    cmd += [f"-L{p}" for p in cpp_extension.library_paths()]
    cmd += ["-lc10", "-ltorch_cpu", "-ltorch"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"building libvllm_mi355x_torch.so failed:\n{res.stdout}\n{res.stderr}")
    os.replace(TORCH_LIBRARY_PATH + ".tmp", TORCH_LIBRARY_PATH)
    if verbose:
        print(f"built {TORCH_LIBRARY_PATH}")
    return TORCH_LIBRARY_PATH


def build(jobs: int | None = None, verbose: bool = False) -> str:
    jobs = jobs or min(len(SOURCES), int(os.environ.get("MAX_JOBS", 0)) or os.cpu_count() or 1)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        classes = pool.submit(build_torch_classes, verbose)
        objs = list(pool.map(_compile, SOURCES))
        classes.result()
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
