"""Build the MI355X paged FP8 decode libraries in-tree (gfx950).

Two shared objects land next to this file:

* ``libl20_paged_decode_hip.so`` -- the HIP kernels and the C ABI declared in
  ``include/l20_paged_decode.h`` (built by hipcc; no torch dependency).
* ``l20_paged_decode_ops.so`` -- the ``TORCH_LIBRARY(l20_stack)`` binding,
  linked against the first one with an ``$ORIGIN`` rpath (built by g++
  against the installed torch headers).

Usage: ``python l20_pd_build.py`` (or ``build_all()`` from Python).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
INCLUDE = ROOT / "include"
HIP_LIB = HERE / "libl20_paged_decode_hip.so"
OPS_LIB = HERE / "l20_paged_decode_ops.so"
ARCH = os.environ.get("L20_PD_ARCH", "gfx950")
# The decode kernels and the paged KV-cache producer, one shared object.
HIP_SOURCES = [CSRC / "l20_paged_decode_fp8.hip", CSRC / "l20_kv_write.hip", CSRC / "l20_tree_suffix.hip"]

# Packed-FP32 VALU forms are kept out of every HIP build.
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the MI355X library)")


def _run(cmd, verbose: bool) -> None:
    if verbose:
        print(" ".join(str(c) for c in cmd), flush=True)
    proc = subprocess.run([str(c) for c in cmd], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}):\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def build_hip_library(verbose: bool = False) -> Path:
    tmp = HIP_LIB.with_suffix(".so.tmp")
    _run([_hipcc(), *HIP_FLAGS, f"-I{INCLUDE}", *HIP_SOURCES, "-o", tmp], verbose)
    os.replace(tmp, HIP_LIB)
    return HIP_LIB


def build_torch_ops(verbose: bool = False) -> Path:
    import torch
    from torch.utils import cpp_extension

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    includes = [f"-I{p}" for p in cpp_extension.include_paths()] + [f"-I{INCLUDE}", "-I/opt/rocm/include"]
    libdirs = cpp_extension.library_paths()
    tmp = OPS_LIB.with_suffix(".so.tmp")
    cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        *includes, CSRC / "l20_paged_decode_ops.cpp",
        *[f"-L{d}" for d in libdirs], "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
        f"-L{HERE}", "-l:libl20_paged_decode_hip.so",
        "-Wl,-rpath,$ORIGIN", *[f"-Wl,-rpath,{d}" for d in libdirs],
        "-L/opt/rocm/lib", "-lamdhip64",
        "-o", tmp,
    ]
    _run(cmd, verbose)
    os.replace(tmp, OPS_LIB)
    return OPS_LIB


def build_all(verbose: bool = False) -> None:
    build_hip_library(verbose)
    build_torch_ops(verbose)


if __name__ == "__main__":
    build_all(verbose="-q" not in sys.argv)
    print(f"built {HIP_LIB.name} and {OPS_LIB.name}")
