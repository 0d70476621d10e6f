"""Build ``libkdattn.so`` for gfx950 with hipcc (in-tree, no JIT cache).

Each ``csrc/*.hip`` file compiles to an object in ``_build/`` in parallel and
the objects link into ``kerneldev_amd/libkdattn.so``.  The library links the
HIP runtime by SONAME (``libamdhip64.so.7``); at run time that resolves to
the copy torch has already loaded.

Usage: ``python -m kerneldev_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(ROOT, "_build")
LIB = os.path.join(PKG, "libkdattn.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    # packed fp32 VALU ops are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


def build_library(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    cc = hipcc()
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
    objs = []

    def compile_one(src):
        obj = os.path.join(BUILD, src[:-4] + ".o")
        _run([cc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        return obj

    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = LIB + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


C_ABI_SRC = os.path.join(ROOT, "tests", "c_abi", "attn_from_c.c")
C_ABI_BIN = os.path.join(ROOT, "tests", "c_abi", "attn_from_c")


def build_c_abi_check(verbose: bool = False) -> str:
    """The C caller of the library (tests/c_abi/attn_from_c.c), built with gcc
    against the HIP runtime's C API and libkdattn.so (found through its rpath)."""
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    _run(["gcc", "-std=c11", "-O2", "-Wall", "-D__HIP_PLATFORM_AMD__", f"-I{rocm}/include",
          f"-I{os.path.join(ROOT, 'include')}", C_ABI_SRC, "-o", C_ABI_BIN, f"-L{PKG}", "-lkdattn",
          f"-L{rocm}/lib", "-lamdhip64", "-lm", "-Wl,-rpath,$ORIGIN/../../kerneldev_amd", f"-Wl,-rpath,{rocm}/lib"])
    if verbose:
        print(f"built {C_ABI_BIN}")
    return C_ABI_BIN


if __name__ == "__main__":
    build_library(verbose=True)
    build_c_abi_check(verbose=True)
    sys.exit(0)
