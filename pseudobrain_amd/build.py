"""Build the HIP library of the operator for gfx950: pseudobrain_amd/libpbgdn.so.

One shared library holds both kernels and the C ABI declared in include/pbgdn.h.
It is compiled in-tree with hipcc (objects in parallel, then one link) and loaded
with ctypes by pseudobrain_amd._lib; it links the HIP runtime by soname, so in a
process that imported torch it binds to the runtime torch already loaded.

    python -m pseudobrain_amd.build
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(PKG, "libpbgdn.so")
# The debug build (-DPBGDN_DEBUG): every kernel fills its LDS with NaN before
# use, and the entry points fill their outputs and workspaces with NaN before
# launching, so that a read of unwritten LDS or an output element no kernel
# writes shows as NaN (tests/test_gpu_debug_canaries.py).
DEBUG_LIB = os.path.join(PKG, "libpbgdn_debug.so")
SOURCES = ("abi.hip", "recurrent.hip", "chunk.hip", "chunk_prep.hip", "chunk_scan.hip", "chunk_wide.hip",
           "chunk_k256.hip", "chunk_bwd.hip", "chunk_residuals.hip",
           "layer.hip", "decode_layer.hip", "device.hip")
ARCH = "gfx950"

# Packed fp32 VALU instructions are disabled (-packed-fp32-ops): the kernels
# are written in scalar / vector-of-4 float code and must not be turned into
# v_pk_*_f32 forms. hipcc's host pass warns that it does not know the feature.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    return path if os.path.exists(path) else "hipcc"


def _run(cmd):
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}{proc.stderr}")
    return proc


def build(verbose: bool = False) -> str:
    """Compile every source and link libpbgdn.so and libpbgdn_debug.so; returns
    the path of the first."""
    cc = hipcc()
    libs = []  # (library, objects)
    jobs = []
    for lib, objdir, extra in ((LIB, "_build", []), (DEBUG_LIB, "_build_debug", ["-DPBGDN_DEBUG"])):
        objdir = os.path.join(PKG, objdir)
        os.makedirs(objdir, exist_ok=True)
        objs = []
        for src in SOURCES:
            obj = os.path.join(objdir, src.replace(".hip", ".o"))
            objs.append(obj)
            jobs.append([cc, *HIPCC_FLAGS, *extra, f"-I{INCLUDE}", "-c", os.path.join(CSRC, src), "-o", obj])
        libs.append((lib, objs))
    with ThreadPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 8)) as pool:
        for proc in pool.map(_run, jobs):
            if verbose and proc.stderr:
                sys.stderr.write(proc.stderr)
    for lib, objs in libs:
        tmp = lib + ".tmp"
        _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
        os.replace(tmp, lib)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
