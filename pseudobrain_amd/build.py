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
SOURCES = ("abi.hip", "recurrent.hip", "chunk.hip", "chunk_prep.hip", "chunk_scan.hip", "chunk_wide.hip",
           "chunk_bwd.hip",
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
    """Compile every source and link libpbgdn.so; returns its path."""
    objdir = os.path.join(PKG, "_build")
    os.makedirs(objdir, exist_ok=True)
    cc = hipcc()
    jobs = []
    for src in SOURCES:
        obj = os.path.join(objdir, src.replace(".hip", ".o"))
        jobs.append((obj, [cc, *HIPCC_FLAGS, f"-I{INCLUDE}", "-c", os.path.join(CSRC, src), "-o", obj]))
    with ThreadPoolExecutor(max_workers=len(jobs)) as pool:
        for proc in pool.map(lambda job: _run(job[1]), jobs):
            if verbose and proc.stderr:
                sys.stderr.write(proc.stderr)
    tmp = LIB + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *(obj for obj, _ in jobs)])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
