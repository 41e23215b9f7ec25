"""Build the gfx950 HIP library deepgemm_amd/libmegamoe_hip.so in-tree with hipcc.

Every .hip file under csrc/ is compiled for gfx950 only (no host-side fallback, no other
architecture) and linked into one shared library exposing the C ABI of
include/megamoe_hip.h. Usage: ``python -m deepgemm_amd.build`` or ``build()``.
"""
from __future__ import annotations

import concurrent.futures
import hashlib
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ_DIR = os.path.join(HERE, "_build")
LIB_NAME = "libmegamoe_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
# sha256 of the sources and flags the library was built from, written next to it by build()
HASH_PATH = LIB_PATH + ".srchash"
HEADER = os.path.join(os.path.dirname(HERE), "include", "megamoe_hip.h")
ARCH = "gfx950"

HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # keep the compiler from forming packed-FP32 VALU ops (v_pk_*_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the MI355X build needs ROCm's hipcc")


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def source_hash() -> str:
    """sha256 over every kernel source and header (csrc/*.hip, *.cuh, *.h, the C-ABI header)
    and the compiler flags: a library whose recorded hash differs is stale."""
    h = hashlib.sha256(" ".join(HIPCC_FLAGS).encode())
    files = sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".cuh", ".h")))
    for path in [os.path.join(CSRC, f) for f in files] + [HEADER]:
        h.update(os.path.basename(path).encode())
        with open(path, "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()


def _compile(src: str, hipcc: str, verbose: bool) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stdout}\n{res.stderr}")
    if verbose and res.stderr.strip():
        print(res.stderr, file=sys.stderr)
    return obj


def build(verbose: bool = False, jobs: int = 8) -> str:
    """Compile all kernels for gfx950 and link libmegamoe_hip.so; returns its path."""
    hipcc = _hipcc()
    digest = source_hash()  # of the sources as they are when the compiles start
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs)))) as ex:
        objs = list(ex.map(lambda s: _compile(s, hipcc, verbose), srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    with open(HASH_PATH, "w") as fh:
        fh.write(digest + "\n")
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
