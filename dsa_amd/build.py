"""Build the gfx950 kernel library ``dsa_amd/libdsa_mi355x.so`` in-tree.

Usage: ``python -m dsa_amd.build`` (or ``__graft_entry__.build()``).  Compiles
every source in ``dsa_amd/csrc`` with ``hipcc --offload-arch=gfx950`` and links
one shared library exporting the C ABI of ``include/dsa_mi355x.h``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libdsa_mi355x.so"
OBJ_DIR = PKG / "_build"
SOURCES = ["sparse_mla_fwd.hip", "merge.hip", "project_uv.hip", "indexer.hip", "fwd_scratch.hip", "abi.cpp"]
ARCH = "gfx950"

COMMON = [
    "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
    f"-I{ROOT / 'include'}",
]
# Device-only code-generation flag: keep hipcc from forming packed-FP32 ops.
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build dsa_amd")
    return path


def _compile(src: str, verbose: bool) -> Path:
    obj = OBJ_DIR / (src + ".o")
    cmd = [hipcc(), *COMMON, *DEVICE, "-c", str(CSRC / src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that warning is noise.
    noise = "is not a recognized feature for this target"
    msgs = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{msgs}")
    if verbose and msgs.strip():
        print(msgs, flush=True)
    return obj


def build(verbose: bool = False) -> Path:
    """Compile all kernels for gfx950 and link the shared library (always rebuilds)."""
    OBJ_DIR.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *DEVICE, "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
