"""Build the gfx950 kernel library ``dsa_amd/libdsa_mi355x.so`` in-tree.

Usage: ``python -m dsa_amd.build`` (or ``__graft_entry__.build()``).  Compiles
the kernel sources in ``dsa_amd/csrc`` with ``hipcc --offload-arch=gfx950`` and
links one shared library exporting the C ABI of ``include/dsa_mi355x.h``, and
builds ``dsa_amd/_fast*.so``, the host fast path of ``forward`` (g++ against
the installed PyTorch-ROCm; no device code).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libdsa_mi355x.so"
OBJ_DIR = PKG / "_build"
SOURCES = ["sparse_mla_fwd.hip", "merge.hip", "project_uv.hip", "indexer.hip", "fwd_scratch.hip", "bucket_rows.hip",
           "abi.cpp"]
ARCH = "gfx950"
ROCM_INCLUDE = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "include"

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


def fast_path_module() -> Path:
    """Path of the host fast-path extension module (csrc/fast_forward.cpp)."""
    return PKG / ("_fast" + sysconfig.get_config_var("EXT_SUFFIX"))


def _compile_fast(verbose: bool) -> Path:
    """The host fast path of forward() as a CPython extension against the
    installed PyTorch-ROCm (host code only: g++ with torch's headers and
    libraries, the HIP headers for the stream type)."""
    import torch
    import torch.utils.cpp_extension as ce

    torch_dir = Path(torch.__file__).resolve().parent
    out = fast_path_module()
    tmp = out.with_suffix(".tmp")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-DTORCH_API_INCLUDE_EXTENSION_H", "-DTORCH_EXTENSION_NAME=_fast", "-D__HIP_PLATFORM_AMD__=1",
           "-DUSE_ROCM=1", *[f"-I{d}" for d in ce.include_paths()], f"-I{sysconfig.get_paths()['include']}",
           f"-I{ROCM_INCLUDE}", str(CSRC / "fast_forward.cpp"), "-o", str(tmp), f"-L{torch_dir / 'lib'}",
           "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
           f"-Wl,-rpath,{torch_dir / 'lib'}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"g++ failed for fast_forward.cpp:\n{res.stdout}{res.stderr}")
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> Path:
    """Compile all kernels for gfx950 and link the shared library, and build
    the host fast-path module (always rebuilds)."""
    OBJ_DIR.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES) + 1) as ex:
        fast = ex.submit(_compile_fast, verbose)
        objs = list(ex.map(lambda s: _compile(s, verbose), SOURCES))
        fast.result()
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
