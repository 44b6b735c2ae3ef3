"""Build the C oracle (test infrastructure) into ``oracle/_build/libdsa_oracle.so``.

The reference implementation itself cannot be built here: its kernels are
Triton-Ascend TLA programs that need torch_npu, the TLA compiler extension and
Ascend hardware, so there is no ``oracle/_ref``.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "dsa_oracle.c"
OUT = HERE / "_build" / "libdsa_oracle.so"


def build() -> Path:
    OUT.parent.mkdir(exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-fopenmp", "-shared", "-fPIC", "-std=c11", "-Wall", str(SRC), "-o", str(tmp), "-lm"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}{res.stderr}")
    tmp.replace(OUT)
    return OUT


if __name__ == "__main__":
    print(build())
