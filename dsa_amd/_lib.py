"""ctypes binding of ``libdsa_mi355x.so`` (C ABI: include/dsa_mi355x.h).

The library is required: there is no fallback path.  Loading it touches no
GPU (the planning entry points are pure host logic), so the binding also works
on a machine without a device.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libdsa_mi355x.so"

# Every entry point the header declares, with its ctypes signature.
_i32, _i64, _vp = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p


class DsaPlan(ctypes.Structure):
    """Mirror of ``struct dsa_plan``."""

    _fields_ = [
        ("heads_per_group", ctypes.c_int32),
        ("tile_rows", ctypes.c_int32),
        ("split", ctypes.c_int32),
        ("kv_waves", ctypes.c_int32),
        ("stages", ctypes.c_int32),
        ("mfma", ctypes.c_int32),
        ("fused_merge", ctypes.c_int32),
        ("pv_cols", ctypes.c_int32),
    ]


class DsaFwdOptions(ctypes.Structure):
    """Mirror of ``struct dsa_fwd_options``."""

    _fields_ = [
        ("scale", ctypes.c_float),
        ("block_size", ctypes.c_int32),
        ("max_blocks", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32),
        ("block_table", ctypes.c_void_p),
        ("kv_format", ctypes.c_int32),
        ("reserved32", ctypes.c_int32),
        ("arrivals", ctypes.c_void_p),
    ]


KV_BF16 = 0  # DSA_KV_BF16
KV_FP8 = 1   # DSA_KV_FP8: 656-byte rows (512 e4m3, 4 fp32 scales, 64 bf16 rope)


SIGNATURES = {
    "dsa_version": (_i32, []),
    "dsa_last_error": (ctypes.c_char_p, []),
    "dsa_plan_for": (_i32, [_i32, _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(DsaPlan)]),
    "dsa_plan_for_opts": (_i32, [_i32, _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(DsaFwdOptions),
                                 ctypes.POINTER(DsaPlan)]),
    "dsa_plan_check": (_i32, [ctypes.POINTER(DsaPlan), _i32, _i32, _i32, _i32, _i32]),
    "dsa_partial_elems": (_i32, [ctypes.POINTER(DsaPlan), _i32, _i32, _i32,
                                 ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "dsa_fwd": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                       _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(DsaPlan), _vp]),
    "dsa_fwd_main": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                            _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(DsaPlan), _vp]),
    "dsa_fwd_opts": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                            _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(DsaFwdOptions),
                            ctypes.POINTER(DsaPlan), _vp]),
    "dsa_fwd_main_opts": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                 _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(DsaFwdOptions),
                                 ctypes.POINTER(DsaPlan), _vp]),
    "dsa_fwd_noalloc": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32,
                               ctypes.POINTER(DsaFwdOptions), ctypes.POINTER(DsaPlan), _vp]),
    "dsa_merge": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp]),
    "dsa_bucket_indices": (_i32, [_vp, _vp, _i32, _i32, _i32, _vp]),
    "dsa_project_uv": (_i32, [_vp, _vp, _i64, _vp, _i32, _i32, _i32, _vp]),
    "dsa_merge_uv": (_i32, [_vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp]),
    "dsa_indexer_logits": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp]),
    "dsa_indexer_topk": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp]),
    "dsa_indexer_topk_ws_bytes": (_i64, [_i32, _i32, _i32, _i32]),
    "dsa_indexer_topk_ws": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _i64, _vp]),
}

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load the kernel library once; raise if it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m dsa_amd.build` "
                    "(dsa_amd has no CPU or fallback path)")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def last_error() -> str:
    return load().dsa_last_error().decode(errors="replace")


def check(rc: int, what: str) -> None:
    """Turn a C status into a Python exception (< 0: ValueError, > 0: RuntimeError)."""
    if rc == 0:
        return
    msg = f"{what}: {last_error()}"
    if rc < 0:
        raise ValueError(msg)
    raise RuntimeError(msg)
