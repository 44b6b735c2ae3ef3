"""The C-ABI library loads on the CPU and exports every symbol the header declares.

No compute entry point is called with device memory here; only argument
validation paths that return before any HIP call.
"""
import ctypes
import re
from pathlib import Path

import pytest

from dsa_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "dsa_mi355x.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(dsa_[a-z_]+)\s*\(", text)))


def test_header_declares_the_expected_entry_points():
    assert declared_functions() == sorted(
        ["dsa_version", "dsa_last_error", "dsa_plan_for", "dsa_plan_check", "dsa_partial_elems",
         "dsa_fwd", "dsa_fwd_main", "dsa_fwd_opts", "dsa_fwd_main_opts", "dsa_plan_for_opts", "dsa_merge",
         "dsa_indexer_logits", "dsa_indexer_topk", "dsa_indexer_topk_ws_bytes", "dsa_indexer_topk_ws",
         "dsa_project_uv", "dsa_merge_uv", "dsa_fwd_noalloc", "dsa_bucket_indices"])


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, name


def test_version_and_last_error():
    lib = _lib.load()
    # 1.1: dsa_plan.pv_cols and dsa_fwd_noalloc; 1.2: dsa_bucket_indices
    assert lib.dsa_version() == (1 << 16) | 2
    assert isinstance(lib.dsa_last_error(), bytes)


def test_magnitude_bound_follows_the_restart_clamp():
    """The header's kv magnitude bound is the one the kernels' restart clamp
    implies: a weight before the division by the sum reaches at most
    2^kRestartLog2, a workgroup sums at most DSA_IDX_CAP of them into an FP32
    accumulator, so max|kv| < 2^(128 - kRestartLog2 - log2(DSA_IDX_CAP)).
    An FP32 emulation of one accumulator shows both sides of the bound."""
    import math

    import numpy as np

    src = (HEADER.parents[1] / "dsa_amd" / "csrc" / "sparse_mla_fwd.hip").read_text()
    clamp = float(re.search(r"constexpr float kRestartLog2 = ([0-9.]+)f;", src).group(1))
    header = HEADER.read_text()
    cap = int(re.search(r"#define DSA_IDX_CAP (\d+)", header).group(1))
    bound_log2 = 128 - clamp - math.log2(cap)
    assert bound_log2 == 53
    assert "max|kv| < 2^53 (9.0e15)" in header and f"more than {int(clamp)} log2 units" in header
    weight = np.float32(2.0 ** clamp)
    with np.errstate(over="ignore"):
        for log2_kv, finite in ((bound_log2 - 0.01, True), (bound_log2 + 0.01, False)):
            acc = np.float32(0.0)
            term = np.float32(weight * np.float32(2.0 ** log2_kv))
            for _ in range(cap):  # one workgroup's slots, each at the largest weight
                acc = np.float32(acc + term)
            assert bool(np.isfinite(acc)) == finite, (log2_kv, acc)


def test_struct_layout_matches_header():
    assert ctypes.sizeof(_lib.DsaPlan) == 32
    assert _lib.DsaPlan.fused_merge.offset == 24 and _lib.DsaPlan.pv_cols.offset == 28
    # float, 3 x int32, pointer, 2 x int32, pointer
    assert ctypes.sizeof(_lib.DsaFwdOptions) == 40
    assert _lib.DsaFwdOptions.block_table.offset == 16
    assert _lib.DsaFwdOptions.kv_format.offset == 24
    assert _lib.DsaFwdOptions.arrivals.offset == 32
    text = HEADER.read_text()
    assert "#define DSA_KV_BF16 0" in text and "#define DSA_KV_FP8 1" in text
    assert (_lib.KV_BF16, _lib.KV_FP8) == (0, 1)


def test_plan_for_rejects_bad_shapes():
    lib = _lib.load()
    plan = _lib.DsaPlan()
    assert lib.dsa_plan_for(1, 1, 24, 10, 10, 256, ctypes.byref(plan)) < 0
    assert b"multiple of 16" in lib.dsa_last_error()
    assert lib.dsa_plan_for(0, 1, 16, 10, 10, 256, ctypes.byref(plan)) < 0
    assert lib.dsa_plan_for(1, 1, 16, 10, 10, 0, ctypes.byref(plan)) < 0
    assert lib.dsa_plan_for(1, 1, 16, 10, 10, 256, None) < 0
    assert lib.dsa_plan_for(1, 1, 16, 10, 10, 256, ctypes.byref(plan)) == 0
    assert lib.dsa_last_error() == b""


def test_fwd_and_merge_validate_before_any_launch():
    lib = _lib.load()
    null = None
    rc = lib.dsa_fwd(null, null, null, null, null, null, null, null, null, null, null,
                     1, 1, 16, 10, 10, None, None)
    assert rc < 0 and b"NULL" in lib.dsa_last_error()
    rc = lib.dsa_merge(null, null, null, null, null, null, 1, 16, 2, None)
    assert rc < 0
    rc = lib.dsa_fwd_main(null, null, null, null, null, null, null, null, null, null, null,
                          1, 1, 16, 10, 10, None, None)
    assert rc < 0


def test_partial_elems():
    lib = _lib.load()
    plan = _lib.DsaPlan(64, 64, 4, 2, 2, 32)
    o, ml = ctypes.c_int64(), ctypes.c_int64()
    assert lib.dsa_partial_elems(ctypes.byref(plan), 8, 1, 128, ctypes.byref(o), ctypes.byref(ml)) == 0
    assert (o.value, ml.value) == (8 * 4 * 128 * 512, 8 * 4 * 128)
    plan.split = 1
    assert lib.dsa_partial_elems(ctypes.byref(plan), 8, 1, 128, ctypes.byref(o), ctypes.byref(ml)) == 0
    assert (o.value, ml.value) == (0, 0)


@pytest.mark.parametrize("split", [1, 3, 32])
def test_plan_check_accepts_valid(split):
    lib = _lib.load()
    plan = _lib.DsaPlan(64, 64, split, 2, 2, 32)
    assert lib.dsa_plan_check(ctypes.byref(plan), 1, 1, 128, 8192, 2048) == 0


def _opts_call(lib, opts, L=1024):
    """dsa_fwd_opts with fake (never dereferenced) 16-byte aligned pointers:
    every case below must be rejected before any HIP call."""
    fake = ctypes.c_void_p(1 << 20)
    return lib.dsa_fwd_opts(fake, fake, fake, fake, fake, fake, fake, fake, None, None, None,
                            1, 1, 16, L, 64, ctypes.byref(opts), None, None)


def test_fwd_opts_validate_before_any_launch():
    lib = _lib.load()
    for bad in (-1.0, float("inf"), float("nan")):
        assert _opts_call(lib, _lib.DsaFwdOptions(scale=bad)) < 0
        assert b"scale" in lib.dsa_last_error()
    table = ctypes.c_void_p(1 << 20)
    # L must equal max_blocks * block_size
    o = _lib.DsaFwdOptions(block_size=64, max_blocks=8, num_blocks=100, block_table=table)
    assert _opts_call(lib, o, L=1000) < 0 and b"max_blocks" in lib.dsa_last_error()
    # non-positive geometry
    o = _lib.DsaFwdOptions(block_size=0, max_blocks=8, num_blocks=100, block_table=table)
    assert _opts_call(lib, o, L=0 + 1024) < 0 and b"positive" in lib.dsa_last_error()
    # pool too large for 32-bit row offsets
    o = _lib.DsaFwdOptions(block_size=64, max_blocks=16, num_blocks=1 << 19, block_table=table)
    assert _opts_call(lib, o, L=1024) < 0 and b"33554432" in lib.dsa_last_error()
    # misaligned block table
    o = _lib.DsaFwdOptions(block_size=64, max_blocks=16, num_blocks=100, block_table=ctypes.c_void_p((1 << 20) + 2))
    assert _opts_call(lib, o, L=1024) < 0 and b"aligned" in lib.dsa_last_error()


def test_fused_merge_plan_checks():
    lib = _lib.load()
    shape = (8, 1, 128, 32768, 2048)
    ok = _lib.DsaPlan(32, 64, 8, 2, 2, 16, 1)
    assert lib.dsa_plan_check(ctypes.byref(ok), *shape) == 0
    # split 1 is accepted (nothing to merge)
    assert lib.dsa_plan_check(ctypes.byref(_lib.DsaPlan(32, 64, 1, 2, 2, 16, 1)), *shape) == 0
    for bad, msg in ((_lib.DsaPlan(32, 64, 8, 2, 2, 16, 2), b"0 or 1"),
                     (_lib.DsaPlan(64, 64, 4, 2, 2, 32, 1), b"narrow"),      # wide variant
                     (_lib.DsaPlan(32, 64, 17, 2, 2, 16, 1), b"split <= 16"),
                     (_lib.DsaPlan(32, 64, 8, 4, 2, 16, 1, 128), b"16 heads per group"),  # column-split PV, 32 heads
                     (_lib.DsaPlan(32, 64, 8, 2, 2, 16, 0, 1), b"pv_cols")):
        assert lib.dsa_plan_check(ctypes.byref(bad), *shape) < 0
        assert msg in lib.dsa_last_error(), lib.dsa_last_error()
    # misaligned arrival counters are rejected before any launch
    o = _lib.DsaFwdOptions(arrivals=ctypes.c_void_p((1 << 20) + 2))
    assert _opts_call(lib, o) < 0 and b"arrivals" in lib.dsa_last_error()


@pytest.mark.parametrize("shape", [(8, 1, 128, 32768, 2048), (64, 2, 16, 65536, 2048), (1, 1, 128, 8192, 2048),
                                   (1, 4096, 128, 32768, 2048)])
def test_planner_fused_merge_only_where_supported(shape):
    lib = _lib.load()
    plan = _lib.DsaPlan()
    assert lib.dsa_plan_for(*shape, 256, ctypes.byref(plan)) == 0
    if plan.fused_merge:
        assert plan.mfma == 16 and 1 < plan.split <= 16
    assert lib.dsa_plan_check(ctypes.byref(plan), *shape) == 0


def test_fp8_kv_format_validation():
    lib = _lib.load()
    assert _opts_call(lib, _lib.DsaFwdOptions(kv_format=2)) < 0 and b"kv_format" in lib.dsa_last_error()
    assert _opts_call(lib, _lib.DsaFwdOptions(reserved32=1)) < 0 and b"reserved" in lib.dsa_last_error()
    # fp8 rows are read by the narrow (mfma 16) variants only; k_rope may be NULL
    fake = ctypes.c_void_p(1 << 20)
    wide = _lib.DsaPlan(128, 32, 1, 1, 4, 32)
    o = _lib.DsaFwdOptions(kv_format=_lib.KV_FP8)
    rc = lib.dsa_fwd_opts(fake, fake, fake, None, fake, fake, fake, fake, None, None, None,
                          1, 1, 128, 1024, 64, ctypes.byref(o), ctypes.byref(wide), None)
    assert rc < 0 and b"narrow" in lib.dsa_last_error()
    # without fp8 a NULL k_rope is an error
    narrow = _lib.DsaPlan(64, 64, 1, 1, 2, 16)
    rc = lib.dsa_fwd_opts(fake, fake, fake, None, fake, fake, fake, fake, None, None, None,
                          1, 1, 128, 1024, 64, ctypes.byref(_lib.DsaFwdOptions()), ctypes.byref(narrow), None)
    assert rc < 0 and b"NULL" in lib.dsa_last_error()


@pytest.mark.parametrize("shape", [(8, 1, 128, 32768, 2048), (64, 2, 16, 65536, 2048), (1, 4096, 128, 32768, 2048)])
def test_fp8_planner_keeps_to_narrow_variants(shape):
    lib = _lib.load()
    plan = _lib.DsaPlan()
    o = _lib.DsaFwdOptions(kv_format=_lib.KV_FP8)
    assert lib.dsa_plan_for_opts(*shape, 256, ctypes.byref(o), ctypes.byref(plan)) == 0
    assert plan.mfma == 16 and lib.dsa_plan_check(ctypes.byref(plan), *shape) == 0
    bad = _lib.DsaFwdOptions(kv_format=5)
    assert lib.dsa_plan_for_opts(*shape, 256, ctypes.byref(bad), ctypes.byref(plan)) < 0
    # NULL options plan like dsa_plan_for
    ref = _lib.DsaPlan()
    assert lib.dsa_plan_for(*shape, 256, ctypes.byref(ref)) == 0
    assert lib.dsa_plan_for_opts(*shape, 256, None, ctypes.byref(plan)) == 0
    assert bytes(plan) == bytes(ref)


def test_indexer_topk_workspace_sizes_and_checks():
    lib = _lib.load()
    # few rows: 8 workgroups per row, each row (8 x (4096 + 64) histogram bins + 8 x 4 + L words)
    # rounded to 4 words
    words = (8 * (4096 + 64) + 32 + 32768 + 3) // 4 * 4
    assert lib.dsa_indexer_topk_ws_bytes(8, 1, 32768, 2048) == 8 * words * 4
    assert lib.dsa_indexer_topk_ws_bytes(32, 1, 1000, 100) > 0
    assert lib.dsa_indexer_topk_ws_bytes(64, 2, 65536, 2048) == 0   # many rows: one workgroup per row
    assert lib.dsa_indexer_topk_ws_bytes(0, 1, 100, 10) == 0
    fake = ctypes.c_void_p(1 << 20)
    need = lib.dsa_indexer_topk_ws_bytes(2, 1, 1000, 100)
    assert lib.dsa_indexer_topk_ws(fake, fake, fake, 2, 1, 1000, 100, fake, need - 1, None) < 0
    assert b"workspace" in lib.dsa_last_error()
    assert lib.dsa_indexer_topk_ws(fake, fake, fake, 2, 1, 1000, 100, ctypes.c_void_p((1 << 20) + 4), need,
                                   None) < 0
    assert b"aligned" in lib.dsa_last_error()
    assert lib.dsa_indexer_topk_ws(None, fake, fake, 2, 1, 1000, 100, fake, need, None) < 0


def test_indexer_entry_points_validate_before_any_launch():
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 20)
    assert lib.dsa_indexer_logits(None, fake, fake, fake, fake, 1, 1, 64, 100, None) < 0
    assert lib.dsa_indexer_logits(fake, fake, fake, fake, fake, 1, 1, 48, 100, None) < 0
    assert b"32 or 64" in lib.dsa_last_error()
    assert lib.dsa_indexer_logits(fake, fake, fake, fake, fake, 1, 1, 64, 1 << 24, None) < 0
    assert lib.dsa_indexer_logits(fake, ctypes.c_void_p((1 << 20) + 8), fake, fake, fake, 1, 1, 64, 100, None) < 0
    assert b"aligned" in lib.dsa_last_error()
    assert lib.dsa_indexer_topk(fake, fake, None, 1, 1, 100, 10, None) < 0
    assert lib.dsa_indexer_topk(fake, fake, fake, 1, 1, 100, 0, None) < 0
    # grid limits: 256-thread workgroups per 256 query heads, 1024-thread workgroups per row
    assert lib.dsa_indexer_logits(fake, fake, fake, fake, fake, 1 << 16, 1024, 64, 100, None) < 0
    assert b"query groups" in lib.dsa_last_error()
    assert lib.dsa_indexer_topk(fake, fake, fake, 1 << 11, 1 << 11, 100, 10, None) < 0
    assert b"4194304" in lib.dsa_last_error()


def test_w_uv_entry_points_validate_before_any_launch():
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 20)
    stride = 128 * 512
    assert lib.dsa_project_uv(None, fake, stride, fake, 8, 16, 128, None) < 0
    assert lib.dsa_project_uv(fake, fake, stride, fake, 0, 16, 128, None) < 0
    for dv in (0, 32, 100, 320):
        assert lib.dsa_project_uv(fake, fake, stride, fake, 8, 16, dv, None) < 0
        assert b"dv" in lib.dsa_last_error()
    assert lib.dsa_project_uv(fake, fake, stride - 8, fake, 8, 16, 128, None) < 0    # heads overlap
    assert lib.dsa_project_uv(fake, fake, stride + 4, fake, 8, 16, 128, None) < 0    # not 16-byte rows
    assert b"w_head_stride" in lib.dsa_last_error()
    assert lib.dsa_project_uv(fake, ctypes.c_void_p((1 << 20) + 8), stride, fake, 8, 16, 128, None) < 0
    assert lib.dsa_project_uv(fake, fake, stride, ctypes.c_void_p((1 << 20) + 2), 8, 16, 128, None) < 0
    assert lib.dsa_project_uv(ctypes.c_void_p((1 << 20) + 8), fake, stride, fake, 8, 16, 128, None) < 0
    assert b"aligned" in lib.dsa_last_error()
    assert lib.dsa_project_uv(fake, fake, stride, fake, 1 << 30, 1 << 10, 128, None) < 0
    assert lib.dsa_project_uv(fake, fake, 256 * 512, fake, 8, 1 << 17, 256, None) < 0
    assert b"H * dv" in lib.dsa_last_error()
    assert lib.dsa_merge_uv(fake, fake, None, fake, stride, fake, fake, fake, 8, 16, 2, 128, None) < 0
    assert lib.dsa_merge_uv(fake, fake, fake, fake, stride, fake, fake, fake, 8, 16, 0, 128, None) < 0
    assert lib.dsa_merge_uv(fake, fake, fake, fake, stride, fake, fake, fake, 8, 16, 2, 96, None) < 0
    assert lib.dsa_merge_uv(ctypes.c_void_p((1 << 20) + 4), fake, fake, fake, stride, fake, fake, fake,
                            8, 16, 2, 128, None) < 0


C_PROGRAM = r"""
#include <stdio.h>
#include "dsa_mi355x.h"
int main(void) {
    dsa_plan plan;
    int64_t po = 0, pml = 0;
    int rc = dsa_plan_for(8, 1, 128, 32768, 2048, 256, &plan);
    if (rc == 0) rc = dsa_partial_elems(&plan, 8, 1, 128, &po, &pml);
    int bad = dsa_fwd(0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 8, 1, 128, 32768, 2048, &plan, 0);
    printf("%d %d %d %lld %lld %d %s\n", dsa_version(), rc, plan.split, (long long)po, (long long)pml, bad,
           dsa_last_error());
    return 0;
}
"""


def test_header_is_plain_c_and_links(tmp_path):
    """A C99 program includes the header on its own (no HIP headers, no
    platform macro) and calls the library: what a cgo / FFI binding does."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    lib = _lib.load()._name
    src = tmp_path / "t.c"
    src.write_text(C_PROGRAM)
    exe = tmp_path / "t"
    libdir = str(Path(lib).parent)
    res = subprocess.run([gcc, "-std=c99", "-Wall", "-Wextra", "-Werror", f"-I{HEADER.parent}", str(src),
                          f"-L{libdir}", "-ldsa_mi355x", f"-Wl,-rpath,{libdir}", "-o", str(exe)],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stderr
    version, rc, split, po, pml, bad, *msg = out.stdout.split()
    assert int(version) == _lib.load().dsa_version() and int(rc) == 0 and int(split) >= 1
    assert (int(po) > 0) == (int(split) > 1) and int(pml) * 512 == int(po)
    assert int(bad) < 0 and "NULL" in " ".join(msg)


def test_column_split_pv_plan_checks():
    """pv_cols = 128 (the reference's Tuning.pv_cols): four waves, 64-row
    tiles, 16 / 32 / 64 heads per group; 0 means 512."""
    lib = _lib.load()
    shape = (8, 1, 128, 32768, 2048)
    for hpg in (16, 32, 64):
        ok = _lib.DsaPlan(hpg, 64, 8, 4, 2, 16, 0, 128)
        assert lib.dsa_plan_check(ctypes.byref(ok), *shape) == 0, lib.dsa_last_error()
    assert lib.dsa_plan_check(ctypes.byref(_lib.DsaPlan(16, 64, 8, 4, 2, 16, 1, 128)), *shape) == 0
    assert lib.dsa_plan_check(ctypes.byref(_lib.DsaPlan(32, 64, 8, 2, 2, 16, 0, 512)), *shape) == 0
    for bad in (_lib.DsaPlan(32, 64, 8, 2, 2, 16, 0, 128),     # kv_waves must be 4
                _lib.DsaPlan(128, 32, 8, 4, 4, 32, 0, 128),    # wide
                _lib.DsaPlan(32, 64, 8, 4, 2, 16, 0, 256)):    # 256 is not a variant
        assert lib.dsa_plan_check(ctypes.byref(bad), *shape) < 0
    # 64 heads: at most 1024 slots per workgroup, so TOPK 2048 needs split >= 2
    assert lib.dsa_plan_check(ctypes.byref(_lib.DsaPlan(64, 64, 1, 4, 2, 16, 0, 128)), *shape) < 0
    assert b"1024 slots" in lib.dsa_last_error()
    assert lib.dsa_plan_check(ctypes.byref(_lib.DsaPlan(64, 64, 2, 4, 2, 16, 0, 128)), *shape) == 0
    # fp8 rows are read by the pv_cols 512 narrow variants only
    fake = ctypes.c_void_p(1 << 20)
    o = _lib.DsaFwdOptions(kv_format=_lib.KV_FP8)
    plan = _lib.DsaPlan(16, 64, 1, 4, 2, 16, 0, 128)
    assert lib.dsa_fwd_opts(fake, fake, fake, fake, fake, fake, fake, fake, None, None, None, 1, 1, 16, 4096, 64,
                            ctypes.byref(o), ctypes.byref(plan), None) < 0
    assert b"pv_cols 512" in lib.dsa_last_error()
