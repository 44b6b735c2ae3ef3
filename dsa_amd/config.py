"""Launch plans and the shape table of the MI355X sparse-MLA forward.

Replaces dsa/config.py of the reference (Tuning :10-19, CASE_SHAPES :23-40,
SELECTED :42-59, select :64-69).  The reference's Tuning fields described an
Ascend Cube/Vector pipeline; here the plan describes gfx950 workgroups:

* ``bm``       -- query heads per workgroup (divides H);
* ``bn``       -- gathered rows per LDS ring stage (32 or 64);
* ``split``    -- KV splits per (token, head group); > 1 adds the FP32 merge;
* ``kv_waves`` -- waves that share a head slice and split each tile's rows
                  (``bm // mfma * kv_waves == 4``: four waves per workgroup);
* ``stages``   -- LDS ring depth (2 or 4);
* ``mfma``     -- heads per wave: 32 (v_mfma_f32_32x32x16_bf16: bm 128 with
                  bn 32 and 4 stages, or bm 64 with kv_waves 2) or 16
                  (v_mfma_f32_16x16x32_bf16: bm 64, 32 or 16, bn 64, 2 stages);
* ``fused_merge`` -- with split in [2, 16] on a narrow plan (mfma 16), the
                  main kernel's last workgroup per (token, head group) merges
                  the partials: one launch instead of two, the same bits.
* ``pv_cols``  -- output columns one wave computes in PV (the reference's
                  Tuning.pv_cols): 512 (each wave: all columns for its own
                  rows) or 128 (the four waves split a 64-row tile's rows for
                  QK, exchange P through LDS and split the columns for PV;
                  mfma 16, kv_waves 4, bm 16, 32 or 64).

Unlike the reference, shapes outside the table are accepted: the library's
planner (``dsa_plan_for``) derives a plan for any supported shape.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

from . import _lib


@dataclass(frozen=True)
class Tuning:
    """Compile-time schedule of one call; never changes the math."""

    bm: int
    bn: int
    split: int
    kv_waves: int = 1
    stages: int = 2
    mfma: int = 32
    fused_merge: bool = False
    pv_cols: int = 512

    def to_c(self) -> _lib.DsaPlan:
        p = _lib.DsaPlan()
        p.heads_per_group, p.tile_rows, p.split = self.bm, self.bn, self.split
        p.kv_waves, p.stages, p.mfma = self.kv_waves, self.stages, self.mfma
        p.fused_merge = 1 if self.fused_merge else 0
        p.pv_cols = self.pv_cols
        return p

    @staticmethod
    def from_c(p: _lib.DsaPlan) -> "Tuning":
        return Tuning(p.heads_per_group, p.tile_rows, p.split, p.kv_waves, p.stages, p.mfma,
                      bool(p.fused_merge), p.pv_cols if p.pv_cols else 512)


# (batch, query length, heads, KV length, number of selected indices).
# The reference's 16 cases (dsa/config.py:23-40) plus the five MI355X
# benchmark configurations.
CASE_SHAPES = {
    "decode_b1": (1, 1, 128, 8192, 2048),
    "decode_b8": (8, 1, 128, 32768, 2048),
    "decode_b32": (32, 1, 128, 32768, 2048),
    "decode_tp8": (8, 1, 16, 32768, 2048),
    "prefill_q16": (1, 16, 128, 8192, 2048),
    "prefill_q64": (1, 64, 128, 32768, 2048),
    "prefill_tp8": (1, 128, 16, 32768, 2048),
    "prefill_k512": (1, 128, 64, 32768, 512),
    "decode_b4_h128": (4, 1, 128, 8192, 2048),
    "prefill_b4_h128": (4, 8192, 128, 8192, 2048),
    "decode_b4_h64": (4, 1, 64, 8192, 2048),
    "prefill_b4_h64": (4, 8192, 64, 8192, 2048),
    "decode_b4_h32": (4, 1, 32, 8192, 2048),
    "prefill_b4_h32": (4, 8192, 32, 8192, 2048),
    "decode_b4_h16": (4, 1, 16, 8192, 2048),
    "prefill_b4_h16": (4, 8192, 16, 8192, 2048),
    # MI355X benchmark configurations C1..C5
    "c1_decode_b1": (1, 1, 128, 8192, 2048),
    "c2_decode_b8": (8, 1, 128, 32768, 2048),
    "c3_decode_h16_mtp": (64, 2, 16, 65536, 2048),
    "c4_prefill_h16": (1, 4096, 16, 8192, 2048),
    "c5_prefill_h128": (1, 4096, 128, 32768, 2048),
}

MI355X_CUS = 256


def plan_for(shape, num_cus: int = MI355X_CUS, kv_fp8: bool = False) -> Tuning:
    """Default plan the library derives for ``shape`` on ``num_cus`` CUs (with
    ``kv_fp8``, among the variants that read 656-byte fp8 kv rows)."""
    b, sq, h, length, topk = shape
    out = _lib.DsaPlan()
    if kv_fp8:
        opts = _lib.DsaFwdOptions(kv_format=_lib.KV_FP8)
        rc = _lib.load().dsa_plan_for_opts(b, sq, h, length, topk, num_cus, ctypes.byref(opts), ctypes.byref(out))
    else:
        rc = _lib.load().dsa_plan_for(b, sq, h, length, topk, num_cus, ctypes.byref(out))
    _lib.check(rc, "dsa_plan_for")
    return Tuning.from_c(out)


def check_tuning(config: Tuning, shape) -> None:
    """Validate a caller-supplied plan (reference: dsa/api.py:41-60)."""
    if not isinstance(config, Tuning):
        raise TypeError("config must be a dsa_amd.Tuning")
    if any(type(v) is not int
           for v in (config.bm, config.bn, config.split, config.kv_waves, config.stages, config.mfma, config.pv_cols)):
        raise ValueError("Tuning fields must be int")
    if type(config.fused_merge) is not bool:
        raise ValueError("Tuning.fused_merge must be a bool")
    b, sq, h, length, topk = shape
    plan = config.to_c()
    _lib.check(_lib.load().dsa_plan_check(ctypes.byref(plan), b, sq, h, length, topk), "invalid Tuning")


# Per-shape plans for MI355X (256 CUs), the counterpart of the reference's
# table (dsa/config.py:42-59): the fastest plan of a measured sweep over
# every variant (narrow, wide, column-split PV, ping-pong) and split around 128-512
# workgroups, per shape; the library planner (dsa_plan_for, a cost model
# fitted to the same measurements) covers every other shape.  The
# column-split PV variants (pv_cols=128) won every 16- and 32-head plan
# (2-15 % over pv_cols=512); the in-kernel merge pays where a (token, head
# group) has little to merge (2 splits x 16 heads).
_XP16 = dict(kv_waves=4, mfma=16, pv_cols=128)
_XP32 = dict(kv_waves=4, mfma=16, pv_cols=128)
# The ping-pong variant (128 heads per workgroup, eight waves) beat wide<4,1>
# by 8 % on the two large 128-head prefills; on decode-sized shapes the
# column-split and narrow plans stay 20 % to 4x ahead.
_PP = dict(kv_waves=1, stages=4, mfma=16, pv_cols=128)
# Specialised waves (16 or 32 heads, 32-row tiles, four gather waves holding
# three tiles in registers): ahead by 4-9 % on the 8- and 32-token decodes
# (input sets cycled beyond the MALL) and the 16- and 128-query prefills
# with 32 heads per group.
_XS = dict(kv_waves=2, stages=4, mfma=16, pv_cols=128)
SELECTED = {
    "decode_b1": Tuning(16, 64, 16, **_XP16),
    "decode_b8": Tuning(32, 32, 8, **_XS),
    "decode_b32": Tuning(32, 32, 2, **_XS),
    "decode_tp8": Tuning(16, 64, 16, **_XP16),
    "prefill_q16": Tuning(32, 32, 4, **_XS),
    "prefill_q64": Tuning(32, 64, 1, **_XP32),
    "prefill_tp8": Tuning(16, 64, 2, fused_merge=True, **_XP16),
    "prefill_k512": Tuning(32, 32, 1, **_XS),
    "decode_b4_h128": Tuning(16, 64, 8, **_XP16),
    "prefill_b4_h128": Tuning(128, 32, 1, **_PP),
    "decode_b4_h64": Tuning(16, 64, 16, **_XP16),
    "prefill_b4_h64": Tuning(64, 64, 1, kv_waves=2),
    "decode_b4_h32": Tuning(16, 64, 16, **_XP16),
    "prefill_b4_h32": Tuning(32, 64, 1, **_XP32),
    "decode_b4_h16": Tuning(16, 64, 32, **_XP16),
    "prefill_b4_h16": Tuning(16, 64, 1, **_XP16),
    "c1_decode_b1": Tuning(16, 64, 16, **_XP16),
    "c2_decode_b8": Tuning(32, 32, 8, **_XS),
    "c3_decode_h16_mtp": Tuning(16, 64, 2, fused_merge=True, **_XP16),
    "c4_prefill_h16": Tuning(16, 64, 1, **_XP16),
    "c5_prefill_h128": Tuning(128, 32, 1, **_PP),
}
_BY_SHAPE = {}
for _name, _shape in CASE_SHAPES.items():
    _BY_SHAPE.setdefault(_shape, SELECTED[_name])


def select(shape, num_cus: int = MI355X_CUS, kv_fp8: bool = False) -> Tuning:
    """Plan for a shape: the table entry on a 256-CU device, else the planner's
    (fp8 kv rows: always the planner's, which keeps to the narrow variants)."""
    shape = tuple(shape)
    if not kv_fp8 and num_cus == MI355X_CUS and shape in _BY_SHAPE:
        return _BY_SHAPE[shape]
    return plan_for(shape, num_cus, kv_fp8)
