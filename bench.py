"""Benchmark of the MI355X sparse-MLA forward (one JSON line on stdout).

python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2_decode_b8]

A step is one forward call (main kernel + FP32 split merge) over one batch of
synthetic inputs already resident in HBM.  The default workload is C2, the
headline decode case (B=8, SQ=1, H=128, L=32768, TOPK=2048).  Steps cycle
through ``--rotate`` independent input sets so that the gathered rows come
from HBM rather than from the 256 MB MALL of a previous call (C2, C3: the
sets' combined gathered rows exceed twice the MALL); the warm (single input
set) span is reported beside it.

Timing: K calls are launched back to back on one stream between two HIP
events (device-synchronised on both sides); the elapsed device time over K is
the span per call (the ``value``).  A call is what ``dsa_amd.forward``
enqueues: one ``dsa_fwd`` (main kernel + merge kernel, or the main kernel
alone with an in-kernel merge).  The main kernel alone (``dsa_fwd_main``)
and the merge alone are timed the same way (K launches each), which gives
the main kernel's average duration for the roofline.  An event between every launch would add
its own few microseconds to each interval, so none is recorded inside a
batch.  ``ms_per_step`` is the host wall clock of the K timed calls (median
over the rounds).
``breakdown.kernel_sum_us`` adds the two kernels' launch-alone durations, and
``breakdown.eager_call_us`` is the median wall clock of one ``dsa_amd.forward``
call (checks, allocation, launches) followed by a device synchronisation.

Every quantity is timed in R rounds (``--rounds``, default 5) of K calls,
interleaved (span, main alone, merge alone, then the next round); the line
gives the median and, in ``breakdown``, the min and max over the rounds.

The metric is "decode B=8 + prefill": the default line is C2 (``value``)
and carries the other GPU configurations timed the same way, as flat scalar
fields: ``decode`` holds C3 (``c3_span_us``, ``c3_span_min_us``,
``c3_frac``, ``c3_cpu_us`` ...) and C2's spread and fixed chain,
``prefill`` holds C5 and C4 (``c5_...``, ``c4_...``); ``roofline`` repeats
their ``frac`` / ``frac_span`` and ``cpu_baseline`` their CPU values
(``--no-legs`` leaves them out).  ``roofline.frac`` is the main kernel's
(its average launch); ``roofline.frac_span`` is the whole call's, split
merge included.  ``breakdown.fixed_chain_us`` is C2's plan on the same input
sets with one tile per workgroup (TOPK = split x tile rows): the part of a
call that does not scale with the gathered rows.

The warm-up and every timed batch walk one continuous rotation over the input
sets, so the warm-up leaves none of the first timed sets in the caches.

``--cases all`` times the reference's 16 validated cases instead, one line
each (span, main, merge with the selected plan) beside the reference's
published Ascend950PR span for the case: context, not a baseline line.

cpu_baseline: the CPU oracle (oracle/dsa_oracle.py, a restatement of the
reference's FP32 PyTorch gather+softmax path) timed on this host on full
calls of the same workload (one warm-up call, then the median of 5 calls, or
of 3 for the 4096-query prefills), with every CPU the process may use
(capped by OMP_NUM_THREADS when the host sets it); the line records the
counts and the CPU model.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import subprocess
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import dsa_amd  # noqa: E402
from dsa_amd import Tuning, _lib  # noqa: E402
from dsa_amd.workloads import (BASELINE_CONFIGS, INDEXER_CONFIGS, baseline_inputs,  # noqa: E402
                               case_inputs, indexer_inputs)

METRIC = json.loads((ROOT / "BASELINE.json").read_text())["metric"]
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense bf16
# Published device span of the reference on Ascend950PR for the same shape
# (PERFORMANCE_FINAL.md:75 of the reference, decode_b8 task span).
PUBLISHED_SPAN_US = {"c2_decode_b8": 74.875}
# The reference's 16 validated cases (dsa/config.py:23-40) and its published
# device span per call on Ascend950PR (PERFORMANCE_FINAL.md:74-89 of the
# reference, refactored TLA column, merge included), for ``--cases``.
REF_CASES = ("decode_b1", "decode_b8", "decode_b32", "decode_tp8", "prefill_q16", "prefill_q64", "prefill_tp8",
             "prefill_k512", "decode_b4_h128", "decode_b4_h64", "decode_b4_h32", "decode_b4_h16",
             "prefill_b4_h128", "prefill_b4_h64", "prefill_b4_h32", "prefill_b4_h16")
REF_CASE_SPAN_US = {"decode_b1": 26.0, "decode_b8": 74.875, "decode_b32": 227.625, "decode_tp8": 47.25,
                    "prefill_q16": 116.0, "prefill_q64": 362.25, "prefill_tp8": 403.25, "prefill_k512": 134.25,
                    "decode_b4_h128": 51.25, "decode_b4_h64": 41.0, "decode_b4_h32": 35.25, "decode_b4_h16": 31.625,
                    "prefill_b4_h128": 139711.0, "prefill_b4_h64": 111399.0, "prefill_b4_h32": 96924.6,
                    "prefill_b4_h16": 89610.8}
# Which roofline binds each configuration.
BOUND = {"c1_decode_b1": "hbm", "c2_decode_b8": "hbm", "c3_decode_h16_mtp": "hbm",
         "c4_prefill_h16": "mfma", "c5_prefill_h128": "mfma"}
# Input sets cycled per workload.  C2 and C3 are HBM-bound headlines: their
# sets' combined gathered rows exceed twice the 256 MB MALL (C2: 32 x 18.9 MB,
# C3: 2 x 302 MB), so a set's rows have left the MALL when it comes round
# again.  C4 and C5 are cache-resident by design (9 MiB / 36 MiB of kv).
DEFAULT_ROTATE = {"c1_decode_b1": 16, "c2_decode_b8": 32, "c3_decode_h16_mtp": 2,
                  "c4_prefill_h16": 1, "c5_prefill_h128": 1}


def algorithmic_units(shape, fp8=False):
    """Gathered bytes and FLOPs of one call: every slot counted once
    (B*SQ*TOPK rows of 576 bf16, or of 656 bytes in the fp8 row format) and
    2*B*SQ*H*TOPK*(576+512) MFMA FLOPs."""
    b, sq, h, _, k = shape
    return b * sq * k * (656 if fp8 else 576 * 2), 2 * b * sq * h * k * (576 + 512)


class Call:
    """One preallocated forward call through the C ABI."""

    _uv_sets = 0  # W_UV weight tensors made so far (each call's own seed)

    def __init__(self, data, config: Tuning, block_table=None, fp8=False, uv_dim=0):
        self.data = data
        q = data[0]
        length = data[1].shape[1] if block_table is None else block_table.shape[1] * data[1].shape[1]
        self.shape = tuple(q.shape[:3]) + (length, data[4].shape[-1])
        self.opts = None
        if block_table is not None:  # paged kv: data[1], data[3] are block pools
            self.block_table = block_table
            self.opts = _lib.DsaFwdOptions(block_size=data[1].shape[1], max_blocks=block_table.shape[1],
                                           num_blocks=data[1].shape[0], block_table=block_table.data_ptr())
        if fp8:  # data[1] holds 656-byte rows, data[3] is None
            if self.opts is None:
                self.opts = _lib.DsaFwdOptions()
            self.opts.kv_format = _lib.KV_FP8
        b, sq, h, _, _ = self.shape
        self.config = config
        self.plan = config.to_c()
        dev = q.device
        # Fused-merge plan: one launch per call, the main kernel merging in
        # its last workgroup per (token, head group) on these arrival counters.
        self.fused = config.fused_merge and config.split > 1 and not uv_dim
        if self.fused:
            self.counters = torch.zeros(b * sq * (h // config.bm), device=dev, dtype=torch.int32)
            if self.opts is None:
                self.opts = _lib.DsaFwdOptions()
            self.opts.arrivals = self.counters.data_ptr()
        # Prefill-sized calls partition each token's indices by kv row range
        # first, as forward() does: full() runs the bucketing into this
        # buffer, main() reads it.
        self.bucket = dsa_amd.api.buckets_rows(self.shape)
        if self.bucket:
            self.order = dsa_amd.bucket_indices(data[4], self.shape[3])
        self.out = torch.empty_like(q)
        self.mx = torch.empty((b, 1, sq, h), device=dev, dtype=torch.float32)
        self.sm = torch.empty_like(self.mx)
        if config.split > 1:
            self.po = torch.empty((b, sq, config.split, h, 512), device=dev, dtype=torch.float32)
            self.pm = torch.empty((b, sq, config.split, h), device=dev, dtype=torch.float32)
            self.pl = torch.empty_like(self.pm)
        else:
            self.po = self.pm = self.pl = None
        p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
        ins = list(data[:4]) + [self.order if self.bucket else data[4]]
        self.args = [p(t) for t in ins] + [p(self.out), p(self.mx), p(self.sm), p(self.po), p(self.pm), p(self.pl)]
        self.lib = _lib.load()
        # W_UV projection after the attention: each call has its own weights
        # (one layer's [H, dv, 512]), so rotating calls do not share them.
        self.uv = uv_dim
        if uv_dim:
            Call._uv_sets += 1
            gen = torch.Generator(device=dev).manual_seed(1000 * uv_dim + Call._uv_sets)
            self.w = (torch.randn((h, uv_dim, 512), generator=gen, device=dev) / 512 ** 0.5).bfloat16()
            self.out_v = torch.empty((b, sq, h, uv_dim), device=dev, dtype=torch.bfloat16)
            self.uv_args = (p(self.w), uv_dim * 512, p(self.out_v))

    def full(self, stream):
        """One whole call as ``dsa_amd.forward`` enqueues it: for 256 tokens
        or more the row bucketing of the indices, then dsa_fwd (or dsa_fwd_opts)
        -- the main kernel and its merge in one C call -- or, with the W_UV
        projection, the main kernel and the merge + W_UV launch."""
        b, sq, h, length, k = self.shape
        if self.bucket:
            rc = self.lib.dsa_bucket_indices(ctypes.c_void_p(self.data[4].data_ptr()), self.args[4], b * sq, k,
                                             length, stream)
            if rc:
                _lib.check(rc, "dsa_bucket_indices")
        if self.uv:
            self.main(stream)
            self.merge(stream)
            return
        if self.opts is None:
            rc = self.lib.dsa_fwd(*self.args, b, sq, h, length, k, ctypes.byref(self.plan), stream)
        else:
            rc = self.lib.dsa_fwd_opts(*self.args, b, sq, h, length, k, ctypes.byref(self.opts),
                                       ctypes.byref(self.plan), stream)
        if rc:
            _lib.check(rc, "dsa_fwd")

    def main(self, stream):
        b, sq, h, length, k = self.shape
        if self.fused:
            rc = self.lib.dsa_fwd_opts(*self.args, b, sq, h, length, k, ctypes.byref(self.opts),
                                       ctypes.byref(self.plan), stream)
        elif self.opts is None:
            rc = self.lib.dsa_fwd_main(*self.args, b, sq, h, length, k, ctypes.byref(self.plan), stream)
        else:
            rc = self.lib.dsa_fwd_main_opts(*self.args, b, sq, h, length, k, ctypes.byref(self.opts),
                                            ctypes.byref(self.plan), stream)
        if rc:
            _lib.check(rc, "dsa_fwd_main")

    def merge(self, stream):
        b, sq, h, _, _ = self.shape
        if self.uv:  # the second launch: merge + W_UV, or W_UV of the bf16 output
            w, stride, out_v = self.uv_args
            if self.po is not None and not self.fused:
                rc = self.lib.dsa_merge_uv(self.args[8], self.args[9], self.args[10], w, stride, out_v,
                                           self.args[6], self.args[7], b * sq, h, self.config.split, self.uv,
                                           stream)
            else:
                rc = self.lib.dsa_project_uv(self.args[5], w, stride, out_v, b * sq, h, self.uv, stream)
            if rc:
                _lib.check(rc, "dsa_merge_uv / dsa_project_uv")
            return
        if self.po is None or self.fused:
            return
        rc = self.lib.dsa_merge(self.args[8], self.args[9], self.args[10], self.args[5], self.args[6],
                                self.args[7], b * sq, h, self.config.split, stream)
        if rc:
            _lib.check(rc, "dsa_merge")


class Rotation:
    """Input sets taken in one continuous cyclic order across the warm-up and
    every timed batch, so a set comes round again only after all the others
    (len(calls) - 1 calls later), whatever K and W are."""

    def __init__(self, calls):
        self.calls, self.next = calls, 0

    def take(self):
        call = self.calls[self.next % len(self.calls)]
        self.next += 1
        return call


def _batch_us(rot, steps, stream_obj, work):
    """Device time per call of ``steps`` back-to-back launches between two
    HIP events on the launch stream (no event inside the batch, so the
    per-event cost of a few microseconds is not charged to every call)."""
    stream = ctypes.c_void_p(stream_obj.cuda_stream)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream_obj)
    for _ in range(steps):
        work(rot.take(), stream)
    e1.record(stream_obj)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / steps


def time_rounds(calls, steps, warmup, rounds=1):
    """W untimed warm-up calls, then R rounds, each of exactly K calls
    (main kernel + merge) back to back between two HIP events with device
    synchronisation on both sides, followed by K main-kernel launches alone
    and K merges alone timed the same way (the rounds interleave the three,
    as the reference's review interleaves its samples).  Returns per-call
    device µs lists ``span``, ``main``, ``merge`` (one entry per round) and
    ``wall``, the host seconds of each round's K calls.  The main kernel's
    launches give its average duration, the roofline's denominator.  All of
    it walks one continuous rotation over the input sets (``Rotation``): the
    warm-up does not leave the first timed sets in the cache."""
    stream_obj = torch.cuda.current_stream()
    stream = ctypes.c_void_p(stream_obj.cuda_stream)
    rot = Rotation(calls)

    def both(c, s):  # one whole call
        if hasattr(c, "full"):
            c.full(s)
        else:
            c.main(s)
            c.merge(s)
    for _ in range(warmup):
        both(rot.take(), stream)
    torch.cuda.synchronize()
    out = {"span": [], "main": [], "merge": [], "wall": []}
    for _ in range(rounds):
        t0 = time.perf_counter()
        out["span"].append(_batch_us(rot, steps, stream_obj, both))
        out["wall"].append(time.perf_counter() - t0)
        out["main"].append(_batch_us(rot, steps, stream_obj, lambda c, s: c.main(s)))
        out["merge"].append(_batch_us(rot, steps, stream_obj, lambda c, s: c.merge(s)))
    return out


def time_calls(calls, steps, warmup):
    """One round of ``time_rounds``: (host wall seconds of the K calls, main
    µs, merge µs, span µs) per call."""
    t = time_rounds(calls, steps, warmup, 1)
    return t["wall"][0], t["main"][0], t["merge"][0], t["span"][0]


def spread(values):
    """Median, min and max of one quantity over the rounds."""
    return statistics.median(values), min(values), max(values)


def cpu_model():
    """The host CPU's model name, for the baseline record: ``lscpu``'s "Model
    name" (with its vendor), else /proc/cpuinfo's "model name"."""
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        fields = dict(ln.split(":", 1) for ln in out.splitlines() if ":" in ln)
        name = fields.get("Model name", "").strip()
        vendor = fields.get("Vendor ID", "").strip()
        if name:
            return f"{name} ({vendor})" if vendor and vendor not in name else name
    except (OSError, subprocess.SubprocessError, ValueError):
        pass
    try:
        for ln in Path("/proc/cpuinfo").read_text().splitlines():
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


# Thread and CPU counts of the CPU baseline, filled in by main().
CPU_COUNTS = {}


def cpu_threads():
    """Threads for the CPU baseline: every CPU this process may run on
    (``os.sched_getaffinity``), capped by OMP_NUM_THREADS when the host sets
    it (the GPU box gives each GPU a 16-CPU share and says so there), and the
    counts it was derived from."""
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS", "")
    threads = min(avail, int(omp)) if omp.isdigit() and int(omp) > 0 else avail
    return threads, {"os_cpu_count": os.cpu_count(), "affinity_cpus": avail, "OMP_NUM_THREADS": omp or None}


def eager_us(data, config, samples=30):
    """Median wall clock of one dsa_amd.forward call (checks, output
    allocation, launches) followed by a device synchronisation, called as a
    caller would: without ``config`` when the plan is the shape's default
    (which lets a repeated shape take forward's C++ fast path)."""
    q, kv, qr, kr, ids = data
    shape = tuple(q.shape[:3]) + (kv.shape[1], ids.shape[-1])
    kw = {} if config == dsa_amd.select(shape) else {"config": config}
    for _ in range(3):
        dsa_amd.forward(q, kv, qr, kr, ids, **kw)
    torch.cuda.synchronize()
    times = []
    for _ in range(samples):
        t0 = time.perf_counter()
        dsa_amd.forward(q, kv, qr, kr, ids, **kw)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    return statistics.median(times) * 1e6


def cpu_baseline(name, data, samples=None):
    """The CPU oracle on full calls of the workload: one warm-up call, then
    the median of 5 calls (C1-C3) or 3 calls (C4, C5), as the reference's
    baseline protocol asks; the inputs are on the host beforehand."""
    from oracle import dsa_oracle as oracle

    fp8 = data[3] is None  # kv holds fp8 rows: the oracle runs on their dequantized values
    if fp8:
        kv, kr = oracle.dequant_fp8_rows(data[1])
        q, qr, ids = (t.cpu() for t in (data[0], data[2], data[4]))
    else:
        q, kv, qr, kr, ids = (t.cpu() for t in data)
    if samples is None:
        samples = 3 if q.shape[1] >= 1024 else 5
    oracle.reference(q, kv, qr, kr, ids)  # warm-up
    times = []
    for _ in range(samples):
        t0 = time.perf_counter()
        oracle.reference(q, kv, qr, kr, ids)
        times.append(time.perf_counter() - t0)
    per_call_us = statistics.median(times) * 1e6
    return {"value": round(per_call_us, 1), "unit": "µs/call", "cores": torch.get_num_threads(),
            "kind": "port", "cpu": cpu_model(), **CPU_COUNTS,
            "min_us": round(min(times) * 1e6, 1), "max_us": round(max(times) * 1e6, 1),
            "sample": (f"full call: FP32 torch gather+softmax oracle over all {q.shape[0] * q.shape[1]} tokens of "
                       f"one {name} call, one warm-up call then the median of {samples}; inputs already on the "
                       f"host (generation and copies not timed)"
                       + ("; kv dequantized from the fp8 rows beforehand (not timed)" if fp8 else ""))}


def traffic_from_profiles(name):
    """(HBM bytes per main-kernel launch measured by rocprofv3 --pmc, the
    commit the profiled build came from), if a summary for this workload is
    committed under profiles/."""
    path = ROOT / "profiles" / f"sparse_mla_fwd_{name}_hbm_traffic.json"
    if not path.exists():
        return None, None
    rec = json.loads(path.read_text())
    return rec.get("hbm_bytes_per_launch"), rec.get("commit")


def paged(data, block_size, seed):
    """The same logical inputs with kv / k_rope moved into block pools under a
    random block permutation: (data with pools, block table)."""
    q, kv, qr, kr, ids = data
    batch, length = kv.shape[:2]
    if length % block_size:
        raise SystemExit(f"--paged {block_size} must divide L={length}")
    per = length // block_size
    g = torch.Generator(device=kv.device).manual_seed(seed)
    perm = torch.randperm(batch * per, device=kv.device, generator=g)
    kv_pool = torch.empty((batch * per, block_size, 1, 512), device=kv.device, dtype=kv.dtype)
    kr_pool = torch.empty((batch * per, block_size, 1, 64), device=kv.device, dtype=kv.dtype)
    kv_pool[perm] = kv.view(batch * per, block_size, 1, 512)
    kr_pool[perm] = kr.view(batch * per, block_size, 1, 64)
    return (q, kv_pool, qr, kr_pool, ids), perm.view(batch, per).int().contiguous()


def plan_text(config):
    """A plan as one string (a JSON record keeps it where nested objects are
    dropped)."""
    return (f"bm={config.bm} bn={config.bn} split={config.split} kv_waves={config.kv_waves} "
            f"stages={config.stages} mfma={config.mfma} pv_cols={config.pv_cols} "
            f"fused_merge={int(config.fused_merge)}")


def fixed_chain_us(calls, config, args):
    """The same plan on the same input sets with only TOPK = split x tile_rows
    slots per token (one tile per workgroup): the per-call cost that does not
    scale with the gathered rows (launches, the cold index and first-tile
    round trips, the partial stores and the merge).  Median span over the
    rounds."""
    slots = config.split * config.bn
    short = []
    for c in calls:
        q, kv, qr, kr, ids = c.data
        short.append(Call((q, kv, qr, kr, ids[..., :slots].contiguous()), config))
    t = time_rounds(short, args.steps, args.warmup, args.rounds)
    return statistics.median(t["span"]), slots


def run(name, args, overrides=True):
    """One workload's line.  ``overrides=False`` ignores --plan and --rotate
    (the legs that follow the headline line use their own defaults)."""
    shape = BASELINE_CONFIGS[name]
    rotate = args.rotate if args.rotate and overrides else DEFAULT_ROTATE[name]
    config = dsa_amd.select(shape, kv_fp8=args.fp8)
    if args.plan and overrides:
        v = [int(x) for x in args.plan.split(",")]
        bm, split, kv_waves, mfma = v[:4]
        bn, stages = (v[4], v[5]) if len(v) > 4 else (64, 2)
        fused = bool(v[6]) if len(v) > 6 else False
        pv_cols = v[7] if len(v) > 7 else 512
        config = Tuning(bm, bn, split, kv_waves=kv_waves, stages=stages, mfma=mfma, fused_merge=fused,
                        pv_cols=pv_cols)
    print(f"[bench] {name} shape={shape} plan={config} rotate={rotate}", file=sys.stderr, flush=True)
    sets = [baseline_inputs(name, seed=args.seed + i, device="cuda", cpu_recipe=False) for i in range(rotate)]
    if args.fp8:  # the same inputs with kv and k_rope written as 656-byte fp8 rows
        for i, d in enumerate(sets):
            sets[i] = (d[0], dsa_amd.quantize_kv_fp8(d[1], d[3]), d[2], None, d[4])
        torch.cuda.synchronize()
    if args.paged:
        calls = []
        for i, d in enumerate(sets):
            pd, table = paged(d, args.paged, args.seed + i)
            calls.append(Call(pd, config, block_table=table, uv_dim=args.uv))
            if i:  # set 0 stays for the CPU baseline
                sets[i] = None
    else:
        calls = [Call(d, config, fp8=args.fp8, uv_dim=args.uv) for d in sets]
    t = time_rounds(calls, args.steps, args.warmup, args.rounds)
    span_us, span_min, span_max = spread(t["span"])
    main_us, main_min, main_max = spread(t["main"])
    merge_us = statistics.median(t["merge"])
    wall = statistics.median(t["wall"])
    warm = time_rounds(calls[:1], args.steps, args.warmup, args.rounds)
    warm_span, warm_main = statistics.median(warm["span"]), statistics.median(warm["main"])
    gbytes, flops = algorithmic_units(shape, args.fp8)
    bound = BOUND[name]
    if bound == "hbm":
        achieved, peak, unit = gbytes / (main_us * 1e-6) / 1e9, HBM_PEAK_GBS, "GB/s"
        achieved_span = gbytes / (span_us * 1e-6) / 1e9
    else:
        achieved, peak, unit = flops / (main_us * 1e-6) / 1e12, MFMA_PEAK_TFLOPS, "TFLOP/s"
        achieved_span = flops / (span_us * 1e-6) / 1e12
    traffic, traffic_commit = traffic_from_profiles(name) if not (args.paged or args.fp8) else (None, None)
    line = {
        "metric": METRIC,
        "value": round(span_us, 3),
        "unit": "µs/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": (round(span_us / PUBLISHED_SPAN_US[name], 4) if name in PUBLISHED_SPAN_US else None),
        "dtype": "bf16",
        "data": (f"synthetic: seeded N(0,1) bf16 q/kv/rope, per-workload index recipe, "
                 f"{rotate} rotating input set(s) resident in HBM"
                 + (f"; kv paged in {args.paged}-row blocks under a random block table" if args.paged else "")
                 + ("; kv cache as 656-byte fp8 rows (e4m3 latent, fp32 block scales, bf16 rope)"
                    if args.fp8 else "")),
        "config": {"workload": name, "B": shape[0], "SQ": shape[1], "H": shape[2], "L": shape[3],
                   "TOPK": shape[4], "plan": plan_text(config), "rounds": args.rounds,
                   "rotating_input_sets": rotate, "paged_block_size": args.paged or None,
                   "kv_format": "fp8" if args.fp8 else "bf16"},
        "roofline": {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
                     "frac": round(achieved / peak, 4), "traffic": traffic,
                     "achieved_span": round(achieved_span, 2), "frac_span": round(achieved_span / peak, 4),
                     "kernel": (f"sparse_mla_fwd (main), {gbytes} gathered B and {flops} FLOP per launch; "
                                f"frac on the main kernel's average launch, frac_span on the whole call "
                                f"(split merge included); medians of {args.rounds} rounds"),
                     "traffic_source": (f"profiles/sparse_mla_fwd_{name}_hbm_traffic.json (build of commit "
                                        f"{traffic_commit})" if traffic is not None else None)},
        **({"dtype_note": "kv stored as fp8 e4m3 rows; MFMA inputs bf16"} if args.fp8 else {}),
        "breakdown": {
            "span_us": round(span_us, 3),
            "span_min_us": round(span_min, 3),
            "span_max_us": round(span_max, 3),
            "main_us": round(main_us, 3),
            "main_min_us": round(main_min, 3),
            "main_max_us": round(main_max, 3),
            "merge_us": round(merge_us, 3),
            "kernel_sum_us": round(main_us + merge_us, 3),
            "warm_span_us": round(warm_span, 3),
            "warm_main_us": round(warm_main, 3),
            "eager_call_us": round(eager_us(sets[0], config), 2) if not args.paged and not args.fp8 else None,
            "gathered_TBps_main": round(gbytes / (main_us * 1e-6) / 1e12, 3),
            "mfma_TFLOPs_main": round(flops / (main_us * 1e-6) / 1e12, 2),
            "gathered_TBps_span": round(gbytes / (span_us * 1e-6) / 1e12, 3),
            "mfma_TFLOPs_span": round(flops / (span_us * 1e-6) / 1e12, 2),
        },
    }
    if bound == "hbm" and config.split > 1 and not (args.paged or args.fp8 or args.uv or args.no_chain):
        chain, slots = fixed_chain_us(calls, config, args)
        line["breakdown"]["fixed_chain_us"] = round(chain, 3)
        line["breakdown"]["fixed_chain_topk"] = slots
    if args.uv:
        line["w_uv"] = uv_line(shape, config, args.uv, merge_us)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(name, sets[0])
    return line


def leg(prefix, line):
    """A workload's line as flat scalar fields named ``<prefix>_...``, for the
    headline line's ``decode`` and ``prefill`` objects."""
    r, b, c = line["roofline"], line["breakdown"], line.get("cpu_baseline") or {}
    out = {"span_us": line["value"], "span_min_us": b["span_min_us"], "span_max_us": b["span_max_us"],
           "main_us": b["main_us"], "merge_us": b["merge_us"], "bound": r["bound"], "achieved": r["achieved"],
           "unit": r["unit"], "frac": r["frac"], "frac_span": r["frac_span"], "traffic": r["traffic"],
           "plan": line["config"]["plan"], "rotating_input_sets": line["config"]["rotating_input_sets"],
           "cpu_us": c.get("value"), "cpu_sample": c.get("sample")}
    if "fixed_chain_us" in b:
        out["fixed_chain_us"] = b["fixed_chain_us"]
    return {f"{prefix}_{k}": v for k, v in out.items()}


def run_case(name, args):
    """One of the reference's 16 cases at full size with the selected plan:
    span, main and merge per call (timed as the workloads are), beside the
    reference's published Ascend950PR span for the same case.  Input sets
    (the review recipe's distribution, drawn on the device) are cycled until
    their gathered rows exceed twice the 256 MB MALL, at most 32; the number
    of timed calls is cut so that each timing takes about two seconds."""
    shape = dsa_amd.CASE_SHAPES[name]
    b, sq, h, length, k = shape
    config = dsa_amd.select(shape)
    rows_bytes = b * sq * k * 1152
    rotate = max(1, min(32, -(-(512 << 20) // rows_bytes)))
    if rotate * (b * length * 1152 + b * sq * h * 1152) > (32 << 30):  # big cases: one set
        rotate = 1
    sets = [case_inputs(shape, seed=args.seed + i) for i in range(rotate)]
    calls = [Call(d, config) for d in sets]
    once = time_calls(calls, 1, 1)[3]
    steps = max(3, min(args.steps, int(2e6 / max(once, 1.0))))
    warmup = max(1, min(args.warmup, steps))
    _, main_us, merge_us, span_us = time_calls(calls, steps, warmup)
    ref = REF_CASE_SPAN_US[name]
    return {"case": name, "B": b, "SQ": sq, "H": h, "L": length, "TOPK": k, "plan": vars(config),
            "span_us": round(span_us, 3), "main_us": round(main_us, 3), "merge_us": round(merge_us, 3),
            "steps": steps, "warmup": warmup, "rotating_input_sets": rotate,
            "reference_ascend950pr_span_us": ref, "span_vs_reference": round(span_us / ref, 4),
            "data": "synthetic: seeded N(0,1) bf16 q/kv/rope, distinct uniform indices per token"}


def uv_line(shape, config, dv, uv_us):
    """The W_UV launch of a call (the merge_us slot of the breakdown):
    algorithmic HBM bytes = the weights once, the latent input (bf16 output,
    or the FP32 split partials with their max and sum when the merge is in
    the same launch), the bf16 result (and max and sum); all HBM-bound."""
    b, sq, h, _, _ = shape
    tokens = b * sq
    merged = config.split > 1
    weights = h * dv * 512 * 2
    latent = tokens * config.split * h * (512 + 2) * 4 if merged else tokens * h * 512 * 2
    out = tokens * h * dv * 2 + (tokens * h * 8 if merged else 0)
    nbytes = weights + latent + out
    gbps = nbytes / (uv_us * 1e-6) / 1e9
    return {"kernel": "merge_uv" if merged else "project_uv", "dv": dv, "us": round(uv_us, 3),
            "bytes": nbytes, "weight_bytes": weights, "GBps": round(gbps, 1),
            "frac_hbm": round(gbps / HBM_PEAK_GBS, 4), "flops": 2 * tokens * h * dv * 512}


# ---------------------------------------------------------------- indexer
# Input sets cycled per indexer workload: decode_b8's keys (64 MiB a set) are
# rotated over 512 MiB, twice the MALL; the MTP case reads 1 GiB of keys a call.
INDEXER_ROTATE = {"idx_decode_b8": 8, "idx_decode_mtp_b64": 1, "idx_prefill_4k": 1}
INDEXER_BOUND = {"idx_decode_b8": "hbm", "idx_decode_mtp_b64": "hbm", "idx_prefill_4k": "mfma"}


def indexer_units(name, lengths):
    """Algorithmic bytes and FLOPs of one logits launch: every key read once
    (B*L rows of 128 bf16), queries and weights read once, every defined
    logit written once (4 B); 2*HI*128 MFMA FLOPs per defined (query, key)."""
    b, sq, hi, length, _, _ = INDEXER_CONFIGS[name]
    pairs = int(lengths.clamp(0, length).sum())
    nbytes = b * length * 128 * 2 + b * sq * hi * (128 * 2 + 4) + pairs * 4
    return nbytes, 2 * hi * 128 * pairs


class IndexerCall:
    """One preallocated indexer call (logits + top-k) through the C ABI."""

    def __init__(self, data, topk):
        self.data = data
        q, k, w, lengths = data
        self.shape = (q.shape[0], q.shape[1], q.shape[2], k.shape[1], topk)
        self.logits = torch.empty((q.shape[0], q.shape[1], k.shape[1]), device=q.device, dtype=torch.float32)
        self.indices = torch.empty((q.shape[0], q.shape[1], 1, topk), device=q.device, dtype=torch.int32)
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        self.largs = [p(q), p(k), p(w), p(lengths), p(self.logits)]
        self.targs = [p(self.logits), p(lengths), p(self.indices)]
        self.lib = _lib.load()
        # few rows: the segmented selection (8 workgroups per row) over a workspace
        self.ws_bytes = self.lib.dsa_indexer_topk_ws_bytes(q.shape[0], q.shape[1], k.shape[1], topk)
        self.ws = torch.empty(max(self.ws_bytes, 1), device=q.device, dtype=torch.uint8)

    def main(self, stream):
        b, sq, hi, length, _ = self.shape
        rc = self.lib.dsa_indexer_logits(*self.largs, b, sq, hi, length, stream)
        if rc:
            _lib.check(rc, "dsa_indexer_logits")

    def merge(self, stream):  # the second step of a call: the selection
        b, sq, _, length, topk = self.shape
        if self.ws_bytes > 0:
            rc = self.lib.dsa_indexer_topk_ws(*self.targs, b, sq, length, topk, ctypes.c_void_p(self.ws.data_ptr()),
                                              self.ws_bytes, stream)
        else:
            rc = self.lib.dsa_indexer_topk(*self.targs, b, sq, length, topk, stream)
        if rc:
            _lib.check(rc, "dsa_indexer_topk")


def indexer_cpu_baseline(name, data, budget_s=10.0):
    """The CPU oracle (logits + selection) on an evenly spaced query sample,
    scaled by the sample's share of (query, key) pairs."""
    from oracle import dsa_oracle as oracle

    q, k, w, lengths = (t.cpu() for t in data)
    topk = INDEXER_CONFIGS[name][4]
    batch, queries = q.shape[:2]

    def run_rows(rows):
        for b, sl in rows:
            lg = oracle.indexer_logits_ref(q[b:b + 1, sl], k[b:b + 1], w[b:b + 1, sl], lengths[b:b + 1, sl])
            oracle.indexer_topk_ref(lg, lengths[b:b + 1, sl], topk)

    probe_t = time.perf_counter()
    run_rows([(0, slice(0, 1))])
    per_query = max(time.perf_counter() - probe_t, 1e-4)
    n = max(1, min(batch * queries, int(budget_s / 3 / per_query)))
    flat = list(range(0, batch * queries, max(1, batch * queries // n)))[:n]
    rows = [(i // queries, slice(i % queries, i % queries + 1)) for i in flat]
    pairs_all = float(lengths.clamp(0, k.shape[1]).sum())
    pairs_sample = float(sum(min(int(lengths[b, sl][0]), k.shape[1]) for b, sl in rows))
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 2:
        t0 = time.perf_counter()
        run_rows(rows)
        times.append(time.perf_counter() - t0)
        if len(times) >= 20:
            break
    per_call_us = statistics.median(times) * 1e6 * pairs_all / pairs_sample
    return {"value": round(per_call_us, 1), "unit": "µs/call", "cores": torch.get_num_threads(),
            "kind": "port", "cpu": cpu_model(), **CPU_COUNTS,
            "sample": (f"FP32 torch indexer logits + numpy top-k oracle on {len(rows)} of {batch * queries} "
                       f"queries of one {name} call, median of {len(times)} runs, scaled by (query, key) pairs")}


def run_indexer(name, args):
    b, sq, hi, length, topk, causal = INDEXER_CONFIGS[name]
    rotate = args.rotate if args.rotate else INDEXER_ROTATE[name]
    print(f"[bench] {name} B={b} SQ={sq} HI={hi} L={length} TOPK={topk} causal={causal} rotate={rotate}",
          file=sys.stderr, flush=True)
    sets = [indexer_inputs(name, seed=args.seed + i, device="cuda") for i in range(rotate)]
    calls = [IndexerCall(d, topk) for d in sets]
    wall, logits_us, topk_us, span_us = time_calls(calls, args.steps, args.warmup)
    _, warm_logits, _, warm_span = time_calls(calls[:1], args.steps, args.warmup)
    nbytes, flops = indexer_units(name, sets[0][3])
    bound = INDEXER_BOUND[name]
    if bound == "hbm":
        achieved, peak, unit = nbytes / (logits_us * 1e-6) / 1e9, HBM_PEAK_GBS, "GB/s"
    else:
        achieved, peak, unit = flops / (logits_us * 1e-6) / 1e12, MFMA_PEAK_TFLOPS, "TFLOP/s"
    traffic = ROOT / "profiles" / f"indexer_logits_{name}_hbm_traffic.json"
    line = {
        "metric": "lightning indexer span (index logits + top-k selection)",
        "value": round(span_us, 3),
        "unit": "µs/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": (f"synthetic: seeded N(0,1) bf16 index queries/keys, N(0,0.01) fp32 head weights, "
                 f"{'causal' if causal else 'decode'} lengths, {rotate} rotating input set(s) resident in HBM"),
        "config": {"workload": name, "B": b, "SQ": sq, "HI": hi, "L": length, "TOPK": topk,
                   "rotating_input_sets": rotate},
        "roofline": {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
                     "frac": round(achieved / peak, 4),
                     "traffic": (json.loads(traffic.read_text()).get("hbm_bytes_per_launch")
                                 if traffic.exists() else None),
                     "kernel": f"indexer_logits, {nbytes} algorithmic B and {flops} FLOP per launch"},
        "breakdown": {
            "span_us": round(span_us, 3),
            "logits_us": round(logits_us, 3),
            "topk_us": round(topk_us, 3),
            "warm_span_us": round(warm_span, 3),
            "warm_logits_us": round(warm_logits, 3),
            "logits_TBps": round(nbytes / (logits_us * 1e-6) / 1e12, 3),
            "logits_TFLOPs": round(flops / (logits_us * 1e-6) / 1e12, 2),
        },
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = indexer_cpu_baseline(name, sets[0], args.cpu_budget)
    return line


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c2_decode_b8", choices=sorted(BASELINE_CONFIGS))
    ap.add_argument("--all", action="store_true", help="one line per configuration C2..C5")
    ap.add_argument("--rotate", type=int, default=0, help="input sets to cycle (default per workload)")
    ap.add_argument("--plan", default="",
                    help="override the plan: bm,split,kv_waves,mfma[,bn,stages[,fused[,pv_cols]]]")
    ap.add_argument("--seed", type=int, default=20261102)
    ap.add_argument("--paged", type=int, default=0, metavar="BLOCK",
                    help="run the workload on paged kv (block pools of BLOCK rows, random block table)")
    ap.add_argument("--fp8", action="store_true",
                    help="run the workload on the fp8 kv row format (656 bytes per row)")
    ap.add_argument("--indexer", default="", metavar="WORKLOAD",
                    help="time the lightning indexer instead: " + ", ".join(INDEXER_CONFIGS) + " or all")
    ap.add_argument("--uv", type=int, default=0, metavar="DV",
                    help="append the W_UV output projection (value head dim DV, e.g. 128) to every call")
    ap.add_argument("--cases", default="", metavar="NAMES",
                    help="time the reference's 16 cases instead (comma list or all): one line each")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--rounds", type=int, default=5, help="timed rounds of K calls (median, min, max reported)")
    ap.add_argument("--no-chain", action="store_true",
                    help="leave out breakdown.fixed_chain_us (its launches are the same kernel: kernel traces)")
    ap.add_argument("--no-legs", action="store_true",
                    help="C2 line only (by default it carries C3, C5 and C4 legs)")
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of indexer CPU oracle timing")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run 5 device copies of MIB MiB (reference kernel for rocprofv3 byte counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each GPU box has one "
              "MI355X); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    torch.cuda.init()
    if args.calibrate_copy:
        n = args.calibrate_copy * 1024 * 1024 // 4
        src = torch.randn(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration_copy_bytes": n * 4, "copies": 5}))
        return
    if args.indexer:
        for name in list(INDEXER_CONFIGS) if args.indexer == "all" else [args.indexer]:
            if name not in INDEXER_CONFIGS:
                raise SystemExit(f"unknown indexer workload {name!r}")
            print(json.dumps(run_indexer(name, args), ensure_ascii=False), flush=True)
        return
    if args.cases:
        for name in list(REF_CASES) if args.cases == "all" else args.cases.split(","):
            if name not in REF_CASE_SPAN_US:
                raise SystemExit(f"unknown reference case {name!r}")
            print(json.dumps(run_case(name, args), ensure_ascii=False), flush=True)
            torch.cuda.empty_cache()
        return
    threads, counts = cpu_threads()
    torch.set_num_threads(threads)
    CPU_COUNTS.update(threads_used=threads, **counts)
    names = ["c2_decode_b8", "c3_decode_h16_mtp", "c4_prefill_h16", "c5_prefill_h128"] if args.all else [args.config]
    for name in names:
        line = run(name, args)
        if not args.all and not args.no_legs and name == "c2_decode_b8":
            # The metric is "decode B=8 + prefill": the headline line carries
            # the other GPU configurations as flat legs timed the same way:
            # C3 (16-head MTP decode, HBM-bound) in ``decode``, C5 (the
            # MFMA-bound prefill) and C4 (16 heads, L2/MALL-bound) in
            # ``prefill``; their roofline fractions also go into ``roofline``.
            legs = {p: run(p, args, overrides=False)
                    for p in ("c3_decode_h16_mtp", "c5_prefill_h128", "c4_prefill_h16")}
            line["decode"] = {**leg("c3", legs["c3_decode_h16_mtp"]),
                              "c2_span_min_us": line["breakdown"]["span_min_us"],
                              "c2_span_max_us": line["breakdown"]["span_max_us"],
                              "c2_fixed_chain_us": line["breakdown"].get("fixed_chain_us")}
            line["prefill"] = {**leg("c5", legs["c5_prefill_h128"]), **leg("c4", legs["c4_prefill_h16"])}
            for p, l in (("c3", legs["c3_decode_h16_mtp"]), ("c5", legs["c5_prefill_h128"]),
                         ("c4", legs["c4_prefill_h16"])):
                line["roofline"][f"{p}_frac"] = l["roofline"]["frac"]
                line["roofline"][f"{p}_frac_span"] = l["roofline"]["frac_span"]
                if "cpu_baseline" in line and "cpu_baseline" in l:
                    line["cpu_baseline"][f"{p}_value"] = l["cpu_baseline"]["value"]
        print(json.dumps(line, ensure_ascii=False), flush=True)


if __name__ == "__main__":
    main()
