"""Host entry point of the MI355X sparse-MLA forward.

Mirrors the reference's public operator ``dsa.forward`` (dsa/api.py:76-132):
same positional arguments, tensor contract, return triple and exception types,
with the device requirement moved from Ascend ("npu") to a ROCm GPU.  The work
is one main-kernel launch plus, when the plan splits the KV range, one FP32
merge -- a second launch, or, with a fused-merge plan, the main kernel's last
workgroup per (token, head group) -- enqueued through the C ABI on the
current stream.  There is no CPU or fallback path.
"""
from __future__ import annotations

import ctypes
import threading
from dataclasses import dataclass

import torch

from . import _lib
from .config import Tuning, check_tuning, select

HEAD_DIM = 512
ROPE_DIM = 64
FP8_ROW = 656  # bytes of an fp8 kv row: 512 e4m3 latent values, 4 fp32 scales, 64 bf16 rope values
SCALE = 1.0 / 24.0  # 576 ** -0.5, the reference's fixed scale (README.md:81-83 of the reference)
_LDS_BYTES = 2 * 64 * 1152 + 2048 * 4
_PP_LDS_BYTES = 4 * 32 * 1152 + 2048 * 4 + 2 * 64 * 64  # ring, index cache, two P buffers


def _xp_lds_bytes(bm):
    # ring (two 64-row stages), index cache (halved for 64 heads), P of one
    # tile (144 bytes a head), per-wave maxima, vote flag (XpLds<bm / 16>)
    idx_cap = 2048 if bm <= 32 else 1024
    return 2 * 64 * 1152 + idx_cap * 4 + bm * 144 + 4 * bm * 4 + 16


def _xs_lds_bytes(bm):
    # ring, index cache, two P buffers, (l, reference max, max) per head, vote flag
    return 4 * 32 * 1152 + 2048 * 4 + 2 * bm * 64 + 3 * bm * 4 + 16


@dataclass(frozen=True)
class Launch:
    """Descriptor of one kernel launch of a call (``return_kernels=True``)."""

    name: str
    grid: int
    block: int
    lds_bytes: int


def _check_inputs(q, kv, q_rope, k_rope, indices, block_table=None):
    """Shape, device, layout and dtype contract (reference: dsa/api.py:18-38).

    Checks run in the reference's order (shapes, then device/contiguity, then
    dtypes) and raise ValueError; index values are never read.  With a
    ``block_table`` (paged kv, no reference counterpart) kv and k_rope are
    block pools ``[num_blocks, block_size, 1, 512 / 64]``, ``block_table`` is
    int32 ``[B, max_blocks]`` and the logical length is
    ``L = max_blocks * block_size``.  A uint8 ``kv`` whose last dim is 656
    holds fp8 rows (no reference counterpart; ``k_rope`` must then be None).
    Returns ``(shape, device, fp8)``.
    """
    fp8 = kv.dtype == torch.uint8 and kv.dim() == 4 and kv.shape[-1] == FP8_ROW
    if fp8 and k_rope is not None:
        raise ValueError("with fp8 kv rows (uint8 [..., 656]) k_rope must be None: the rope values are in the rows")
    if not fp8 and k_rope is None:
        raise ValueError("k_rope is required unless kv holds fp8 rows (uint8 [..., 656])")
    q_shape, kv_shape, ids_shape = q.shape, kv.shape, indices.shape
    if len(q_shape) != 4 or len(kv_shape) != 4 or len(ids_shape) != 4:
        raise ValueError("q, kv and indices must be 4-D tensors")
    batch, queries, heads, width = q_shape
    topk = ids_shape[3]
    if block_table is None:
        length = kv_shape[1]
        pool = (batch, length)
    else:
        if block_table.dim() != 2 or block_table.shape[0] != batch:
            raise ValueError("block_table must be [B, max_blocks]")
        pool = (kv_shape[0], kv_shape[1])
        length = block_table.shape[1] * kv_shape[1]
    if (width != HEAD_DIM or kv_shape != (*pool, 1, FP8_ROW if fp8 else HEAD_DIM)
            or q_rope.shape != (batch, queries, heads, ROPE_DIM)
            or (not fp8 and k_rope.shape != (*pool, 1, ROPE_DIM))
            or ids_shape != (batch, queries, 1, topk)
            or min(batch, queries, heads, length, topk, *pool) <= 0):
        if fp8:
            raise ValueError("expected q[B,SQ,H,512], kv fp8 rows [B,L,1,656] (or a [N,BS,1,656] pool), "
                             "q_rope[B,SQ,H,64], indices[B,SQ,1,K]")
        if block_table is None:
            raise ValueError("expected q[B,SQ,H,512], kv[B,L,1,512], q_rope[B,SQ,H,64], "
                             "k_rope[B,L,1,64], indices[B,SQ,1,K]")
        raise ValueError("expected q[B,SQ,H,512], kv[N,BS,1,512], q_rope[B,SQ,H,64], "
                         "k_rope[N,BS,1,64], indices[B,SQ,1,K], block_table[B,M]")
    if heads % 16:
        raise ValueError(f"the number of heads must be a multiple of 16 (got {heads})")
    device = q.device
    if (device.type != "cuda" or torch.version.hip is None
            or kv.device != device or q_rope.device != device or indices.device != device
            or (not fp8 and k_rope.device != device)
            or (block_table is not None and block_table.device != device)
            or not (q.is_contiguous() and kv.is_contiguous() and q_rope.is_contiguous()
                    and indices.is_contiguous() and (fp8 or k_rope.is_contiguous())
                    and (block_table is None or block_table.is_contiguous()))):
        raise ValueError("all inputs must be contiguous and on the same ROCm GPU")
    bf16 = torch.bfloat16
    if (q.dtype != bf16 or (not fp8 and kv.dtype != bf16) or q_rope.dtype != bf16
            or (not fp8 and k_rope.dtype != bf16)
            or indices.dtype != torch.int32
            or (block_table is not None and block_table.dtype != torch.int32)):
        raise ValueError("q/kv/q_rope/k_rope must be bfloat16 and indices (and block_table) int32")
    return (batch, queries, heads, length, topk), device, fp8


def _check_scale(scale):
    if scale is None:
        return None
    if isinstance(scale, bool) or not isinstance(scale, (int, float)):
        raise TypeError("scale must be a float")
    scale = float(scale)
    if not (scale > 0.0 and scale < float("inf")):
        raise ValueError(f"scale must be a positive finite number (got {scale})")
    return scale


def _uv_launch(tokens: int, heads: int, dv: int, merge: bool) -> Launch:
    """Launch descriptor of the W_UV kernel (mirrors project_uv.hip:uv_shape)."""
    ndt = dv // 16

    def d_shape(wgs):
        nj = 2 if ndt % 8 == 0 and wgs * (ndt // 8) >= 256 else 1
        return ndt // (4 * nj)

    if merge:
        nchunk = (tokens + 15) // 16
        dsplit = d_shape(heads * nchunk)
        return Launch("merge_uv", heads * nchunk * dsplit, 256, 16 * 1024)
    tb = 32  # tokens per tile, four LDS buffers
    ntiles = (tokens + tb - 1) // tb
    dsplit = d_shape(heads * ntiles)
    want = ((256 + heads - 1) // heads + dsplit - 1) // dsplit
    per = (ntiles + want - 1) // want
    nchunk = (ntiles + per - 1) // per
    return Launch("project_uv", heads * nchunk * dsplit, 256, 4 * tb * 1024)


BUCKET_MIN_TOKENS = 256  # calls with this many tokens or more bucket each token's indices first
BUCKET_MAX_TOPK = 4096   # the row bucketing's limit (dsa_bucket_indices)


def buckets_rows(shape) -> bool:
    """Whether a call of this (B, SQ, H, L, TOPK) partitions each token's
    indices by kv row range before the main kernel (dsa_bucket_indices):
    prefill-sized calls, whose workgroups then gather from the same row
    ranges at the same time and share L2 lines.  Decode calls have too few
    workgroups per kv row to gain and skip the extra launch."""
    return shape[0] * shape[1] >= BUCKET_MIN_TOKENS and shape[4] <= BUCKET_MAX_TOPK


def bucket_lds_bytes(topk: int) -> int:
    """LDS of the bucketing kernel: 65 counts per 64-slot chunk, 65 bucket
    bases and the assembled row, 4 bytes each."""
    return 4 * (-(-topk // 64) * 65 + 65 + topk)


def plan_call(shape, config=None, cores: int = 256, kv_fp8: bool = False, w_uv_dim: int | None = None):
    """Plan of one call: (Tuning, partial-buffer shapes or None, launches).

    Pure host logic (reference: dsa/api.py:88-113); usable without a GPU.
    ``kv_fp8``: the call reads fp8 kv rows, which only the narrow variants
    (``mfma=16``) do.  ``w_uv_dim``: the value head dimension of a W_UV
    projection that follows (no reference counterpart): a split plan then
    merges and projects in one launch after the main kernel (its in-kernel
    merge, if any, is not used: the W_UV launch is there anyway), a plan
    without a split adds a projection launch.
    """
    if type(cores) is not int or cores <= 0:
        raise ValueError("cores must be a positive int")
    if config is None:
        config = select(shape, cores, kv_fp8)
    else:
        check_tuning(config, shape)
        if kv_fp8 and (config.mfma != 16 or config.pv_cols != 512):
            raise ValueError("fp8 kv rows need a narrow plan (mfma 16, pv_cols 512)")
    batch, queries, heads, _, _ = shape
    tokens = batch * queries
    if config.pv_cols == 128:
        variant = "pp" if config.bm == 128 else "xs" if config.bn == 32 else "xp"
    else:
        variant = "wide" if config.mfma == 32 else "narrow"
    threads, lds = (512, _PP_LDS_BYTES) if variant == "pp" else (256, _LDS_BYTES)
    if variant == "xp":
        lds = _xp_lds_bytes(config.bm)
        if config.bm == 16:
            threads = 512  # four compute waves and four gather waves
    if variant == "xs":  # QK waves (one per 16 heads), two PV waves, four gather waves
        threads, lds = 64 * (config.bm // 16 + 6), _xs_lds_bytes(config.bm)
    launches = [Launch(f"sparse_mla_fwd_{variant}_h{config.bm}_kw{config.kv_waves}_bn{config.bn}_s{config.stages}",
                       tokens * config.split * (heads // config.bm), threads, lds)]
    if buckets_rows(shape):
        launches.insert(0, Launch("bucket_rows", tokens, 256, bucket_lds_bytes(shape[4])))
    partials = None
    merged = False
    if config.split > 1:
        partials = ((batch, queries, config.split, heads, HEAD_DIM), (batch, queries, config.split, heads))
        if w_uv_dim is not None:
            launches.append(_uv_launch(tokens, heads, w_uv_dim, True))
            merged = True
        elif not config.fused_merge:
            launches.append(Launch("merge_partials", tokens * ((heads + 1) // 2), 256, 0))
    if w_uv_dim is not None and not merged:
        launches.append(_uv_launch(tokens, heads, w_uv_dim, False))
    return config, partials, tuple(launches)


# Arrival counters of the in-kernel merge, one zeroed int32 array per (device,
# stream).  Every call leaves its counters at zero once its kernel completes,
# so calls in stream order share one array; a call on another stream gets its
# own.  The arrays hold no inputs or results: only the counters' zeros persist.
# Hazards of the shared array (also stated in forward's docstring): a stream
# handle that is destroyed and handed out again while a fused kernel of the
# old stream still runs would share that kernel's counters; a kernel that does
# not complete (a device fault ends the process's GPU context anyway) leaves
# them non-zero.  Callers that want no shared state pass their own counters
# (forward's ``arrivals``).  Under stream capture every call gets fresh
# zero-filled counters from the graph's own pool, so each graph records and
# replays its own fill kernel and graphs never share counters.
_arrivals_lock = threading.Lock()
_arrivals = {}


def _arrival_counters(device, stream: int, count: int) -> torch.Tensor:
    if torch.cuda.is_current_stream_capturing():
        return torch.zeros(count, device=device, dtype=torch.int32)
    key = (device.index, stream)
    with _arrivals_lock:
        buf = _arrivals.get(key)
        if buf is None or buf.numel() < count:
            # zero-filled on this stream, so ordered before the kernel that uses it
            size = max(count, 2 * buf.numel() if buf is not None else 1024)
            buf = torch.zeros(size, device=device, dtype=torch.int32)
            _arrivals[key] = buf
        return buf


def _check_arrivals(arrivals, device):
    if arrivals is None:
        return
    if not isinstance(arrivals, torch.Tensor) or arrivals.dtype != torch.int32 or arrivals.dim() != 1:
        raise ValueError("arrivals must be a 1-D int32 tensor")
    if arrivals.device != device or not arrivals.is_contiguous():
        raise ValueError("arrivals must be contiguous and on the same ROCm GPU as the other inputs")


def _check_w_uv(w_uv, heads: int, device):
    """W_UV weights: bf16 ``[H, dv, 512]`` with unit strides in the last two
    dims and any head stride (a multiple of 8 elements, at least dv * 512).
    Returns ``(dv, head_stride)``."""
    if not isinstance(w_uv, torch.Tensor) or w_uv.dim() != 3 or w_uv.shape[0] != heads \
            or w_uv.shape[2] != HEAD_DIM:
        raise ValueError(f"w_uv must be [H={heads}, dv, 512]")
    dv = w_uv.shape[1]
    if dv < 64 or dv > 256 or dv % 64:
        raise ValueError(f"w_uv's dv must be a multiple of 64 in [64, 256] (got {dv})")
    if w_uv.dtype != torch.bfloat16:
        raise ValueError("w_uv must be bfloat16")
    if w_uv.device != device:
        raise ValueError("w_uv must be on the same ROCm GPU as the other inputs")
    s0, s1, s2 = w_uv.stride()
    if s2 != 1 or s1 != HEAD_DIM or (heads > 1 and (s0 < dv * HEAD_DIM or s0 % 8)) or w_uv.data_ptr() % 16:
        raise ValueError("w_uv needs rows of 512 contiguous elements, 16-byte aligned, and a head stride "
                         ">= dv * 512 that is a multiple of 8 (a slice of wkv_b's value rows qualifies)")
    return dv, (s0 if heads > 1 else dv * HEAD_DIM)


def _vp(t):
    return ctypes.c_void_p(t.data_ptr())


def project_uv(output, w_uv):
    """W_UV output projection of a latent attention output (no reference
    counterpart; DeepSeek-V3.2-Exp inference/model.py, MLA.forward absorb
    branch: ``einsum("bshc,hdc->bshd", x, wkv_b[:, -v_head_dim:])``).

    ``output [..., H, 512]`` bf16 (contiguous, e.g. :func:`forward`'s) and
    ``w_uv [H, dv, 512]`` bf16 (see :func:`forward`); returns bf16
    ``[..., H, dv]``: ``out[t, h, d] = sum_c output[t, h, c] * w_uv[h, d, c]``
    accumulated in fp32 and rounded once.
    """
    if output.dim() < 2 or output.shape[-1] != HEAD_DIM:
        raise ValueError("output must be [..., H, 512]")
    heads = output.shape[-2]
    device = output.device
    if device.type != "cuda" or torch.version.hip is None or not output.is_contiguous():
        raise ValueError("output must be contiguous on a ROCm GPU")
    if output.dtype != torch.bfloat16:
        raise ValueError("output must be bfloat16")
    dv, head_stride = _check_w_uv(w_uv, heads, device)
    tokens = output.numel() // (heads * HEAD_DIM)
    out_v = torch.empty((*output.shape[:-1], dv), device=device, dtype=torch.bfloat16)
    if tokens == 0:
        return out_v
    stream = torch.cuda.current_stream(device).cuda_stream
    with torch.cuda.device(device):
        rc = _lib.load().dsa_project_uv(_vp(output), _vp(w_uv), head_stride, _vp(out_v), tokens, heads, dv,
                                        ctypes.c_void_p(stream))
    _lib.check(rc, "dsa_project_uv")
    return out_v


def forward(q, kv, q_rope, k_rope, indices, *, config=None, cores=None, return_kernels=False,
            scale=None, block_table=None, w_uv=None, arrivals=None):
    """Sparse MLA attention over given top-k indices.

    Returns ``(output, softmax_max, softmax_sum)``: bf16 ``[B,SQ,H,512]`` and
    two fp32 ``[B,1,SQ,H]`` tensors (max and sum of exp(score - max), not LSE).
    The scale is 1/24 as in the reference unless ``scale`` is given.
    Duplicate indices keep their weight; indices outside ``[0, L)`` are masked;
    every query needs at least one valid index.

    ``config``: a :class:`dsa_amd.Tuning` (default: the shape's table entry or
    the library planner).  ``cores``: CU budget for planning (default: the
    device's CU count).  ``return_kernels=True`` also returns the launch
    descriptors.  Outputs are fresh tensors; no input or result is kept across
    calls (only the plan of each shape, and the arrival counters below), and
    the call does not synchronise.

    Calls of 256 tokens or more (TOPK up to 4096) first partition each
    token's indices by kv row range into a fresh buffer
    (``dsa_bucket_indices``, :func:`bucket_indices`; the caller's tensor is
    not touched): the attention does not depend on the slots' order, and
    with every token's tiles drawn from the same row ranges the workgroups
    share L2 lines.

    Beyond the reference: ``scale`` (positive float) replaces the fixed 1/24,
    and ``block_table`` (int32 ``[B, max_blocks]``) selects paged kv, with kv
    and k_rope given as block pools ``[num_blocks, block_size, 1, 512 / 64]``;
    logical row ``I`` of batch ``b`` is pool row
    ``block_table[b, I // block_size] * block_size + I % block_size`` and a
    slot whose block entry is outside ``[0, num_blocks)`` is masked.  An fp8
    kv cache is a uint8 ``kv [B, L, 1, 656]`` (or pool) of rows written by
    :func:`dsa_amd.quantize_kv_fp8`, with ``k_rope=None``; the kernel computes
    with ``bf16(fp32(e4m3) * scale)`` latent values.

    ``w_uv`` (bf16 ``[H, dv, 512]``, dv a multiple of 64 up to 256; heads may
    be any stride apart, so ``wkv_b.view(H, d_nope + dv, 512)[:, -dv:]`` goes
    in as it is) appends the W_UV output projection: the first result is then
    bf16 ``[B,SQ,H,dv]`` = :func:`project_uv` of the latent output, bit for
    bit.  With a split plan the merge runs in the W_UV launch (also for a
    fused-merge plan: the main kernel then leaves its partials), and the
    latent output is never written.

    ``arrivals`` (int32 ``[n]``, n >= B*SQ*H/heads_per_group, zero before its
    first use) are the caller's own arrival counters for a fused-merge plan
    (the last workgroup of each (token, head group) merges the split
    partials inside the main kernel; every call leaves the counters zero
    again once its kernel completes, so one tensor serves calls in stream
    order, and calls that may overlap need tensors of their own).  Without
    it, calls share one counter array per (device, stream), and a captured
    call gets counters of its own in the graph's pool.  Ignored by plans that
    do not fuse the merge.
    """
    if (config is None and cores is None and not return_kernels and scale is None and block_table is None
            and w_uv is None and arrivals is None):
        fast = _fast_path()
        if fast is not None:  # a planned shape: checks, outputs and launch in C++ (None: not taken)
            r = fast.forward(q, kv, q_rope, k_rope, indices)
            if r is not None:
                if type(r) is int:
                    _lib.check(r, "dsa_fwd")
                return r
    scale = _check_scale(scale)
    shape, device, fp8 = _check_inputs(q, kv, q_rope, k_rope, indices, block_table)
    batch, queries, heads, length, topk = shape
    uv = None if w_uv is None else _check_w_uv(w_uv, heads, device)
    _check_arrivals(arrivals, device)
    if cores is None:
        cores = _device_cus(device)
    default_plan = config is None
    config, partials, launches, plan, fused, groups = _call_plan(shape, config, cores, fp8,
                                                                 None if uv is None else uv[0])
    if fused and arrivals is not None and arrivals.numel() < groups:
        raise ValueError(f"arrivals holds {arrivals.numel()} counters; this call needs {groups}")
    bucket = buckets_rows(shape)
    if (default_plan and cores == _device_cus(device) and not fused and not fp8 and scale is None
            and block_table is None and uv is None and not bucket):
        _register_fast(device, shape, plan, partials)

    output = torch.empty_like(q)
    maximum = torch.empty((batch, 1, queries, heads), device=device, dtype=torch.float32)
    denominator = torch.empty_like(maximum)
    if partials is None:
        part_o = part_m = part_l = None
    else:
        # One buffer carved into part_o, part_m, part_l (each 256-byte aligned):
        # only their addresses leave this function.
        part_buf = torch.empty(partials[2], device=device, dtype=torch.float32)
        part_o = part_buf.data_ptr()
        part_m = part_o + partials[3]
        part_l = part_o + partials[4]

    stream = torch._C._cuda_getCurrentRawStream(device.index)
    lib = _lib.load()
    idx_ptr = indices.data_ptr()
    if bucket:
        order = torch.empty_like(indices)
        with _on_device(device):
            rc = lib.dsa_bucket_indices(idx_ptr, order.data_ptr(), batch * queries, topk, length, stream)
        if rc:
            _lib.check(rc, "dsa_bucket_indices")
        idx_ptr = order.data_ptr()
    args = (q.data_ptr(), kv.data_ptr(), q_rope.data_ptr(), None if k_rope is None else k_rope.data_ptr(),
            idx_ptr, output.data_ptr(), maximum.data_ptr(), denominator.data_ptr(),
            part_o, part_m, part_l, batch, queries, heads, length, topk)
    merge_uv = uv is not None and config.split > 1
    with _on_device(device):
        if merge_uv:
            # Main kernel only; the merge runs inside the W_UV launch below.
            opts = _options(scale, fp8, kv, block_table)
            rc = lib.dsa_fwd_main_opts(*args, ctypes.byref(opts), plan, stream)
        elif scale is None and block_table is None and not fp8 and not fused:
            rc = lib.dsa_fwd(*args, plan, stream)
        else:
            opts = _options(scale, fp8, kv, block_table)
            if fused:
                counters = arrivals if arrivals is not None else _arrival_counters(device, stream, groups)
                opts.arrivals = counters.data_ptr()
            rc = lib.dsa_fwd_opts(*args, ctypes.byref(opts), plan, stream)
    if rc:
        _lib.check(rc, "dsa_fwd_main" if merge_uv else "dsa_fwd")
    if uv is None:
        result = (output, maximum, denominator)
    elif merge_uv:
        dv, head_stride = uv
        out_v = torch.empty((batch, queries, heads, dv), device=device, dtype=torch.bfloat16)
        with _on_device(device):
            rc = lib.dsa_merge_uv(part_o, part_m, part_l, w_uv.data_ptr(), head_stride, out_v.data_ptr(),
                                  maximum.data_ptr(), denominator.data_ptr(), batch * queries, heads,
                                  config.split, dv, stream)
        _lib.check(rc, "dsa_merge_uv")
        result = (out_v, maximum, denominator)
    else:
        result = (project_uv(output, w_uv), maximum, denominator)
    if return_kernels:
        return result, launches
    return result


def _options(scale, fp8, kv, block_table):
    opts = _lib.DsaFwdOptions()
    opts.scale = 0.0 if scale is None else scale
    opts.kv_format = _lib.KV_FP8 if fp8 else _lib.KV_BF16
    if block_table is not None:
        opts.block_size = kv.shape[1]
        opts.max_blocks = block_table.shape[1]
        opts.num_blocks = kv.shape[0]
        opts.block_table = block_table.data_ptr()
    return opts


# Plans of the calls seen so far, keyed by everything plan_call reads: a
# repeated shape skips the table lookup, the plan checks and the descriptor
# construction (the reference checks its table once, at import:
# dsa/api.py:63-73).  Entries are immutable; a bounded dict, cleared when full.
_PLAN_CACHE_MAX = 4096
_plan_cache = {}


def _call_plan(shape, config, cores, fp8, uv_dim):
    """plan_call's result for one call, with the C plan struct (passed by
    reference, read only), whether the merge runs in the main kernel and the
    number of (token, head group) pairs.  ``partials`` becomes (part_o shape,
    part_m shape, floats of the one buffer holding all three, byte offsets of
    part_m and part_l in it) when the plan splits."""
    if type(cores) is not int or cores <= 0:
        raise ValueError("cores must be a positive int")
    if config is not None and not isinstance(config, Tuning):
        raise TypeError("config must be a dsa_amd.Tuning")
    # A Tuning equals one whose int fields are given as bools or floats (True
    # == 1), which check_tuning rejects: the field types are part of the key.
    key = (shape, config, None if config is None else tuple(map(type, vars(config).values())), cores, fp8,
           uv_dim)
    hit = _plan_cache.get(key)
    if hit is not None:
        return hit
    config, partials, launches = plan_call(shape, config, cores, fp8, uv_dim)
    if partials is not None:
        o_elems = 1
        for d in partials[0]:
            o_elems *= d
        m_elems = o_elems // HEAD_DIM
        align = 64  # floats: 256 bytes
        o_pad = -(-o_elems // align) * align
        m_pad = -(-m_elems // align) * align
        partials = (partials[0], partials[1], o_pad + 2 * m_pad, 4 * o_pad, 4 * (o_pad + m_pad))
    batch, queries, heads, _, _ = shape
    fused = config.fused_merge and config.split > 1 and uv_dim is None
    hit = (config, partials, launches, config.to_c(), fused,
           batch * queries * (heads // config.bm))
    if len(_plan_cache) >= _PLAN_CACHE_MAX:
        _plan_cache.clear()
    _plan_cache[key] = hit
    return hit


_device_cu_counts = {}


def _device_cus(device) -> int:
    n = _device_cu_counts.get(device.index)
    if n is None:
        n = torch.cuda.get_device_properties(device).multi_processor_count
        _device_cu_counts[device.index] = n
    return n


# The host fast path (dsa_amd/_fast*.so, built from csrc/fast_forward.cpp):
# forward() for a shape the Python path has already planned on that device
# with the default plan and no options, checked, allocated and launched in
# C++.  It returns None for anything the Python path would reject or has not
# planned, so errors always come from the Python path.  Absent (not built),
# every call takes the Python path.
_fast_lock = threading.Lock()
_fast_state = []  # [module or None] once loaded


def _fast_path():
    if _fast_state:
        return _fast_state[0]
    with _fast_lock:
        if not _fast_state:
            module = None
            from . import build as _build

            path = _build.fast_path_module()
            if path.exists():
                import importlib.util

                spec = importlib.util.spec_from_file_location("dsa_amd._fast", path)
                module = importlib.util.module_from_spec(spec)
                spec.loader.exec_module(module)
                lib = _lib.load()
                module.set_entry(*(ctypes.cast(f, ctypes.c_void_p).value
                                   for f in (lib.dsa_fwd, lib.dsa_fwd_main, lib.dsa_merge)))
            _fast_state.append(module)
    return _fast_state[0]


def _register_fast(device, shape, plan, partials):
    fast = _fast_path()
    if fast is None:
        return
    fields = [plan.heads_per_group, plan.tile_rows, plan.split, plan.kv_waves, plan.stages, plan.mfma,
              plan.fused_merge, plan.pv_cols]
    part = (0, 0, 0) if partials is None else partials[2:]
    fast.register_plan(device.index, *shape, fields, *part)


class _NoDeviceSwitch:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_SAME_DEVICE = _NoDeviceSwitch()


def _on_device(device):
    """``torch.cuda.device(device)`` unless it is already the current device
    (the library launches on the current HIP device)."""
    if torch.cuda.current_device() == device.index:
        return _SAME_DEVICE
    return torch.cuda.device(device)


def bucket_indices(indices, kv_len: int):
    """Each token's indices stably partitioned by kv row range, as
    ``forward`` orders them for prefill-sized calls (no reference
    counterpart): bucket ``x >> s`` for a row index ``0 <= x < kv_len``
    (``s`` the least shift with ``(kv_len - 1) >> s < 64``), then every
    other entry (-1, out of range); within a bucket the caller's order.
    ``indices [B,SQ,1,K]`` int32, contiguous, on a ROCm GPU, K <= 4096;
    returns a new tensor of the same shape."""
    if not isinstance(indices, torch.Tensor) or indices.dim() != 4 or indices.shape[2] != 1:
        raise ValueError("indices must be [B,SQ,1,K]")
    if isinstance(kv_len, bool) or not isinstance(kv_len, int) or not 0 < kv_len < 2 ** 31:
        raise ValueError("kv_len must be a positive int below 2^31")
    device = indices.device
    if device.type != "cuda" or torch.version.hip is None or not indices.is_contiguous():
        raise ValueError("indices must be contiguous on a ROCm GPU")
    if indices.dtype != torch.int32:
        raise ValueError("indices must be int32")
    batch, queries, _, topk = indices.shape
    if min(batch, queries, topk) <= 0 or topk > BUCKET_MAX_TOPK:
        raise ValueError(f"indices must be non-empty with K <= {BUCKET_MAX_TOPK}")
    out = torch.empty_like(indices)
    stream = torch._C._cuda_getCurrentRawStream(device.index)
    with _on_device(device):
        rc = _lib.load().dsa_bucket_indices(indices.data_ptr(), out.data_ptr(), batch * queries, topk, kv_len,
                                            stream)
    _lib.check(rc, "dsa_bucket_indices")
    return out


def _check_partials(part_o, part_m, part_l):
    if part_o.dim() != 5 or part_o.shape[-1] != HEAD_DIM:
        raise ValueError("part_o must be [B,SQ,S,H,512]")
    batch, queries, split, heads, _ = part_o.shape
    for t in (part_m, part_l):
        if tuple(t.shape) != (batch, queries, split, heads):
            raise ValueError("part_m/part_l must be [B,SQ,S,H]")
    device = part_o.device
    if (device.type != "cuda" or any(t.device != device for t in (part_m, part_l))
            or not all(t.is_contiguous() for t in (part_o, part_m, part_l))):
        raise ValueError("partials must be contiguous and on the same ROCm GPU")
    if any(t.dtype != torch.float32 for t in (part_o, part_m, part_l)):
        raise ValueError("partials must be float32")
    return batch, queries, split, heads


def merge(part_o, part_m, part_l):
    """FP32 merge of split partials (reference: dsa/merge.py:13-91).

    ``part_o [B,SQ,S,H,512]``, ``part_m``/``part_l [B,SQ,S,H]`` fp32 on one ROCm
    GPU; returns ``(output, softmax_max, softmax_sum)`` as :func:`forward`.
    """
    batch, queries, split, heads = _check_partials(part_o, part_m, part_l)
    device = part_o.device
    output = torch.empty((batch, queries, heads, HEAD_DIM), device=device, dtype=torch.bfloat16)
    maximum = torch.empty((batch, 1, queries, heads), device=device, dtype=torch.float32)
    denominator = torch.empty_like(maximum)
    stream = torch.cuda.current_stream(device).cuda_stream
    with torch.cuda.device(device):
        rc = _lib.load().dsa_merge(
            ctypes.c_void_p(part_o.data_ptr()), ctypes.c_void_p(part_m.data_ptr()),
            ctypes.c_void_p(part_l.data_ptr()), ctypes.c_void_p(output.data_ptr()),
            ctypes.c_void_p(maximum.data_ptr()), ctypes.c_void_p(denominator.data_ptr()),
            batch * queries, heads, split, ctypes.c_void_p(stream))
    _lib.check(rc, "dsa_merge")
    return output, maximum, denominator


def merge_uv(part_o, part_m, part_l, w_uv):
    """:func:`merge` and :func:`project_uv` in one launch (no reference
    counterpart): returns ``(out_v [B,SQ,H,dv], softmax_max, softmax_sum)``,
    bit-identical to ``project_uv(merge(...)[0], w_uv)`` and ``merge``'s
    max and sum; the merged 512-wide rows are never written."""
    batch, queries, split, heads = _check_partials(part_o, part_m, part_l)
    device = part_o.device
    dv, head_stride = _check_w_uv(w_uv, heads, device)
    out_v = torch.empty((batch, queries, heads, dv), device=device, dtype=torch.bfloat16)
    maximum = torch.empty((batch, 1, queries, heads), device=device, dtype=torch.float32)
    denominator = torch.empty_like(maximum)
    stream = torch.cuda.current_stream(device).cuda_stream
    with torch.cuda.device(device):
        rc = _lib.load().dsa_merge_uv(_vp(part_o), _vp(part_m), _vp(part_l), _vp(w_uv), head_stride, _vp(out_v),
                                      _vp(maximum), _vp(denominator), batch * queries, heads, split, dv,
                                      ctypes.c_void_p(stream))
    _lib.check(rc, "dsa_merge_uv")
    return out_v, maximum, denominator
