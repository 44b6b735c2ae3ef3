"""CPU oracle of the sparse-MLA attention forward.

TEST INFRASTRUCTURE ONLY.  Imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` -- as the checker, never as the
thing measured or shipped.  The product path (``dsa_amd``) never imports it.

Functions and the reference code each one restates:

* ``reference``       -- the reference harness's FP32 oracle
                         (tools/review.py:130-145): per batch and 16-query chunk,
                         gather kv/k_rope rows in fp32, two bmm / 24, -inf mask
                         from the raw index, amax / exp / sum, bmm(P / sum, kv).
* ``accuracy``        -- its metrics (tools/review.py:146-175): max-normalised
                         error N, relative RMS, per-row normalised error.
* ``golden_stats``    -- the oracle statistics the reference's validation
                         records hold (ref_max, ref_sq, elements).
* ``online_softmax``  -- the tiled online-softmax recurrence
                         (DSA从原理到实现.md:159-199; dsa/workspace.py:242-354).
* ``merge_states``    -- the split-KV merge (dsa/merge.py:1-5, :56-87).
* ``c_exact`` / ``c_tiled`` -- the C restatement in oracle/dsa_oracle.c:
                         FP64 brute force, and the device-side arithmetic
                         (tiles, bf16 P, FP32 state, split + merge).
* ``unpage`` / ``mask_unbacked`` -- paged-kv pools to the reference's
                         contiguous layout (no reference counterpart: the
                         reference takes contiguous kv only), so paged runs are
                         checked against the same ``reference``.

* ``e4m3_decode`` / ``dequant_fp8_rows`` -- the fp8 kv cache rows (656
                         bytes: 512 OCP e4m3, 4 fp32 scales, 64 bf16 rope; no
                         reference counterpart, which takes bf16 kv only,
                         dsa/api.py:30-33) back to the bf16 kv and rope the
                         kernels compute with, so fp8 runs are checked against
                         the same ``reference``.
* ``indexer_logits_ref`` / ``indexer_topk_ref`` / ``float_key`` -- the
                         lightning indexer (no reference counterpart: the
                         reference takes the indices as an input,
                         README.md:19-21).  The logits restate the published
                         DSA indexer score I[t,s] = sum_j w[t,j] *
                         ReLU(q[t,j] . k[s]) (DeepSeek-V3.2-Exp report, eq. 1);
                         the selection keeps the TOPK largest (ties: lower s)
                         in ascending s, -1 padded.

* ``bucket_shift`` / ``bucket_rows_ref`` -- the row-range bucketing of
                         prefill calls' indices (no reference counterpart:
                         the reference takes the slots in the caller's order,
                         dsa/workspace.py:76-141): a stable partition by
                         x >> shift (shift the least with (L - 1) >> shift
                         < 64), entries outside [0, L) last.

* ``project_uv_ref``  -- the W_UV output projection after the attention (no
                         reference counterpart: the reference stops at the
                         latent output, README.md:81-83): DeepSeek-V3.2-Exp
                         inference/model.py, MLA.forward absorb branch,
                         ``einsum("bshc,hdc->bshd", x, wkv_b[:, -v_head_dim:])``,
                         in FP64.

``reference(scale=...)`` generalises the fixed 1/24 (tools/review.py:140) to
another softmax scale; the default keeps the reference's exact division.

Pinning (tests/test_oracle.py): golden statistics of 20 reference validation
records, both tutorial known-answer tests, reduction to a library
scaled_dot_product_attention (which also pins ``scale``), FP64 brute force,
closed forms of the uniform family, index-permutation / -1-removal /
duplicate-counting invariants, an identity block table and a gather
restatement for ``unpage``, and planted mistakes that each check must reject.
FP8 rows: ``e4m3_decode`` against torch's float8_e4m3fn on all 256 codes and
against hand-worked values; ``dequant_fp8_rows`` against an element-wise
restatement, with planted mistakes (a 64-dim scale block, rounding to bf16
before the scale) rejected.
W_UV: an FP64 triple-loop brute force, one-hot weight rows (the projection
then gathers latent columns exactly) and linearity, with planted mistakes
(weights of the wrong head, the transposed head matrix) rejected.
Bucketing: the shift's closed form at the 64-bucket boundaries, a
distribution into 65 lists restatement, permutation / non-decreasing-key /
stability properties, with planted mistakes (an unstable order, a sort by
value, masked entries first) rejected.
Indexer: FP64 brute-force logits (planted: ReLU or head weights dropped),
brute-force selection over tie-heavy rows, -0.0 / +0.0, -inf and short rows
(planted: ties taken from the top), and the float-key order.
"""
from __future__ import annotations

import ctypes
import math
from pathlib import Path

import numpy as np
import torch

SCALE_DIVISOR = 24.0  # score = dot / 24 (tools/review.py:140)
HERE = Path(__file__).resolve().parent
C_LIB = HERE / "_build" / "libdsa_oracle.so"


def reference(q, kv, q_rope, k_rope, indices, chunk: int = 16, tokens=None, scale=None):
    """FP32 oracle: returns (output fp32 [B,SQ,H,512], max [B,1,SQ,H], sum [B,1,SQ,H]).

    ``tokens``: optional iterable of (b, s) pairs; only those rows are computed
    (the rest of the outputs stay NaN).  ``scale``: softmax scale (None: the
    reference's fixed division by 24, tools/review.py:140).
    """
    q, kv, q_rope, k_rope, indices = (t.cpu() for t in (q, kv, q_rope, k_rope, indices))
    batch, queries, heads, _ = q.shape
    length = kv.shape[1]
    out = torch.full((batch, queries, heads, 512), float("nan"))
    mx = torch.full((batch, 1, queries, heads), float("nan"))
    sm = torch.full((batch, 1, queries, heads), float("nan"))
    if tokens is None:
        work = [(bi, list(range(s, min(queries, s + chunk))))
                for bi in range(batch) for s in range(0, queries, chunk)]
    else:
        by_b: dict[int, list[int]] = {}
        for bi, s in tokens:
            by_b.setdefault(int(bi), []).append(int(s))
        work = [(bi, ss[i:i + chunk]) for bi, ss in sorted(by_b.items()) for i in range(0, len(ss), chunk)]
    for bi, rows in work:
        rows_t = torch.tensor(rows)
        index = indices[bi, rows_t, 0].long()
        valid = (index >= 0) & (index < length)
        index = index.clamp(0, length - 1)
        selected = kv[bi, index, 0].float()
        rope = k_rope[bi, index, 0].float()
        score = (torch.bmm(q[bi, rows_t].float(), selected.transpose(1, 2))
                 + torch.bmm(q_rope[bi, rows_t].float(), rope.transpose(1, 2)))
        score = score / SCALE_DIVISOR if scale is None else score * scale
        score.masked_fill_(~valid[:, None, :], -float("inf"))
        maximum = score.amax(-1)
        exponent = (score - maximum[..., None]).exp()
        denominator = exponent.sum(-1)
        out[bi, rows_t] = torch.bmm(exponent / denominator[..., None], selected)
        mx[bi, 0, rows_t] = maximum
        sm[bi, 0, rows_t] = denominator
    return out, mx, sm


def unpage(kv_pool, rope_pool, block_table):
    """Contiguous ``[B, L, 1, D]`` copies of paged kv / k_rope pools
    ``[num_blocks, block_size, 1, D]`` under ``block_table [B, max_blocks]``
    (logical row I of batch b = pool row block_table[b, I // block_size] *
    block_size + I % block_size), and a ``[B, L]`` bool that is False where
    the block entry lies outside the pool (those rows are masked)."""
    kv_pool, rope_pool, block_table = (t.cpu() for t in (kv_pool, rope_pool, block_table))
    blocks, size = kv_pool.shape[:2]
    rows = torch.arange(block_table.shape[1] * size)
    blk = block_table[:, rows // size].long()
    ok = (blk >= 0) & (blk < blocks)
    flat = blk.clamp(0, blocks - 1) * size + rows % size
    kv = kv_pool.reshape(blocks * size, 1, -1)[flat]
    rope = rope_pool.reshape(blocks * size, 1, -1)[flat]
    return kv, rope, ok


def mask_unbacked(indices, ok):
    """indices with every slot that points at a row without a valid block
    (``ok`` False, see :func:`unpage`) replaced by -1."""
    indices = indices.cpu().clone()
    batch, length = ok.shape
    inside = (indices >= 0) & (indices < length)
    rows = indices.clamp(0, length - 1).long()
    backed = torch.gather(ok[:, None, None, :].expand(-1, indices.shape[1], 1, -1), 3, rows)
    indices[inside & ~backed] = -1
    return indices


def e4m3_decode(codes):
    """OCP float8 e4m3 (bias 7, no infinities, S.1111.111 = NaN) to float32,
    from the format's definition: normal (1 + m/8) 2^(e-7), subnormal
    (m/8) 2^-6."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 15
    m = c & 7
    mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * 2.0 ** (e - 7))
    out = (sign * mag).astype(np.float32)
    out[(c & 0x7F) == 0x7F] = np.nan
    return out


def dequant_fp8_rows(rows):
    """FP8 kv cache rows ``[..., 656]`` (uint8) -> ``(kv [..., 512], rope
    [..., 64])`` bf16: ``kv[d] = bf16(fp32(e4m3[d]) * scale[d // 128])`` with
    fp32 round-to-nearest-even product and bf16 round-to-nearest-even (no
    reference counterpart; the DeepSeek-V3.2 FP8 MLA cache row layout)."""
    u8 = rows.cpu().contiguous()
    lead = u8.shape[:-1]
    vals = torch.from_numpy(e4m3_decode(u8[..., :512].numpy())).reshape(*lead, 4, 128)
    scales = u8[..., 512:528].contiguous().view(torch.float32).reshape(*lead, 4, 1)
    kv = (vals * scales).reshape(*lead, 512).bfloat16()
    rope = u8[..., 528:656].contiguous().view(torch.bfloat16)
    return kv, rope


def indexer_logits_ref(q_idx, k_idx, weights, lengths, chunk: int = 64):
    """FP32 lightning-indexer logits ``[B, SQ, L]``:
    ``sum_j w[t, j] * relu(q_idx[t, j] . k_idx[s])`` for ``s < lengths[t]``,
    -inf beyond (no reference counterpart; the DSA indexer's definition)."""
    q, k, w, lengths = (t.cpu() for t in (q_idx, k_idx, weights, lengths))
    batch, queries, _, _ = q.shape
    length = k.shape[1]
    out = torch.empty((batch, queries, length))
    for b in range(batch):
        kb = k[b].float()
        for t0 in range(0, queries, chunk):
            qs = q[b, t0:t0 + chunk].float()                      # [c, HI, 128]
            dots = torch.einsum("chd,sd->chs", qs, kb)            # [c, HI, L]
            out[b, t0:t0 + chunk] = (dots.clamp_min(0) * w[b, t0:t0 + chunk].float()[..., None]).sum(1)
    cols = torch.arange(length)
    out.masked_fill_(cols[None, None, :] >= lengths.clamp(0, length)[..., None].long(), -float("inf"))
    return out


def project_uv_ref(output, w_uv):
    """FP64 W_UV projection ``out[..., h, d] = sum_c output[..., h, c] *
    w_uv[h, d, c]`` (DeepSeek-V3.2-Exp inference/model.py, MLA.forward:
    ``einsum("bshc,hdc->bshd", x, wkv_b[:, -v_head_dim:])``); ``output
    [..., H, 512]``, ``w_uv [H, dv, 512]``; returns float64 ``[..., H, dv]``."""
    x = output.detach().cpu().double()
    w = w_uv.detach().cpu().double()
    heads = x.shape[-2]
    xs = x.reshape(-1, heads, x.shape[-1]).transpose(0, 1)   # [H, T, 512]
    out = torch.bmm(xs, w.transpose(1, 2))                    # [H, T, dv], FP64 on the CPU
    return out.transpose(0, 1).reshape(*x.shape[:-1], w.shape[1])


def bucket_shift(kv_len: int) -> int:
    """The least shift with (kv_len - 1) >> shift < 64."""
    shift = 0
    while (kv_len - 1) >> shift >= 64:
        shift += 1
    return shift


def bucket_rows_ref(indices, kv_len: int):
    """``indices [..., K]`` int32 with each row stably ordered by bucket:
    ``x >> bucket_shift(kv_len)`` for ``0 <= x < kv_len``, 64 for any other
    entry."""
    ids = np.ascontiguousarray(indices.cpu().numpy())
    valid = (ids >= 0) & (ids < kv_len)
    keys = np.where(valid, ids.astype(np.int64) >> bucket_shift(kv_len), 64)
    order = np.argsort(keys, axis=-1, kind="stable")
    return torch.from_numpy(np.take_along_axis(ids, order, axis=-1))


def float_key(values):
    """Order-preserving uint32 keys of float32 values (larger value, larger
    key; -0.0 below +0.0), the order the device selection uses."""
    bits = np.ascontiguousarray(np.asarray(values, dtype=np.float32)).view(np.uint32)
    return np.where(bits & np.uint32(0x80000000), ~bits, bits | np.uint32(0x80000000)).astype(np.uint32)


def indexer_topk_ref(logits, lengths, topk: int):
    """``indices [B, SQ, 1, topk]`` int32: per row the ``topk`` largest logits
    among ``s < lengths`` by :func:`float_key` (ties: lower s first), in
    ascending s order, padded with -1."""
    logits = logits.cpu().float().numpy()
    lengths = lengths.cpu().numpy()
    batch, queries, length = logits.shape
    out = np.full((batch, queries, 1, topk), -1, dtype=np.int32)
    for b in range(batch):
        for t in range(queries):
            n = int(min(max(lengths[b, t], 0), length))
            keys = float_key(logits[b, t, :n])
            order = np.lexsort((np.arange(n), ~keys))  # key descending, then s ascending
            chosen = np.sort(order[:topk])
            out[b, t, 0, :chosen.size] = chosen
    return torch.from_numpy(out)


def accuracy(actual, expected):
    """Reference metrics (tools/review.py:146-175) of one output tensor pair.

    ``max_row_normalized`` is the reference's per-row error
    (tools/review.py:160-161): for every row of the last dimension,
    max|delta| / max|expected| over that row, maximised over rows -- per
    (token, head) over the 512 columns for the output ``[..., H, 512]``, per
    query over the H heads for softmax_max / softmax_sum ``[B, 1, SQ, H]`` --
    so one erroneous row cannot hide behind another row's scale.  Rows the
    oracle left NaN (``reference(tokens=...)``) are skipped.
    """
    actual = actual.float().cpu()
    expected = expected.float().cpu()
    keep = ~torch.isnan(expected)
    a, e = actual[keep], expected[keep]
    delta = a - e
    ref_max = float(e.abs().max())
    width = expected.shape[-1]
    rows_e = expected.reshape(-1, width)
    rows_a = actual.reshape(-1, width)
    full = ~torch.isnan(rows_e).any(-1)
    rows_e, rows_a = rows_e[full], rows_a[full]
    row_error = (rows_a - rows_e).abs().amax(-1) / rows_e.abs().amax(-1).clamp_min(1e-30)
    return {
        "max_abs": float(delta.abs().max()),
        "reference_max": ref_max,
        "max_normalized": float(delta.abs().max()) / max(ref_max, 1e-30),
        "max_row_normalized": float(row_error.max()) if row_error.numel() else 0.0,
        "relative_rms": (float(delta.double().square().sum()) / max(float(e.double().square().sum()), 1e-30)) ** 0.5,
        "finite": bool(torch.isfinite(a).all()),
        "elements": int(e.numel()),
        "rows": int(row_error.numel()),
    }


def rel_error(actual, expected):
    """max |actual - expected| / |expected| elementwise (for max/sum rtol gates)."""
    actual = actual.double().cpu()
    expected = expected.double().cpu()
    keep = ~torch.isnan(expected)
    return float(((actual[keep] - expected[keep]).abs() / expected[keep].abs().clamp_min(1e-30)).max())


def golden_stats(out, mx, sm, chunk: int = 16):
    """(reference_max, ref_sq, elements) per output, accumulated like the
    reference harness: Python floats of fp32 per-(batch, chunk) sums."""
    stats = {}
    for key, t in (("output", out), ("maximum", mx), ("denominator", sm)):
        t = t.float()
        batch = t.shape[0]
        queries = t.shape[1] if key == "output" else t.shape[2]
        ref_sq, ref_max, n = 0.0, 0.0, 0
        for bi in range(batch):
            for s in range(0, queries, chunk):
                piece = t[bi, s:s + chunk] if key == "output" else t[bi, 0, s:s + chunk]
                ref_sq += float(piece.square().sum())
                ref_max = max(ref_max, float(piece.abs().max()))
                n += piece.numel()
        stats[key] = {"reference_max": ref_max, "ref_sq": ref_sq, "elements": n}
    return stats


def online_softmax(scores, values, chunks):
    """Scalar online softmax over ``chunks`` [(begin, end), ...] (float64).

    Returns (m, l, u, u / l).  Restates DSA从原理到实现.md:181-197.
    """
    m, den, num = -math.inf, 0.0, 0.0
    for begin, end in chunks:
        nxt = max(m, max(scores[begin:end]))
        rescale = math.exp(m - nxt) if m != -math.inf else 0.0
        w = [math.exp(s - nxt) for s in scores[begin:end]]
        den = rescale * den + sum(w)
        num = rescale * num + sum(p * v for p, v in zip(w, values[begin:end]))
        m = nxt
    return m, den, num, num / den


def merge_states(states):
    """Merge split states [(m_s, l_s, u_s), ...] (dsa/merge.py:1-5) -> (m, l, u / l)."""
    m = max(s[0] for s in states)
    w = [math.exp(s[0] - m) for s in states]
    den = sum(wi * s[1] for wi, s in zip(w, states))
    num = sum(wi * s[2] for wi, s in zip(w, states))
    return m, den, num / den


# ------------------------------------------------------------------ C oracle
_c = None


def _c_lib():
    global _c
    if _c is None:
        if not C_LIB.exists():
            from . import build as _build  # noqa: F401  (oracle/build.py)
            _build.build()
        lib = ctypes.CDLL(str(C_LIB))
        vp, i32 = ctypes.c_void_p, ctypes.c_int
        for name, extra in (("dsa_oracle_exact", []), ("dsa_oracle_tiled", [i32, i32])):
            fn = getattr(lib, name)
            fn.restype = i32
            fn.argtypes = [vp] * 5 + [i32] * 5 + extra + [vp] * 3
        _c = lib
    return _c


def _bits(t):
    return np.ascontiguousarray(t.cpu().contiguous().view(torch.int16).numpy())


def _run_c(name, q, kv, q_rope, k_rope, indices, extra, dtype):
    batch, queries, heads, _ = q.shape
    length, topk = kv.shape[1], indices.shape[-1]
    arrs = [_bits(q), _bits(kv), _bits(q_rope), _bits(k_rope),
            np.ascontiguousarray(indices.cpu().int().numpy())]
    out = np.zeros((batch, queries, heads, 512), dtype=dtype)
    mx = np.zeros((batch, 1, queries, heads), dtype=dtype)
    sm = np.zeros_like(mx)
    ptrs = [ctypes.c_void_p(a.ctypes.data) for a in arrs + [out, mx, sm]]
    rc = getattr(_c_lib(), name)(*ptrs[:5], batch, queries, heads, length, topk, *extra, *ptrs[5:])
    if rc != 0:
        raise ValueError(f"{name} rejected its arguments (rc={rc})")
    return torch.from_numpy(out), torch.from_numpy(mx), torch.from_numpy(sm)


def c_exact(q, kv, q_rope, k_rope, indices):
    """FP64 brute force in C (float64 outputs)."""
    return _run_c("dsa_oracle_exact", q, kv, q_rope, k_rope, indices, [], np.float64)


def c_tiled(q, kv, q_rope, k_rope, indices, tile: int = 64, split: int = 1):
    """Device-arithmetic model in C: FP32 tiles of ``tile`` slots, bf16 P,
    ``split`` contiguous tile ranges merged in FP32.  Output is fp32 before the
    final bf16 rounding."""
    return _run_c("dsa_oracle_tiled", q, kv, q_rope, k_rope, indices, [tile, split], np.float32)
