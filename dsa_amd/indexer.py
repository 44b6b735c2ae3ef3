"""Lightning indexer: the token selector that produces ``indices`` for
:func:`dsa_amd.forward` (the step before the sparse attention; the reference
takes the indices as an input, README.md:19-21, and has no counterpart).

``logits[b, t, s] = sum_j weights[b, t, j] * relu(q_idx[b, t, j] . k_idx[b, s])``
for ``s < lengths[b, t]``; the selection keeps, per query, the ``topk`` keys of
largest logit (ties: lower ``s`` first) in ascending ``s`` order, padded with
-1.  Both steps run on the gfx950 kernels of ``dsa_amd/csrc/indexer.hip``
through the C ABI; there is no CPU path.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

INDEX_DIM = 128
INDEX_HEADS = (32, 64)


def _device_ok(device, tensors):
    return (device.type == "cuda" and torch.version.hip is not None
            and all(t.device == device for t in tensors) and all(t.is_contiguous() for t in tensors))


def _check_lengths(lengths, batch, queries, device):
    if tuple(lengths.shape) != (batch, queries):
        raise ValueError("lengths must be [B, SQ]")
    if lengths.dtype != torch.int32:
        raise ValueError("lengths must be int32")


def indexer_logits(q_idx, k_idx, weights, lengths):
    """Index logits ``[B, SQ, L]`` fp32 (entries past a row's length unspecified)."""
    if q_idx.dim() != 4 or k_idx.dim() != 3 or weights.dim() != 3:
        raise ValueError("expected q_idx[B,SQ,HI,128], k_idx[B,L,128], weights[B,SQ,HI], lengths[B,SQ]")
    batch, queries, heads, dim = q_idx.shape
    length = k_idx.shape[1]
    if (dim != INDEX_DIM or tuple(k_idx.shape) != (batch, length, INDEX_DIM)
            or tuple(weights.shape) != (batch, queries, heads) or min(batch, queries, length) <= 0):
        raise ValueError("expected q_idx[B,SQ,HI,128], k_idx[B,L,128], weights[B,SQ,HI], lengths[B,SQ]")
    if heads not in INDEX_HEADS:
        raise ValueError(f"the number of indexer heads must be 32 or 64 (got {heads})")
    _check_lengths(lengths, batch, queries, q_idx.device)
    device = q_idx.device
    if not _device_ok(device, (q_idx, k_idx, weights, lengths)):
        raise ValueError("all inputs must be contiguous and on the same ROCm GPU")
    if q_idx.dtype != torch.bfloat16 or k_idx.dtype != torch.bfloat16 or weights.dtype != torch.float32:
        raise ValueError("q_idx and k_idx must be bfloat16, weights float32")
    logits = torch.empty((batch, queries, length), device=device, dtype=torch.float32)
    stream = torch.cuda.current_stream(device).cuda_stream
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    with torch.cuda.device(device):
        rc = _lib.load().dsa_indexer_logits(p(q_idx), p(k_idx), p(weights), p(lengths), p(logits),
                                            batch, queries, heads, length, ctypes.c_void_p(stream))
    _lib.check(rc, "dsa_indexer_logits")
    return logits


def indexer_topk(logits, lengths, topk: int, *, segmented: bool = True):
    """``indices [B, SQ, 1, topk]`` int32: per row the ``topk`` largest logits among
    ``s < lengths`` (ties: lower ``s`` first), ascending, padded with -1.

    With few rows (``B * SQ <= 32``) and ``segmented`` the selection splits every
    row over 8 workgroups (three launches, same result bit for bit)."""
    if type(topk) is not int or topk <= 0:
        raise ValueError("topk must be a positive int")
    if logits.dim() != 3 or min(logits.shape) <= 0:
        raise ValueError("logits must be [B, SQ, L]")
    batch, queries, length = logits.shape
    _check_lengths(lengths, batch, queries, logits.device)
    device = logits.device
    if not _device_ok(device, (logits, lengths)):
        raise ValueError("all inputs must be contiguous and on the same ROCm GPU")
    if logits.dtype != torch.float32:
        raise ValueError("logits must be float32")
    indices = torch.empty((batch, queries, 1, topk), device=device, dtype=torch.int32)
    stream = torch.cuda.current_stream(device).cuda_stream
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    lib = _lib.load()
    # few rows: the segmented selection (8 workgroups per row) over a scratch workspace
    ws_bytes = lib.dsa_indexer_topk_ws_bytes(batch, queries, length, topk) if segmented else 0
    with torch.cuda.device(device):
        if ws_bytes > 0:
            ws = torch.empty(ws_bytes, device=device, dtype=torch.uint8)
            rc = lib.dsa_indexer_topk_ws(p(logits), p(lengths), p(indices), batch, queries, length, topk,
                                         p(ws), ws_bytes, ctypes.c_void_p(stream))
        else:
            rc = lib.dsa_indexer_topk(p(logits), p(lengths), p(indices), batch, queries, length, topk,
                                      ctypes.c_void_p(stream))
    _lib.check(rc, "dsa_indexer_topk")
    return indices


def indexer(q_idx, k_idx, weights, lengths, topk: int):
    """Logits then selection: the ``indices`` input of :func:`dsa_amd.forward`."""
    return indexer_topk(indexer_logits(q_idx, k_idx, weights, lengths), lengths, topk)
