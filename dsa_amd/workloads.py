"""Seeded synthetic inputs of the operator's benchmark and test workloads.

``review_inputs`` restates the reference harness's generator
(tools/review.py:35-61): a CPU ``torch.Generator`` seeded once, ``randn`` in
fp32 rounded to bf16 in the order q, kv, q_rope, k_rope, then one
``randperm(L)[:TOPK]`` per token, and the value families ``uniform``,
``peaked``, ``duplicates`` and ``invalid``.  With the reference's seeds it
reproduces the inputs behind the reference's validation records.

``baseline_inputs`` builds the five MI355X benchmark configurations C1..C5 on
a device (C3..C5 are too large for the CPU recipe's fp32 temporaries).
"""
from __future__ import annotations

import torch

REVIEW_SEED = 20261102
FAMILIES = ("normal", "uniform", "peaked", "duplicates", "invalid")

# (B, SQ, H, L, TOPK)
BASELINE_CONFIGS = {
    "c1_decode_b1": (1, 1, 128, 8192, 2048),
    "c2_decode_b8": (8, 1, 128, 32768, 2048),
    "c3_decode_h16_mtp": (64, 2, 16, 65536, 2048),
    "c4_prefill_h16": (1, 4096, 16, 8192, 2048),
    "c5_prefill_h128": (1, 4096, 128, 32768, 2048),
}
C5_HOT_ROWS = 8


def review_inputs(shape, seed: int = REVIEW_SEED, family: str = "normal"):
    """CPU tensors (q, kv, q_rope, k_rope, indices) of the reference recipe."""
    if family not in FAMILIES:
        raise ValueError(f"unknown family {family!r}")
    batch, queries, heads, length, selected = shape
    gen = torch.Generator().manual_seed(seed)

    def normal(*dims):
        return torch.randn(dims, generator=gen).bfloat16()

    q = normal(batch, queries, heads, 512)
    kv = normal(batch, length, 1, 512)
    qr = normal(batch, queries, heads, 64)
    kr = normal(batch, length, 1, 64)
    ids = torch.stack([torch.randperm(length, generator=gen)[:selected]
                       for _ in range(batch * queries)]).reshape(batch, queries, 1, selected).int()
    if family == "uniform":
        q.zero_()
        qr.zero_()
    elif family == "peaked":
        q.mul_(4)
        qr.mul_(4)
    elif family == "duplicates":
        ids[..., 1::2] = ids[..., 0::2]
    elif family == "invalid":
        ids[..., selected // 2:] = -1
    return q, kv, qr, kr, ids


def _normal_bf16(dims, gen, device):
    return torch.randn(dims, generator=gen, device=device, dtype=torch.float32).bfloat16()


def _subset_rows(n_rows, length, k, gen, device, limit=None):
    """``n_rows`` index rows, each ``k`` distinct values uniform over [0, limit_i)."""
    keys = torch.rand((n_rows, length), generator=gen, device=device)
    if limit is not None:
        cols = torch.arange(length, device=device)
        keys.masked_fill_(cols[None, :] >= limit[:, None], 2.0)
    return keys.topk(k, dim=1, largest=False).indices.int()


def case_inputs(shape, seed: int = REVIEW_SEED, device="cuda"):
    """Inputs of any (B, SQ, H, L, TOPK) shape drawn on ``device`` from the
    review recipe's distribution (family normal: N(0,1) bf16 q/kv/rope, per
    token TOPK distinct indices uniform over [0, L)).  ``review_inputs`` draws
    the same distribution on the CPU call for call as the reference does; this
    one is for timing the reference's cases at full size (its largest, 4 x 8192
    tokens x 128 heads, takes seconds here)."""
    batch, queries, heads, length, k = shape
    gen = torch.Generator(device=device).manual_seed(seed)
    q = _normal_bf16((batch, queries, heads, 512), gen, device)
    kv = _normal_bf16((batch, length, 1, 512), gen, device)
    qr = _normal_bf16((batch, queries, heads, 64), gen, device)
    kr = _normal_bf16((batch, length, 1, 64), gen, device)
    tokens = batch * queries
    rows = max(1, (64 << 20) // (4 * length))  # 64 MiB of sort keys per chunk
    ids = torch.cat([_subset_rows(min(rows, tokens - i), length, k, gen, device) for i in range(0, tokens, rows)])
    return q, kv, qr, kr, ids.reshape(batch, queries, 1, k).contiguous()


def baseline_inputs(name: str, seed: int = REVIEW_SEED, device="cuda", cpu_recipe: bool = True):
    """Inputs of MI355X benchmark configuration ``name`` on ``device``.

    c1, c2: the reference recipe (family normal), generated on the CPU; with
        ``cpu_recipe=False`` the same distribution is drawn on ``device``
        (N(0,1) bf16, distinct uniform indices per token) -- much faster for
        the benchmark's rotating input sets.
    c3: N(0,1) bf16; per token ``TOPK`` distinct indices uniform over [0, L).
    c4: query i sits at position 4096 + i; its indices are distinct and
        uniform over [0, 4096 + i] (all valid).
    c5: four families over contiguous quarters of SQ --
        peaked (8 hot rows of kv/k_rope scaled x4, forced into every index set),
        duplicates (sampled with replacement), invalid (512 of 2048 slots = -1),
        uniform (distinct, uniform).
    """
    shape = BASELINE_CONFIGS[name]
    batch, queries, heads, length, k = shape
    if name in ("c1_decode_b1", "c2_decode_b8") and cpu_recipe:
        return tuple(t.to(device) for t in review_inputs(shape, seed, "normal"))
    gen = torch.Generator(device=device).manual_seed(seed)
    q = _normal_bf16((batch, queries, heads, 512), gen, device)
    kv = _normal_bf16((batch, length, 1, 512), gen, device)
    qr = _normal_bf16((batch, queries, heads, 64), gen, device)
    kr = _normal_bf16((batch, length, 1, 64), gen, device)
    tokens = batch * queries
    if name in ("c1_decode_b1", "c2_decode_b8", "c3_decode_h16_mtp"):
        ids = torch.cat([_subset_rows(min(32, tokens - i), length, k, gen, device)
                         for i in range(0, tokens, 32)])
    elif name == "c4_prefill_h16":
        limit = torch.arange(queries, device=device) + 4097  # [0, 4096 + i] inclusive
        ids = _subset_rows(queries, length, k, gen, device, limit)
    elif name == "c5_prefill_h128":
        fam = queries // 4
        hot = torch.randperm(length, generator=gen, device=device)[:C5_HOT_ROWS]
        kv[0, hot] *= 4
        kr[0, hot] *= 4
        # peaked: hot rows first in key order, then shuffled within the row
        keys = torch.rand((fam, length), generator=gen, device=device)
        keys[:, hot] = -1.0
        peaked = keys.topk(k, dim=1, largest=False).indices
        order = torch.rand((fam, k), generator=gen, device=device).argsort(dim=1)
        peaked = torch.gather(peaked, 1, order).int()
        dup = torch.randint(0, length, (fam, k), generator=gen, device=device, dtype=torch.int32)
        inv = _subset_rows(fam, length, k, gen, device)
        slots = torch.rand((fam, k), generator=gen, device=device).argsort(dim=1)[:, : k // 4]
        inv.scatter_(1, slots, -1)
        uni = _subset_rows(queries - 3 * fam, length, k, gen, device)
        ids = torch.cat([peaked, dup, inv, uni])
    else:
        raise ValueError(name)
    return q, kv, qr, kr, ids.reshape(batch, queries, 1, k).contiguous()


# Lightning-indexer workloads: (B, SQ, HI, L, TOPK, causal).  The decode
# pair feeds C2 / C3's attention (same B, SQ, L, TOPK); the prefill one is C5's
# query block, with query i at position L - SQ + i (keys [0, L - SQ + i]).
INDEXER_CONFIGS = {
    "idx_decode_b8": (8, 1, 64, 32768, 2048, False),
    "idx_decode_mtp_b64": (64, 2, 64, 65536, 2048, False),
    "idx_prefill_4k": (1, 4096, 64, 32768, 2048, True),
}


def indexer_lengths(name: str, device="cuda"):
    """Candidate keys per query ``[B, SQ]`` int32 of indexer workload ``name``:
    query i of SQ sits at position L - SQ + i and sees keys [0, L - SQ + i]
    (decode: the last SQ positions; prefill: causal prefixes)."""
    batch, queries, _, length, _, _ = INDEXER_CONFIGS[name]
    row = torch.arange(queries, device=device, dtype=torch.int32) + (length - queries + 1)
    return row.expand(batch, queries).contiguous()


def indexer_inputs(name: str, seed: int = REVIEW_SEED, device="cuda"):
    """(q_idx, k_idx, weights, lengths) of indexer workload ``name``: N(0,1)
    bf16 queries and keys, N(0, 0.1^2) fp32 head weights."""
    batch, queries, heads, length, _, _ = INDEXER_CONFIGS[name]
    gen = torch.Generator(device=device).manual_seed(seed)
    q = _normal_bf16((batch, queries, heads, 128), gen, device)
    k = _normal_bf16((batch, length, 128), gen, device)
    w = torch.randn((batch, queries, heads), generator=gen, device=device) * 0.1
    return q, k, w, indexer_lengths(name, device)
