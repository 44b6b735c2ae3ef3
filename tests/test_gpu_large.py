"""Maximum sizes: L at the contract's limit (2^25 - 1 rows per batch, 36 GiB of
kv and k_rope per batch), and a paged pool of the same size.

Only the rows a call reads are written (the selected rows, row 0 -- where a
masked slot's gather points -- and row L - 1, where an index >= L is
clamped); the rest of the allocation is never touched.  The check runs the
FP32 oracle on a compacted copy: the selected rows renumbered 0..n-1 and the
indices mapped accordingly (-1 and >= L both become -1), which leaves the
oracle's result unchanged (the index-relabelling and -1 invariants of the
oracle tests).
"""
import pytest
import torch

import dsa_amd
from dsa_amd import Tuning
from _parity import check
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu

L_MAX = (1 << 25) - 1


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    torch.cuda.init()


def _indices(g, B, SQ, K, L):
    """Slots near the top of [0, L), around 2^24 and anywhere, with -1,
    >= L and duplicated entries."""
    parts = [L - 1 - torch.randint(0, 5000, (B, SQ, 1, K // 4), generator=g),
             (1 << 24) + torch.randint(-3000, 3000, (B, SQ, 1, K // 4), generator=g),
             torch.randint(0, L, (B, SQ, 1, K - K // 2), generator=g)]
    ids = torch.cat(parts, dim=-1).to(torch.int32)
    u = torch.rand(ids.shape, generator=g)
    ids[u < 0.04] = -1
    ids[(u >= 0.04) & (u < 0.06)] = L + 7
    dup = (u >= 0.06) & (u < 0.10)
    ids[..., 1:][dup[..., 1:]] = ids[..., :-1][dup[..., 1:]]
    ids[..., :1] = L - 1 - torch.randint(0, 5000, (B, SQ, 1, 1), generator=g, dtype=torch.int32)
    return ids.contiguous()


def _compact(ids, L):
    """Renumber each batch's selected rows 0..n-1: returns the row lists and
    the relabelled indices (-1 for every masked slot)."""
    B = ids.shape[0]
    sel = []
    out = torch.full_like(ids, -1)
    for b in range(B):
        valid = ids[b][(ids[b] >= 0) & (ids[b] < L)]
        uniq = torch.unique(valid)
        sel.append(uniq)
        pos = torch.searchsorted(uniq, ids[b].clamp(0, L - 1))
        ok = (ids[b] >= 0) & (ids[b] < L)
        out[b][ok] = pos[ok].to(torch.int32)
    return sel, out


def _check(tag, got, ref):
    return check(tag, *got, ref)


@pytest.mark.parametrize("H,config", [(16, None), (128, Tuning(128, 32, 1, stages=4)),
                                      (32, Tuning(32, 32, 2, kv_waves=2, stages=4, mfma=16, pv_cols=128))],
                         ids=["h16-planner", "h128-wide", "h32-specialised"])
def test_max_length_contiguous(H, config):
    B, SQ, K, L = 2, 2, 1024, L_MAX
    g = torch.Generator().manual_seed(H)
    ids = _indices(g, B, SQ, K, L)
    sel, ids_small = _compact(ids, L)
    nmax = max(int(s.numel()) for s in sel)
    kv_small = torch.zeros(B, nmax, 1, 512).bfloat16()
    kr_small = torch.zeros(B, nmax, 1, 64).bfloat16()
    for b in range(B):
        n = sel[b].numel()
        kv_small[b, :n] = torch.randn(n, 1, 512, generator=g).bfloat16()
        kr_small[b, :n] = torch.randn(n, 1, 64, generator=g).bfloat16()
    q = torch.randn(B, SQ, H, 512, generator=g).bfloat16()
    qr = torch.randn(B, SQ, H, 64, generator=g).bfloat16()
    tag = f"L=2^25-1 H={H}"
    print(f"[{tag}] allocating {B * L * 1152 / 2 ** 30:.1f} GiB", flush=True)
    kv = torch.empty(B, L, 1, 512, dtype=torch.bfloat16, device="cuda")
    kr = torch.empty(B, L, 1, 64, dtype=torch.bfloat16, device="cuda")
    for b in range(B):
        kv[b, 0] = 0
        kv[b, L - 1] = 0
        kr[b, 0] = 0
        kr[b, L - 1] = 0
        rows = sel[b].cuda().long()
        kv[b, rows] = kv_small[b, :rows.numel()].cuda()
        kr[b, rows] = kr_small[b, :rows.numel()].cuda()
    print(f"[{tag}] launching", flush=True)
    got = dsa_amd.forward(q.cuda(), kv, qr.cuda(), kr, ids.cuda(), config=config)
    torch.cuda.synchronize()
    del kv, kr
    torch.cuda.empty_cache()
    ref = O.reference(q, kv_small, qr, kr_small, ids_small)
    _check(tag, got, ref)


def test_max_pool_paged():
    B, SQ, H, K, bs = 2, 1, 32, 1024, 64
    nblocks = L_MAX // bs            # pool rows: nblocks * 64 < 2^25
    M = 64                           # logical blocks per sequence: L = 4096
    Llog = M * bs
    g = torch.Generator().manual_seed(5)
    # logical blocks mapped to the top of the pool (and one around 2^18 blocks)
    table = (nblocks - 1 - torch.randperm(2 * M, generator=g)[: B * M]).view(B, M).to(torch.int32)
    table[0, 3] = 1 << 18
    ids = torch.randint(0, Llog, (B, SQ, 1, K), generator=g, dtype=torch.int32)
    ids[torch.rand(ids.shape, generator=g) < 0.05] = -1
    ids[..., :1] = torch.randint(0, Llog, (B, SQ, 1, 1), generator=g, dtype=torch.int32)
    kv_log = torch.randn(B, Llog, 1, 512, generator=g).bfloat16()
    kr_log = torch.randn(B, Llog, 1, 64, generator=g).bfloat16()
    q = torch.randn(B, SQ, H, 512, generator=g).bfloat16()
    qr = torch.randn(B, SQ, H, 64, generator=g).bfloat16()
    tag = "paged pool 2^25-64 rows"
    print(f"[{tag}] allocating {nblocks * bs * 1152 / 2 ** 30:.1f} GiB", flush=True)
    pool = torch.empty(nblocks, bs, 1, 512, dtype=torch.bfloat16, device="cuda")
    rpool = torch.empty(nblocks, bs, 1, 64, dtype=torch.bfloat16, device="cuda")
    pool[0] = 0      # a masked slot's gather reads pool row 0
    rpool[0] = 0
    blocks = table.view(-1).long().cuda()
    pool[blocks] = kv_log.view(B * M, bs, 1, 512).cuda()
    rpool[blocks] = kr_log.view(B * M, bs, 1, 64).cuda()
    print(f"[{tag}] launching", flush=True)
    got = dsa_amd.forward(q.cuda(), pool, qr.cuda(), rpool, ids.cuda(), block_table=table.cuda())
    torch.cuda.synchronize()
    del pool, rpool
    torch.cuda.empty_cache()
    ref = O.reference(q, kv_log, qr, kr_log, ids)
    _check(tag, got, ref)
