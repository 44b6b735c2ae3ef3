"""Parity of the options beyond the reference's operator contract: a softmax
scale other than 1/24, and paged kv (block pools + block table).

Paged runs must equal the contiguous run on the same logical rows bit for bit
(the kernels compute exactly the same values; only the gather address
differs), and both are checked against the FP32 oracle at the tolerances of
tests/test_gpu_parity.py.
"""
import pytest
import torch

import dsa_amd
from dsa_amd import Tuning
from _parity import check
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu

_PP = dict(kv_waves=1, stages=4, mfma=16, pv_cols=128)
PLANS = [None, Tuning(128, 32, 1, stages=4), Tuning(128, 32, 3, stages=4), Tuning(64, 64, 2, kv_waves=2),
         Tuning(32, 64, 1, kv_waves=2, mfma=16), Tuning(16, 64, 3, kv_waves=4, mfma=16),
         Tuning(128, 32, 1, **_PP), Tuning(128, 32, 3, **_PP),
         Tuning(16, 32, 2, kv_waves=2, stages=4, mfma=16, pv_cols=128),
         Tuning(32, 32, 1, kv_waves=2, stages=4, mfma=16, pv_cols=128)]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    torch.cuda.init()


def _case(seed, B=2, SQ=3, H=128, L=4096, K=700):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, SQ, H, 512, generator=g).bfloat16()
    kv = torch.randn(B, L, 1, 512, generator=g).bfloat16()
    qr = torch.randn(B, SQ, H, 64, generator=g).bfloat16()
    kr = torch.randn(B, L, 1, 64, generator=g).bfloat16()
    ids = torch.randint(0, L, (B, SQ, 1, K), generator=g, dtype=torch.int32)
    u = torch.rand(ids.shape, generator=g)
    ids[u < 0.05] = -1
    ids[u > 0.97] = L + 11
    ids[..., :1] = torch.randint(0, L, (B, SQ, 1, 1), generator=g, dtype=torch.int32)
    d = torch.rand(ids.shape, generator=g) < 0.1
    ids[..., 1:][d[..., 1:]] = ids[..., :-1][d[..., 1:]]
    return q, kv, qr, kr, ids.contiguous()


def _paged(kv, kr, block_size, seed, holes=0):
    """Block pools holding kv / k_rope under a random block permutation plus
    spare blocks of noise; optionally `holes` table entries set to -1 and one
    set past the pool."""
    g = torch.Generator().manual_seed(seed)
    batch, length = kv.shape[:2]
    per = length // block_size
    blocks = batch * per + 5
    order = torch.randperm(blocks, generator=g)[: batch * per].view(batch, per)
    kv_pool = torch.randn(blocks, block_size, 1, 512, generator=g).bfloat16()
    kr_pool = torch.randn(blocks, block_size, 1, 64, generator=g).bfloat16()
    kv_pool[order.reshape(-1)] = kv.reshape(batch * per, block_size, 1, 512)
    kr_pool[order.reshape(-1)] = kr.reshape(batch * per, block_size, 1, 64)
    table = order.int().contiguous()
    if holes:
        flat = table.view(-1)
        pick = torch.randperm(flat.numel(), generator=g)[: holes + 1]
        flat[pick[:-1]] = -1
        flat[pick[-1]] = blocks + 7
    return kv_pool, kr_pool, table


def _check(tag, out, mx, sm, ref):
    return check(tag, out, mx, sm, ref)


@pytest.mark.parametrize("scale", [192 ** -0.5, 0.03, 1.0 / 24.0])
@pytest.mark.parametrize("config", [None, Tuning(32, 64, 1, kv_waves=2, mfma=16), Tuning(128, 32, 2, **_PP),
                                    Tuning(16, 32, 3, kv_waves=2, stages=4, mfma=16, pv_cols=128)], ids=str)
def test_scale_parity(scale, config):
    data = _case(1)
    print(f"[scale {scale:.5f} {config}] launching", flush=True)
    out, mx, sm = dsa_amd.forward(*(t.cuda() for t in data), config=config, scale=scale)
    torch.cuda.synchronize()
    _check(f"scale {scale:.5f}", out, mx, sm, O.reference(*data, scale=scale))


@pytest.mark.parametrize("config", PLANS, ids=str)
@pytest.mark.parametrize("block_size", [64, 16])
def test_paged_equals_contiguous_bitwise(config, block_size):
    q, kv, qr, kr, ids = _case(2)
    kv_pool, kr_pool, table = _paged(kv, kr, block_size, seed=3)
    print(f"[paged bs={block_size} {config}] launching", flush=True)
    dev = [t.cuda() for t in (q, kv, qr, kr, ids, kv_pool, kr_pool, table)]
    contiguous = dsa_amd.forward(dev[0], dev[1], dev[2], dev[3], dev[4], config=config)
    paged = dsa_amd.forward(dev[0], dev[5], dev[2], dev[6], dev[4], config=config, block_table=dev[7])
    torch.cuda.synchronize()
    for a, b in zip(contiguous, paged):
        assert torch.equal(a, b)
    _check(f"paged bs={block_size}", *paged, O.reference(q, kv, qr, kr, ids))


@pytest.mark.parametrize("H,config", [(16, None), (128, None), (16, Tuning(16, 64, 1, kv_waves=4, mfma=16))],
                         ids=str)
def test_paged_prefill_bucketed_equals_contiguous(H, config):
    """260 tokens: forward buckets each token's indices by logical row range
    first (the same order for the paged and the contiguous call, which then
    agree bit for bit)."""
    q, kv, qr, kr, ids = _case(12, B=1, SQ=260, H=H, L=4096, K=700)
    kv_pool, kr_pool, table = _paged(kv, kr, 64, seed=13)
    dev = [t.cuda() for t in (q, kv, qr, kr, ids, kv_pool, kr_pool, table)]
    print(f"[paged prefill H={H} {config}] launching", flush=True)
    contiguous = dsa_amd.forward(dev[0], dev[1], dev[2], dev[3], dev[4], config=config)
    paged = dsa_amd.forward(dev[0], dev[5], dev[2], dev[6], dev[4], config=config, block_table=dev[7])
    torch.cuda.synchronize()
    for a, b in zip(contiguous, paged):
        assert torch.equal(a, b)
    _check(f"paged prefill H={H}", *paged, O.reference(q, kv, qr, kr, ids))


@pytest.mark.parametrize("config", [None, Tuning(16, 64, 3, kv_waves=4, mfma=16)], ids=str)
def test_paged_holes_are_masked(config):
    q, kv, qr, kr, ids = _case(4)
    kv_pool, kr_pool, table = _paged(kv, kr, 64, seed=5, holes=6)
    _, _, ok = O.unpage(kv_pool, kr_pool, table)
    masked = O.mask_unbacked(ids, ok)
    dev = [t.cuda() for t in (q, kv, qr, kr, masked, kv_pool, kr_pool, table, ids)]
    print(f"[paged holes {config}] launching", flush=True)
    expect = dsa_amd.forward(dev[0], dev[1], dev[2], dev[3], dev[4], config=config)
    paged = dsa_amd.forward(dev[0], dev[5], dev[2], dev[6], dev[8], config=config, block_table=dev[7])
    torch.cuda.synchronize()
    for a, b in zip(expect, paged):
        assert torch.equal(a, b)
    _check("paged holes", *paged, O.reference(q, kv, qr, kr, masked))


# Block-table entries far outside the pool.  With 64-row blocks the 32-bit
# row product entry * 64 + offset wraps: (2^26 + 1) * 64 = 2^32 + 64 lands on
# pool row 64, (2^25 + 1) * 64 and INT32_MAX * 64 turn negative.  Each such
# slot must be masked like a -1 index (the reference masks by the raw index,
# dsa/workspace.py:254-257; a row without a block has no data to read).
FAR_ENTRIES = [2 ** 25 + 1, 2 ** 26 + 1, 2 ** 31 - 1, -(2 ** 31), -2]


@pytest.mark.parametrize("config", [None, Tuning(128, 32, 1, stages=4), Tuning(16, 64, 3, kv_waves=4, mfma=16),
                                    Tuning(128, 32, 1, **_PP),
                                    Tuning(32, 32, 2, kv_waves=2, stages=4, mfma=16, pv_cols=128)],
                         ids=str)
def test_paged_far_block_entries_are_masked(config):
    q, kv, qr, kr, ids = _case(8)
    kv_pool, kr_pool, table = _paged(kv, kr, 64, seed=9)
    g = torch.Generator().manual_seed(10)
    flat = table.view(-1)
    pick = torch.randperm(flat.numel(), generator=g)[: len(FAR_ENTRIES) + 1]
    for i, v in enumerate(FAR_ENTRIES):
        flat[pick[i]] = v
    flat[pick[-1]] = kv_pool.shape[0]  # one past the last block
    _, _, ok = O.unpage(kv_pool, kr_pool, table)
    masked = O.mask_unbacked(ids, ok)
    hit = (masked == -1) & (ids >= 0) & (ids < kv.shape[1])
    assert int(hit.sum()) > 0, "the far entries must be referenced by some slots"
    dev = [t.cuda() for t in (q, kv, qr, kr, masked, kv_pool, kr_pool, table, ids)]
    print(f"[paged far entries {config}] launching ({int(hit.sum())} slots on far blocks)", flush=True)
    expect = dsa_amd.forward(dev[0], dev[1], dev[2], dev[3], dev[4], config=config)
    paged = dsa_amd.forward(dev[0], dev[5], dev[2], dev[6], dev[8], config=config, block_table=dev[7])
    torch.cuda.synchronize()
    for a, b in zip(expect, paged):
        assert torch.equal(a, b)
    _check("paged far entries", *paged, O.reference(q, kv, qr, kr, masked))


def test_paged_with_scale_and_split_merge():
    q, kv, qr, kr, ids = _case(6, B=3, SQ=2, H=64, L=2048, K=2048)
    kv_pool, kr_pool, table = _paged(kv, kr, 32, seed=7)
    dq, dkv, dqr, dkr, dids, dtab = (t.cuda() for t in (q, kv_pool, qr, kr_pool, ids, table))
    scale = 0.07
    print("[paged + scale] launching", flush=True)
    out, mx, sm = dsa_amd.forward(dq, dkv, dqr, dkr, dids, block_table=dtab, scale=scale,
                                  config=Tuning(64, 64, 4, kv_waves=2))
    torch.cuda.synchronize()
    _check("paged + scale", out, mx, sm, O.reference(q, kv, qr, kr, ids, scale=scale))
