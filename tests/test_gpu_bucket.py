"""Row-range bucketing of the top-k indices (dsa_bucket_indices /
dsa_amd.bucket_indices), the pre-pass forward() runs for calls of 256
tokens or more.  No reference counterpart: the attention does not depend on
the order of a token's slots; the order only improves the gathers' L2
locality.

Checked bit for bit against the oracle's stable partition
(oracle.dsa_oracle.bucket_rows_ref) on ragged, tiny and maximal rows with
duplicates, -1, out-of-range and INT32_MIN entries and kv lengths at the
64-bucket boundaries; a prefill-sized forward equals the same call on
indices bucketed beforehand, bit for bit, leaves the caller's indices
untouched and matches the attention oracle.
"""
import pytest
import torch

import dsa_amd
from dsa_amd import api as A
from oracle import dsa_oracle as O
from _parity import check

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")


@pytest.mark.parametrize("B,SQ,K,L", [(1, 1, 1, 1), (2, 3, 7, 64), (1, 5, 64, 65), (3, 2, 100, 129),
                                      (1, 7, 2047, 5000), (2, 4, 2048, 8192), (1, 3, 4096, 100000),
                                      (1, 300, 2048, 32768), (1, 2, 4096, 2 ** 31 - 1)])
def test_bucketing_matches_oracle(B, SQ, K, L):
    g = torch.Generator().manual_seed(B * 100 + K)
    ids = torch.randint(0, min(L, 2 ** 30), (B, SQ, 1, K), generator=g, dtype=torch.int32)
    u = torch.rand(ids.shape, generator=g)
    ids[u < 0.1] = -1
    ids[(u >= 0.1) & (u < 0.15)] = min(L, 2 ** 31 - 1)
    ids[(u >= 0.15) & (u < 0.2)] = -(2 ** 31)
    d = torch.rand(ids.shape, generator=g) < 0.1
    ids[..., 1:][d[..., 1:]] = ids[..., :-1][d[..., 1:]]
    dev = ids.contiguous().cuda()
    keep = dev.clone()
    print(f"[bucket {B}x{SQ}x{K} L={L}]", flush=True)
    out = dsa_amd.bucket_indices(dev, L)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), O.bucket_rows_ref(ids, L))
    assert torch.equal(dev, keep)


def test_bucketing_rejects_what_it_cannot_take():
    ids = torch.zeros(1, 2, 1, 4097, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError):
        dsa_amd.bucket_indices(ids, 100)
    with pytest.raises(ValueError):
        dsa_amd.bucket_indices(ids[..., :100].contiguous().long(), 100)
    with pytest.raises(ValueError):
        dsa_amd.bucket_indices(ids[..., ::2], 100)
    with pytest.raises(ValueError):
        dsa_amd.bucket_indices(ids[..., :100].contiguous(), 0)


@pytest.mark.parametrize("H", [16, 128])
def test_prefill_forward_buckets_rows_first(H):
    B, SQ, L, K = 1, 260, 5000, 2048
    assert A.buckets_rows((B, SQ, H, L, K))
    g = torch.Generator().manual_seed(40 + H)
    q = torch.randn(B, SQ, H, 512, generator=g).bfloat16()
    kv = torch.randn(B, L, 1, 512, generator=g).bfloat16()
    qr = torch.randn(B, SQ, H, 64, generator=g).bfloat16()
    kr = torch.randn(B, L, 1, 64, generator=g).bfloat16()
    ids = torch.randint(0, L, (B, SQ, 1, K), generator=g, dtype=torch.int32)
    ids[torch.rand(ids.shape, generator=g) < 0.2] = -1
    ids[..., :1] = torch.randint(0, L, (B, SQ, 1, 1), generator=g, dtype=torch.int32)
    data = [t.cuda() for t in (q, kv, qr, kr, ids.contiguous())]
    keep = data[4].clone()
    print(f"[forward bucketed H={H}]", flush=True)
    got = dsa_amd.forward(*data)
    pre = dsa_amd.forward(*data[:4], O.bucket_rows_ref(ids, L).cuda())
    torch.cuda.synchronize()
    assert torch.equal(data[4], keep)
    for a, b in zip(got, pre):
        assert torch.equal(a, b)
    check(f"prefill bucketed rows H={H}", *got, O.reference(q, kv, qr, kr, ids))
