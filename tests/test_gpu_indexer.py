"""Parity of the lightning indexer kernels (dsa_amd.indexer*, through the C
ABI) with the CPU oracle.

* logits: against the FP32 oracle, max |diff| <= 1e-4 x max |logit| over the
  defined entries (s < length); bf16 inputs, FP32 accumulation on both sides;
* top-k: bit-exact against the oracle given the same logits (integer output),
  including ties, -0.0 / +0.0, -inf, rows shorter than TOPK, empty rows,
  constant rows, rows whose keys share one first-digit bin (no candidate
  compaction) and rows longer than the 65536 keys the kernel caches in LDS;
* end to end: the selected indices drive dsa_amd.forward, checked against the
  attention oracle on the same indices.
"""
import pytest
import torch

import dsa_amd
from _parity import check
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-4


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    torch.cuda.init()


def _inputs(seed, B, SQ, HI, L, lengths=None):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, SQ, HI, 128, generator=g).bfloat16()
    k = torch.randn(B, L, 128, generator=g).bfloat16()
    w = torch.randn(B, SQ, HI, generator=g) * 0.1
    if lengths is None:
        lengths = torch.randint(1, L + 1, (B, SQ), generator=g, dtype=torch.int32)
    return q, k, w, lengths.int().contiguous()


def _check_logits(tag, got, ref, lengths):
    length = ref.shape[-1]
    defined = torch.arange(length)[None, None, :] < lengths.clamp(0, length)[..., None].long()
    g, r = got.cpu()[defined], ref[defined]
    scale = r.abs().max().clamp_min(1e-30)
    err = ((g - r).abs().max() / scale).item()
    print(f"[{tag}] logits max-normalised error {err:.2e} over {int(defined.sum())} entries", flush=True)
    assert torch.isfinite(g).all(), tag
    assert err <= LOGIT_TOL, (tag, err)


LOGIT_CASES = [
    ("decode h64", 0, 4, 1, 64, 5000, None),
    ("mtp h32", 1, 3, 2, 32, 3000, None),
    ("prefill causal h64", 2, 1, 300, 64, 1024, "causal"),
    ("lengths 0 and > L", 3, 2, 5, 64, 700, "edge"),
    ("mtp h64", 4, 3, 2, 64, 4500, None),      # two waves per query (SQ * HI = 128)
    ("sq3 h32", 5, 2, 3, 32, 2100, None),      # two waves per query, one slot idle
    ("decode h32", 6, 5, 1, 32, 1500, None),   # four waves per query
]


@pytest.mark.parametrize("tag,seed,B,SQ,HI,L,mode", LOGIT_CASES, ids=[c[0] for c in LOGIT_CASES])
def test_indexer_logits_parity(tag, seed, B, SQ, HI, L, mode):
    lengths = None
    if mode == "causal":
        lengths = (L - SQ + 1 + torch.arange(SQ)).expand(B, SQ)
    elif mode == "edge":
        lengths = torch.tensor([[0, L, L + 9, 1, 65], [64, 63, 129, 700, 2]])
    q, k, w, lengths = _inputs(seed, B, SQ, HI, L, lengths)
    print(f"[{tag}] launching B={B} SQ={SQ} HI={HI} L={L}", flush=True)
    got = dsa_amd.indexer_logits(q.cuda(), k.cuda(), w.cuda(), lengths.cuda())
    torch.cuda.synchronize()
    _check_logits(tag, got, O.indexer_logits_ref(q, k, w, lengths), lengths)


TOPK_CASES = [
    ("ties", 10, 3, 4, 3000, 512, "ties"),
    ("short rows", 11, 2, 3, 600, 2048, None),
    ("long cached rows", 12, 1, 2, 40000, 2048, None),
    ("uncached rows", 14, 1, 2, 70000, 2048, None),
    ("signed zeros and -inf", 13, 1, 2, 5000, 1000, "zeros"),
    ("narrow values", 15, 2, 2, 20000, 2048, "narrow"),
    ("constant rows", 16, 1, 3, 3000, 700, "constant"),
    # more first-digit candidates than the segmented path keeps in LDS (8192)
    ("constant long rows", 17, 1, 2, 20000, 2048, "constant"),
    ("32 rows", 18, 8, 4, 9000, 2048, None),      # the most rows the segmented path takes
    ("64 rows", 19, 16, 4, 5000, 1024, None),     # one workgroup per row either way
]


@pytest.mark.parametrize("segmented", [True, False], ids=["segmented", "one-wg-per-row"])
@pytest.mark.parametrize("tag,seed,B,SQ,L,K,mode", TOPK_CASES, ids=[c[0] for c in TOPK_CASES])
def test_indexer_topk_bit_exact(tag, seed, B, SQ, L, K, mode, segmented):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(B, SQ, L, generator=g)
    lengths = torch.randint(0, L + 3, (B, SQ), generator=g, dtype=torch.int32)
    lengths[0, 0] = L
    if mode == "ties":
        logits = torch.randint(-3, 4, (B, SQ, L), generator=g).float()
    elif mode == "zeros":
        logits[..., ::3] = -0.0
        logits[..., 1::3] = 0.0
        logits[..., 2::7] = -float("inf")
        lengths[:] = L
    elif mode == "narrow":  # one first-digit bin holds every key: no candidate compaction
        logits = 1.0 + logits * 1e-6
    elif mode == "constant":
        logits = torch.full((B, SQ, L), 0.25)
    print(f"[{tag}] launching B={B} SQ={SQ} L={L} K={K} segmented={segmented}", flush=True)
    got = dsa_amd.indexer_topk(logits.cuda(), lengths.cuda(), K, segmented=segmented)
    torch.cuda.synchronize()
    ref = O.indexer_topk_ref(logits, lengths, K)
    assert torch.equal(got.cpu(), ref), tag


def test_indexer_end_to_end_into_attention():
    B, SQ, HI, L, K = 2, 2, 64, 4096, 2048
    q, k, w, lengths = _inputs(20, B, SQ, HI, L, torch.tensor([[4096, 3000], [2500, 4096]]))
    print("[indexer -> forward] launching", flush=True)
    logits = dsa_amd.indexer_logits(q.cuda(), k.cuda(), w.cuda(), lengths.cuda())
    idx = dsa_amd.indexer_topk(logits, lengths.cuda(), K)
    torch.cuda.synchronize()
    # the selection is exact on the kernel's own logits
    assert torch.equal(idx.cpu(), O.indexer_topk_ref(logits.cpu(), lengths, K))
    # and every chosen key scores at least the oracle's K-th best, up to the logit tolerance
    ref = O.indexer_logits_ref(q, k, w, lengths)
    for b in range(B):
        for t in range(SQ):
            chosen = idx[b, t, 0].cpu().long()
            chosen = chosen[chosen >= 0]
            kth = ref[b, t].topk(min(K, int(lengths[b, t]))).values[-1]
            tol = LOGIT_TOL * ref[b, t][torch.isfinite(ref[b, t])].abs().max()
            assert (ref[b, t, chosen] >= kth - 2 * tol).all()
    # the indices feed the sparse attention directly
    g = torch.Generator().manual_seed(21)
    qa = torch.randn(B, SQ, 128, 512, generator=g).bfloat16()
    kv = torch.randn(B, L, 1, 512, generator=g).bfloat16()
    qr = torch.randn(B, SQ, 128, 64, generator=g).bfloat16()
    kr = torch.randn(B, L, 1, 64, generator=g).bfloat16()
    out, mx, sm = dsa_amd.forward(qa.cuda(), kv.cuda(), qr.cuda(), kr.cuda(), idx)
    torch.cuda.synchronize()
    check("indexer -> forward", out, mx, sm, O.reference(qa, kv, qr, kr, idx.cpu()))
