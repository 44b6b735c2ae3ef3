"""In-kernel split merge (plan.fused_merge): the last workgroup of each
(token, head group) merges the partials inside the main kernel.

The two paths share the merge arithmetic, so the fused call must equal the
two-launch call (main kernel + merge kernel) bit for bit, on every plan,
input family and call sequence; one case per plan family is also checked
against the FP32 oracle.  The arrival counters must be back at zero after
every call.
"""
import ctypes
import dataclasses

import pytest
import torch

import dsa_amd
from dsa_amd import Tuning, _lib
from dsa_amd import api as A
from _parity import check
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu



@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    torch.cuda.init()


def _case(seed, B=2, SQ=3, H=128, L=4096, K=2048, masked_tail=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, SQ, H, 512, generator=g).bfloat16()
    kv = torch.randn(B, L, 1, 512, generator=g).bfloat16()
    qr = torch.randn(B, SQ, H, 64, generator=g).bfloat16()
    kr = torch.randn(B, L, 1, 64, generator=g).bfloat16()
    ids = torch.randint(0, L, (B, SQ, 1, K), generator=g, dtype=torch.int32)
    u = torch.rand(ids.shape, generator=g)
    ids[u < 0.05] = -1
    ids[u > 0.97] = L + 3
    ids[..., :1] = torch.randint(0, L, (B, SQ, 1, 1), generator=g, dtype=torch.int32)
    if masked_tail:  # every split past the first quarter sees only masked slots
        ids[..., K // 4:] = -1
    return q, kv, qr, kr, ids.contiguous()


def _fused(cfg: Tuning) -> Tuning:
    return dataclasses.replace(cfg, fused_merge=True)


def _counters_zero():
    torch.cuda.synchronize()
    for buf in A._arrivals.values():
        assert int(buf.abs().sum()) == 0


def _check_oracle(tag, out, mx, sm, ref):
    return check(tag, out, mx, sm, ref)


PLANS = [Tuning(16, 64, 2, kv_waves=4, mfma=16), Tuning(16, 64, 3, kv_waves=4, mfma=16),
         Tuning(16, 64, 5, kv_waves=4, mfma=16), Tuning(16, 64, 16, kv_waves=4, mfma=16),
         Tuning(32, 64, 2, kv_waves=2, mfma=16), Tuning(32, 64, 8, kv_waves=2, mfma=16),
         Tuning(64, 64, 4, kv_waves=1, mfma=16), Tuning(64, 64, 7, kv_waves=1, mfma=16),
         Tuning(16, 64, 2, kv_waves=4, mfma=16, pv_cols=128), Tuning(16, 64, 5, kv_waves=4, mfma=16, pv_cols=128),
         # specialised waves (16 heads, 32-row tiles): the PV waves merge in the last workgroup
         Tuning(16, 32, 2, kv_waves=2, stages=4, mfma=16, pv_cols=128),
         Tuning(16, 32, 7, kv_waves=2, stages=4, mfma=16, pv_cols=128),
         Tuning(16, 32, 16, kv_waves=2, stages=4, mfma=16, pv_cols=128)]


@pytest.mark.parametrize("config", PLANS, ids=str)
def test_fused_equals_two_launches_bitwise(config):
    data = _case(11)
    dev = [t.cuda() for t in data]
    print(f"[fused {config}] launching", flush=True)
    two = dsa_amd.forward(*dev, config=config)
    one, launches = dsa_amd.forward(*dev, config=_fused(config), return_kernels=True)
    assert len(launches) == 1
    torch.cuda.synchronize()
    for a, b in zip(two, one):
        assert torch.equal(a, b)
    _counters_zero()
    if config.split in (2, 8, 7):
        _check_oracle(f"fused {config}", *one, O.reference(*data))


def test_fused_repeated_calls_reset_counters():
    cfg = _fused(Tuning(16, 64, 4, kv_waves=4, mfma=16))
    for i, shape in enumerate([(4, 2, 16, 8192), (2, 3, 32, 4096), (4, 2, 16, 8192)]):
        B, SQ, H, L = shape
        data = [t.cuda() for t in _case(20 + i, B=B, SQ=SQ, H=H, L=L)]
        print(f"[fused repeat {i} {shape}] launching", flush=True)
        one = dsa_amd.forward(*data, config=cfg)
        two = dsa_amd.forward(*data, config=Tuning(16, 64, 4, kv_waves=4, mfma=16))
        torch.cuda.synchronize()
        for a, b in zip(two, one):
            assert torch.equal(a, b), (i, shape)
        _counters_zero()


def test_fused_many_groups():
    # 256 tokens x 1 head group x 2 splits: 512 workgroups, 256 counters
    data = _case(30, B=128, SQ=2, H=16, L=8192)
    dev = [t.cuda() for t in data]
    cfg = Tuning(16, 64, 2, kv_waves=4, mfma=16)
    print("[fused many groups] launching", flush=True)
    two = dsa_amd.forward(*dev, config=cfg)
    one = dsa_amd.forward(*dev, config=_fused(cfg))
    torch.cuda.synchronize()
    for a, b in zip(two, one):
        assert torch.equal(a, b)
    _counters_zero()


def test_fused_with_masked_splits():
    data = _case(31, masked_tail=True)
    dev = [t.cuda() for t in data]
    cfg = Tuning(16, 64, 8, kv_waves=4, mfma=16)
    print("[fused masked splits] launching", flush=True)
    two = dsa_amd.forward(*dev, config=cfg)
    one = dsa_amd.forward(*dev, config=_fused(cfg))
    torch.cuda.synchronize()
    for a, b in zip(two, one):
        assert torch.equal(a, b)
    _check_oracle("fused masked splits", *one, O.reference(*data))
    _counters_zero()


def test_fused_fp8_and_paged():
    q, kv, qr, kr, ids = _case(32, H=64)
    rows = dsa_amd.quantize_kv_fp8(kv, kr)
    cfg = Tuning(32, 64, 4, kv_waves=2, mfma=16)
    dq, dqr, dids, drows = (t.cuda() for t in (q, qr, ids, rows))
    print("[fused fp8] launching", flush=True)
    two = dsa_amd.forward(dq, drows, dqr, None, dids, config=cfg)
    one = dsa_amd.forward(dq, drows, dqr, None, dids, config=_fused(cfg))
    torch.cuda.synchronize()
    for a, b in zip(two, one):
        assert torch.equal(a, b)
    # paged bf16 rows, 64-row blocks in reverse order
    B, L = kv.shape[:2]
    per = L // 64
    order = torch.arange(B * per).flip(0).view(B, per)
    kv_pool = torch.empty(B * per, 64, 1, 512, dtype=kv.dtype)
    kr_pool = torch.empty(B * per, 64, 1, 64, dtype=kr.dtype)
    kv_pool[order.reshape(-1)] = kv.reshape(B * per, 64, 1, 512)
    kr_pool[order.reshape(-1)] = kr.reshape(B * per, 64, 1, 64)
    dev = [t.cuda() for t in (kv, kr, kv_pool, kr_pool, order.int().contiguous())]
    print("[fused paged] launching", flush=True)
    two = dsa_amd.forward(dq, dev[0], dqr, dev[1], dids, config=cfg)
    one = dsa_amd.forward(dq, dev[2], dqr, dev[3], dids, config=_fused(cfg), block_table=dev[4])
    torch.cuda.synchronize()
    for a, b in zip(two, one):
        assert torch.equal(a, b)
    _counters_zero()


def test_fused_through_c_abi_with_caller_counters():
    B, SQ, H, L, K = 3, 2, 32, 4096, 2048
    data = _case(33, B=B, SQ=SQ, H=H, L=L, K=K)
    q, kv, qr, kr, ids = (t.cuda() for t in data)
    lib = _lib.load()
    plan = _lib.DsaPlan(16, 64, 6, 4, 2, 16, 1)
    po, pml = ctypes.c_int64(), ctypes.c_int64()
    assert lib.dsa_partial_elems(ctypes.byref(plan), B, SQ, H, ctypes.byref(po), ctypes.byref(pml)) == 0
    dev = q.device
    part_o = torch.empty(po.value, device=dev, dtype=torch.float32)
    part_m = torch.empty(pml.value, device=dev, dtype=torch.float32)
    part_l = torch.empty(pml.value, device=dev, dtype=torch.float32)
    counters = torch.zeros(B * SQ * (H // 16), device=dev, dtype=torch.int32)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def call(opts):
        out = torch.empty_like(q)
        mx = torch.empty(B, 1, SQ, H, device=dev, dtype=torch.float32)
        sm = torch.empty_like(mx)
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        rc = lib.dsa_fwd_opts(p(q), p(kv), p(qr), p(kr), p(ids), p(out), p(mx), p(sm),
                              p(part_o), p(part_m), p(part_l), B, SQ, H, L, K,
                              ctypes.byref(opts), ctypes.byref(plan), stream)
        assert rc == 0, lib.dsa_last_error()
        return out, mx, sm

    print("[fused c-abi] launching", flush=True)
    fused = call(_lib.DsaFwdOptions(arrivals=counters.data_ptr()))
    again = call(_lib.DsaFwdOptions(arrivals=counters.data_ptr()))
    fallback = call(_lib.DsaFwdOptions())  # fused plan without counters: the merge kernel runs
    torch.cuda.synchronize()
    assert int(counters.abs().sum()) == 0
    for a, b, c in zip(fused, again, fallback):
        assert torch.equal(a, b) and torch.equal(a, c)
    _check_oracle("fused c-abi", *fused, O.reference(*data))


def _growing_case(seed, B=1, SQ=2, H=128, L=4096, K=2048):
    """kv rows ramp 0 -> 4 along L and the indices are sorted, so the scores
    rise by far more than 2^64 along the slots: a workgroup's first tiles sit
    far below its max and it recomputes its range (second pass)."""
    g = torch.Generator().manual_seed(seed)
    q = (1.0 + 0.1 * torch.randn(B, SQ, H, 512, generator=g)).bfloat16()
    kv = (torch.linspace(0.0, 4.0, L).view(1, L, 1, 1) + 0.1 * torch.randn(B, L, 1, 512, generator=g)).bfloat16()
    qr = (0.1 * torch.randn(B, SQ, H, 64, generator=g)).bfloat16()
    kr = (0.1 * torch.randn(B, L, 1, 64, generator=g)).bfloat16()
    ids = torch.stack([torch.randperm(L, generator=g)[:K].sort().values for _ in range(B * SQ)])
    return q, kv, qr, kr, ids.view(B, SQ, 1, K).int().contiguous()


def test_fused_with_second_pass():
    data = _growing_case(12)
    dev = [t.cuda() for t in data]
    for cfg in (Tuning(16, 64, 4, kv_waves=4, mfma=16), Tuning(32, 64, 2, kv_waves=2, mfma=16)):
        print(f"[fused second pass {cfg}] launching", flush=True)
        two = dsa_amd.forward(*dev, config=cfg)
        one = dsa_amd.forward(*dev, config=_fused(cfg))
        torch.cuda.synchronize()
        for a, b in zip(two, one):
            assert torch.equal(a, b), cfg
        _check_oracle(f"fused second pass {cfg}", *one, O.reference(*data))
    _counters_zero()


@pytest.mark.parametrize("K,split", [(100, 2), (2047, 3), (70, 2)])
def test_fused_ragged_topk(K, split):
    data = _case(40 + K, B=2, SQ=2, H=48, L=3000, K=K)
    dev = [t.cuda() for t in data]
    cfg = Tuning(16, 64, split, kv_waves=4, mfma=16)
    print(f"[fused ragged K={K} split={split}] launching", flush=True)
    two = dsa_amd.forward(*dev, config=cfg)
    one = dsa_amd.forward(*dev, config=_fused(cfg))
    torch.cuda.synchronize()
    for a, b in zip(two, one):
        assert torch.equal(a, b)
    _check_oracle(f"fused ragged K={K}", *one, O.reference(*data))
    _counters_zero()
