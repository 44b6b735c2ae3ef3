"""Parity of fp8 kv cache rows (656 bytes: 512 OCP e4m3 latent values, 4 fp32
scales, 64 bf16 rope values; written by dsa_amd.quantize_kv_fp8).

The kernels expand every latent value to bf16(fp32(e4m3) * scale) before the
MFMAs (one scaled conversion per two values when a wave's scales are all
powers of two, the exact same value), so an fp8 run must equal, bit for
bit, the bf16 run on the kv the
oracle dequantizes from the same rows (oracle.dequant_fp8_rows) with the same
plan; both are checked against the FP32 oracle at the tolerances of
tests/test_gpu_parity.py.  Paged fp8 runs equal contiguous ones bit for bit.
"""
import pytest
import torch

import dsa_amd
from dsa_amd import Tuning
from _parity import check
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu

PLANS = [Tuning(16, 64, 1, kv_waves=4, mfma=16), Tuning(16, 64, 5, kv_waves=4, mfma=16),
         Tuning(32, 64, 1, kv_waves=2, mfma=16), Tuning(32, 64, 8, kv_waves=2, mfma=16),
         Tuning(64, 64, 1, mfma=16), Tuning(64, 64, 3, mfma=16)]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    torch.cuda.init()


def _case(seed, B=2, SQ=2, H=128, L=4096, K=2048):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, SQ, H, 512, generator=g).bfloat16()
    kv = (torch.randn(B, L, 1, 512, generator=g) * 2).bfloat16()
    qr = torch.randn(B, SQ, H, 64, generator=g).bfloat16()
    kr = torch.randn(B, L, 1, 64, generator=g).bfloat16()
    ids = torch.randint(0, L, (B, SQ, 1, K), generator=g, dtype=torch.int32)
    u = torch.rand(ids.shape, generator=g)
    ids[u < 0.05] = -1
    ids[u > 0.97] = L + 3
    ids[..., :1] = torch.randint(0, L, (B, SQ, 1, 1), generator=g, dtype=torch.int32)
    return q, kv, qr, kr, ids.contiguous()


def _check(tag, out, mx, sm, ref):
    return check(tag, out, mx, sm, ref)


@pytest.mark.parametrize("pow2", [True, False], ids=["pow2-scales", "fp32-scales"])
@pytest.mark.parametrize("config", [None] + PLANS, ids=str)
def test_fp8_rows_equal_bf16_on_dequantized_kv(config, pow2):
    q, kv, qr, kr, ids = _case(1)
    rows = dsa_amd.quantize_kv_fp8(kv.cuda(), kr.cuda(), pow2_scales=pow2)
    kv_deq, rope = O.dequant_fp8_rows(rows)
    plan = config if config is not None else dsa_amd.plan_call(tuple(q.shape[:3]) + (kv.shape[1], ids.shape[-1]),
                                                               None, 256, kv_fp8=True)[0]
    print(f"[fp8 {plan}] launching", flush=True)
    dq, dqr, dids = q.cuda(), qr.cuda(), ids.cuda()
    fp8 = dsa_amd.forward(dq, rows, dqr, None, dids, config=config)
    bf16 = dsa_amd.forward(dq, kv_deq.cuda(), dqr, rope.cuda(), dids, config=plan)
    torch.cuda.synchronize()
    for a, b in zip(fp8, bf16):
        assert torch.equal(a, b)
    _check(f"fp8 {plan}", *fp8, O.reference(q, kv_deq, qr, rope, ids))


@pytest.mark.parametrize("shape", [(1, 1, 128, 8192, 2048), (4, 2, 16, 8192, 2048)])
def test_fp8_decode_shapes_with_scale(shape):
    B, SQ, H, L, K = shape
    q, kv, qr, kr, ids = _case(2, B, SQ, H, L, K)
    rows = dsa_amd.quantize_kv_fp8(kv.cuda(), kr.cuda())
    kv_deq, rope = O.dequant_fp8_rows(rows)
    scale = 192 ** -0.5
    print(f"[fp8 {shape} scale] launching", flush=True)
    out = dsa_amd.forward(q.cuda(), rows, qr.cuda(), None, ids.cuda(), scale=scale)
    torch.cuda.synchronize()
    _check(f"fp8 {shape} scale", *out, O.reference(q, kv_deq, qr, rope, ids, scale=scale))


@pytest.mark.parametrize("block_size", [64, 16])
def test_fp8_paged_equals_contiguous_bitwise(block_size):
    q, kv, qr, kr, ids = _case(3)
    rows = dsa_amd.quantize_kv_fp8(kv, kr)  # [B, L, 1, 656] on the CPU
    g = torch.Generator().manual_seed(4)
    batch, length = rows.shape[:2]
    per = length // block_size
    blocks = batch * per + 3
    order = torch.randperm(blocks, generator=g)[: batch * per].view(batch, per)
    pool = torch.randint(0, 120, (blocks, block_size, 1, 656), generator=g, dtype=torch.uint8)  # finite noise
    pool[order.reshape(-1)] = rows.reshape(batch * per, block_size, 1, 656)
    table = order.int().contiguous()
    print(f"[fp8 paged bs={block_size}] launching", flush=True)
    dq, dqr, dids = q.cuda(), qr.cuda(), ids.cuda()
    contiguous = dsa_amd.forward(dq, rows.cuda(), dqr, None, dids)
    paged = dsa_amd.forward(dq, pool.cuda(), dqr, None, dids, block_table=table.cuda())
    torch.cuda.synchronize()
    for a, b in zip(contiguous, paged):
        assert torch.equal(a, b)
    kv_deq, rope = O.dequant_fp8_rows(rows)
    _check(f"fp8 paged bs={block_size}", *paged, O.reference(q, kv_deq, qr, rope, ids))


def test_fp8_rejects_wide_plans():
    q, kv, qr, kr, ids = _case(5, 1, 1, 128, 1024, 256)
    rows = dsa_amd.quantize_kv_fp8(kv.cuda(), kr.cuda())
    with pytest.raises(ValueError, match="narrow"):
        dsa_amd.forward(q.cuda(), rows, qr.cuda(), None, ids.cuda(), config=Tuning(128, 32, 1, stages=4))
    # column-split PV (pv_cols 128) reads bf16 rows only
    with pytest.raises(ValueError, match="narrow"):
        dsa_amd.forward(q.cuda(), rows, qr.cuda(), None, ids.cuda(),
                        config=Tuning(16, 64, 2, kv_waves=4, mfma=16, pv_cols=128))
