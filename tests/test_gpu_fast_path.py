"""The host fast path of dsa_amd.forward (dsa_amd/_fast*.so, built from
csrc/fast_forward.cpp): for a shape the Python path has planned on the
device, the C++ path's outputs equal the Python path's bit for bit; for
every input the Python path rejects it declines (returns None) before
allocating anything, so the Python path raises the reference's error.
No reference counterpart (host cost only).
"""
import pytest
import torch

import dsa_amd
from dsa_amd import api as A

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fast():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    module = A._fast_path()
    assert module is not None, "the fast path module is built by dsa_amd.build"
    return module


def _case(seed, B, SQ, H, L, K):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, SQ, H, 512, generator=g).bfloat16()
    kv = torch.randn(B, L, 1, 512, generator=g).bfloat16()
    qr = torch.randn(B, SQ, H, 64, generator=g).bfloat16()
    kr = torch.randn(B, L, 1, 64, generator=g).bfloat16()
    ids = torch.randint(-2, L + 2, (B, SQ, 1, K), generator=g, dtype=torch.int32)
    ids[..., :1] = torch.randint(0, L, (B, SQ, 1, 1), generator=g, dtype=torch.int32)
    return [t.cuda() for t in (q, kv, qr, kr, ids)]


SHAPES = [(8, 1, 128, 32768, 2048),   # C2's shape: split plan, merge kernel
          (2, 40, 128, 4096, 2048),   # no split (ping-pong)
          (3, 2, 48, 1000, 100),      # planner's plan, ragged TOPK
          (64, 2, 16, 8192, 2048)]    # an in-kernel-merge plan: never registered, always the Python path


@pytest.mark.parametrize("shape", SHAPES, ids=str)
def test_fast_path_equals_python_path(fast, shape, monkeypatch):
    data = _case(sum(shape), *shape)
    fast.clear_plans()
    assert fast.forward(*data) is None  # not planned yet
    first = dsa_amd.forward(*data)      # the Python path, which registers the plan
    taken = fast.forward(*data)
    fused = dsa_amd.select(shape).fused_merge
    print(f"[fast path {shape}] taken={taken is not None} fused={fused}", flush=True)
    assert (taken is None) == fused
    again = dsa_amd.forward(*data)      # the fast path when registered
    monkeypatch.setattr(A, "_fast_path", lambda: None)
    python = dsa_amd.forward(*data)
    torch.cuda.synchronize()
    for outs in ([taken] if taken is not None else []) + [again, first]:
        for a, b in zip(outs, python):
            assert a.shape == b.shape and a.dtype == b.dtype and torch.equal(a, b)


def test_fast_path_declines_every_rejected_input(fast):
    base = _case(5, 2, 3, 16, 300, 128)
    dsa_amd.forward(*base)  # plans and registers the shape
    torch.cuda.synchronize()
    assert fast.forward(*base) is not None
    cases = []
    for i, t in enumerate(base):
        cases.append((f"cpu-{i}", i, t.cpu()))
        cases.append((f"dtype-{i}", i, t.float() if i < 4 else t.long()))
        wide = torch.zeros(t.shape[:-1] + (2 * t.shape[-1],), dtype=t.dtype, device="cuda")
        cases.append((f"strided-{i}", i, wide[..., ::2]))
        cases.append((f"rank-{i}", i, t[0]))
        if i < 4:  # another TOPK is a valid call (the planner takes any)
            cases.append((f"width-{i}", i, torch.zeros(t.shape[:-1] + (t.shape[-1] + 1,), dtype=t.dtype,
                                                       device="cuda")))
        cases.append((f"empty-{i}", i, torch.zeros((0,) + tuple(t.shape[1:]), dtype=t.dtype, device="cuda")))
    cases.append(("heads-48", 0, torch.zeros(2, 3, 24, 512, dtype=torch.bfloat16, device="cuda")))
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    for name, i, t in cases:
        args = list(base)
        args[i] = t
        assert fast.forward(*args) is None, name
        assert torch.cuda.memory_allocated() == before, name
        with pytest.raises((ValueError, TypeError)):
            dsa_amd.forward(*args)
    print(f"[fast path] {len(cases)} rejected inputs declined with nothing allocated", flush=True)


def test_fast_path_declines_what_is_not_a_tensor(fast):
    """None (fp8 kv rows come without k_rope) or any other non-tensor goes to
    the Python path, which takes the fp8 call and raises for the rest."""
    base = _case(6, 2, 3, 16, 256, 128)
    dsa_amd.forward(*base)
    torch.cuda.synchronize()
    for i, bad in ((3, None), (4, base[4].tolist()), (0, 1.5), (1, "kv")):
        args = list(base)
        args[i] = bad
        assert fast.forward(*args) is None, (i, type(bad))
    # an fp8 call: the Python path, equal to the bf16 call on the dequantized rows
    from oracle import dsa_oracle as O
    rows = dsa_amd.quantize_kv_fp8(base[1], base[3])
    kv_deq, rope = O.dequant_fp8_rows(rows)
    got = dsa_amd.forward(base[0], rows, base[2], None, base[4])
    want = dsa_amd.forward(base[0], kv_deq.cuda(), base[2], rope.cuda(), base[4],
                           config=dsa_amd.plan_call((2, 3, 16, 256, 128), None, A._device_cus(base[0].device),
                                                    kv_fp8=True)[0])
    torch.cuda.synchronize()
    for a, b in zip(got, want):
        assert torch.equal(a, b)
