"""Every rejection of ``dsa_amd.forward`` happens before any allocation or
launch (reference: tools/check_host_api.py:43-54, 88-129, which records every
``torch.empty`` / ``empty_like`` through a TorchSpy and every kernel launch,
and requires each mutation of a valid call to raise with nothing recorded).

Here the spy replaces ``torch`` inside ``dsa_amd.api`` (recording every
allocating constructor) and the C library handle (recording every entry point
that enqueues work).  The CPU test covers the shape and device rejections
(CPU tensors stop at the device check); the GPU test covers every other
class -- dtypes, layout, cores, plans, scale, paged tables, W_UV weights and
arrival counters -- on real device tensors, and checks that the unmutated
call does allocate and launch (so the spy sees what it should).
"""
import pytest
import torch

import dsa_amd
from dsa_amd import Tuning, _lib
from dsa_amd import api as A

ALLOCATORS = ("empty", "empty_like", "empty_strided", "zeros", "zeros_like", "ones", "ones_like", "full",
              "full_like", "tensor", "randn")
ENQUEUING = ("dsa_fwd", "dsa_fwd_main", "dsa_fwd_opts", "dsa_fwd_main_opts", "dsa_merge", "dsa_merge_uv",
             "dsa_project_uv", "dsa_indexer_logits", "dsa_indexer_topk", "dsa_indexer_topk_ws", "dsa_bucket_indices")


class TorchSpy:
    """``torch`` with every allocating constructor recorded."""

    def __init__(self, events):
        self._events = events

    def __getattr__(self, name):
        attr = getattr(torch, name)
        if name not in ALLOCATORS:
            return attr

        def allocate(*args, **kwargs):
            self._events.append(("allocate", name))
            return attr(*args, **kwargs)
        return allocate


class LibSpy:
    """The C library with every entry point that enqueues work recorded
    (planning entry points pass through unrecorded: they touch no device)."""

    def __init__(self, real, events):
        self._real, self._events = real, events

    def __getattr__(self, name):
        fn = getattr(self._real, name)
        if name not in ENQUEUING:
            return fn

        def call(*args):
            self._events.append(("launch", name))
            return fn(*args)
        return call


@pytest.fixture
def spy(monkeypatch):
    events = []
    real_load = _lib.load
    monkeypatch.setattr(A, "torch", TorchSpy(events))
    monkeypatch.setattr(A._lib, "load", lambda: LibSpy(real_load(), events))
    # the C++ fast path allocates where the spy cannot see it: the Python
    # path here (tests/test_gpu_fast_path.py covers the fast path's refusals)
    monkeypatch.setattr(A, "_fast_path", lambda: None)
    return events


def _tensors(B=2, SQ=3, H=16, L=300, K=128, device="cpu"):
    return [torch.zeros(B, SQ, H, 512, dtype=torch.bfloat16, device=device),
            torch.zeros(B, L, 1, 512, dtype=torch.bfloat16, device=device),
            torch.zeros(B, SQ, H, 64, dtype=torch.bfloat16, device=device),
            torch.zeros(B, L, 1, 64, dtype=torch.bfloat16, device=device),
            torch.zeros(B, SQ, 1, K, dtype=torch.int32, device=device)]


def _shape_mutations(base, device):
    """Rank, width and empty-batch mutations of each input.  A different
    TOPK (the last dim of ``indices``) is a valid call here -- unlike the
    reference, whose shape-keyed table rejects unknown shapes, the planner
    takes any TOPK -- so indices get the rank and batch mutations only."""
    out = []
    for i, t in enumerate(base):
        widths = (t.shape[:-1] + (t.shape[-1] + 1,),) if i < 4 else ()
        for shape in (t.shape[:-1], *widths, (0,) + tuple(t.shape[1:])):
            args = list(base)
            args[i] = torch.zeros(shape, dtype=t.dtype, device=device)
            out.append((f"shape-{i}-{tuple(shape)}", args, {}, ValueError))
    return out


def _expect_rejected(spy, name, args, kwargs, exc):
    del spy[:]
    with pytest.raises(exc):
        dsa_amd.forward(*args, **kwargs)
    assert spy == [], (name, spy)


def test_cpu_rejections_allocate_and_launch_nothing(spy):
    base = _tensors()
    cases = _shape_mutations(base, "cpu")
    cases.append(("device-cpu", base, {}, ValueError))
    cases.append(("device-meta", _tensors(device="meta"), {}, ValueError))
    for name, args, kwargs, exc in cases:
        _expect_rejected(spy, name, args, kwargs, exc)


@pytest.mark.gpu
def test_gpu_rejections_allocate_and_launch_nothing(spy):
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    base = _tensors(device="cuda")
    for t in base[:4]:
        t.normal_()
    base[4].copy_(torch.randint(0, 300, base[4].shape, dtype=torch.int32))
    # the unmutated call allocates its outputs and launches: the spy sees both
    del spy[:]
    dsa_amd.forward(*base)
    torch.cuda.synchronize()
    assert ("launch", "dsa_fwd") in spy and any(e[0] == "allocate" for e in spy), spy

    cases = _shape_mutations(base, "cuda")
    for i, t in enumerate(base):
        args = list(base)
        args[i] = t.cpu()
        cases.append((f"device-{i}", args, {}, ValueError))
        args = list(base)
        args[i] = t.float() if i < 4 else t.long()
        cases.append((f"dtype-{i}", args, {}, ValueError))
        args = list(base)
        wide = torch.zeros(t.shape[:-1] + (2 * t.shape[-1],), dtype=t.dtype, device="cuda")
        args[i] = wide[..., ::2]
        cases.append((f"contiguous-{i}", args, {}, ValueError))
    for core in (0, -1, True, 1.5, "28"):
        cases.append((f"cores-{core!r}", base, {"cores": core}, ValueError))
    for name, cfg in (("bm", Tuning(48, 64, 1, mfma=16)), ("split", Tuning(16, 64, 3, kv_waves=4, mfma=16)),
                      ("kv_waves", Tuning(16, 64, 1, kv_waves=2, mfma=16)),
                      ("fused-wide", Tuning(64, 64, 2, kv_waves=2, mfma=32, fused_merge=True))):
        cases.append((f"config-{name}", base, {"config": cfg}, ValueError))
    cases.append(("config-type", base, {"config": {}}, TypeError))
    cases.append(("config-tuple", base, {"config": (16, 64, 1)}, TypeError))
    for bad, exc in (("0.1", TypeError), (-1.0, ValueError), (float("nan"), ValueError)):
        cases.append((f"scale-{bad!r}", base, {"scale": bad}, exc))
    cases.append(("block_table-shape", base, {"block_table": torch.zeros(3, 2, dtype=torch.int32, device="cuda")},
                  ValueError))
    pools = [base[0], base[1].view(10, 60, 1, 512), base[2], base[3].view(10, 60, 1, 64), base[4]]
    cases.append(("block_table-dtype", pools, {"block_table": torch.zeros(2, 5, dtype=torch.int64, device="cuda")},
                  ValueError))
    w = torch.zeros(16, 128, 512, dtype=torch.bfloat16, device="cuda")
    cases.append(("w_uv-heads", base, {"w_uv": w[:8]}, ValueError))
    cases.append(("w_uv-dv", base, {"w_uv": w[:, :100]}, ValueError))
    cases.append(("w_uv-dtype", base, {"w_uv": w.float()}, ValueError))
    fused = Tuning(16, 64, 2, kv_waves=4, mfma=16, fused_merge=True)
    cases.append(("arrivals-dtype", base, {"config": fused,
                                           "arrivals": torch.zeros(6, dtype=torch.int64, device="cuda")}, ValueError))
    cases.append(("arrivals-small", base, {"config": fused,
                                           "arrivals": torch.zeros(5, dtype=torch.int32, device="cuda")}, ValueError))
    cases.append(("arrivals-device", base, {"config": fused, "arrivals": torch.zeros(6, dtype=torch.int32)},
                  ValueError))
    # fp8 kv rows with a plan whose kernels read bf16 rows only
    rows = torch.zeros(2, 300, 1, 656, dtype=torch.uint8, device="cuda")
    fp8_args = [base[0], rows, base[2], None, base[4]]
    cases.append(("config-fp8-pv_cols", fp8_args, {"config": Tuning(16, 64, 2, kv_waves=4, mfma=16, pv_cols=128)},
                  ValueError))
    for name, args, kwargs, exc in cases:
        _expect_rejected(spy, name, args, kwargs, exc)
    print(f"[no allocation before rejection] {len(cases)} mutations rejected with nothing allocated or launched",
          flush=True)


def test_spy_records_what_it_should(spy):
    # planted: an allocation and a launch made through the spied names are seen
    A.torch.empty(3)
    assert spy == [("allocate", "empty")]
    with pytest.raises(TypeError):
        A._lib.load().dsa_merge(None)
    assert spy[-1] == ("launch", "dsa_merge")
