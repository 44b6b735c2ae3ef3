"""dsa_fwd_noalloc: the forward call that allocates nothing (split partials
and arrival counters in the library's static scratch array), checked against
dsa_fwd_opts -- the same call with caller-allocated partials and counters --
through the C ABI, bit for bit, on two calls in a row with the second one
smaller (so stale partials of the first call left in the scratch must not
leak into the second).  No reference counterpart: it exists for callers that
cannot allocate (graph capture, serving loops).

CPU part: every rejection (partials beyond the scratch, caller counters,
a bad plan) happens before any HIP call.
"""
import ctypes

import pytest
import torch

from dsa_amd import Tuning, _lib
from oracle import dsa_oracle as O
from _parity import check

CAP = 32 * 1024 * 1024  # DSA_NOALLOC_PARTIAL_BYTES


def _fake_call(lib, plan, opts=None, shape=(1, 1, 16, 4096, 2048)):
    """dsa_fwd_noalloc with fake (never dereferenced) pointers: the call must
    be rejected during validation."""
    fake = ctypes.c_void_p(1 << 20)
    B, SQ, H, L, K = shape
    return lib.dsa_fwd_noalloc(fake, fake, fake, fake, fake, fake, fake, fake, B, SQ, H, L, K,
                               None if opts is None else ctypes.byref(opts), ctypes.byref(plan), None)


def test_noalloc_rejections_before_any_launch():
    lib = _lib.load()
    # 64 tokens x 128 heads x split 16: 269 MB of partials, beyond the scratch
    big = _lib.DsaPlan(32, 64, 16, 2, 2, 16, 0)
    assert _fake_call(lib, big, shape=(64, 1, 128, 32768, 2048)) < 0
    assert b"scratch holds" in lib.dsa_last_error()
    # the caller's arrival counters are not taken: the counters are in the scratch
    fused = _lib.DsaPlan(16, 64, 2, 4, 2, 16, 1)
    assert _fake_call(lib, fused, _lib.DsaFwdOptions(arrivals=1 << 20)) < 0
    assert b"arrivals" in lib.dsa_last_error()
    # an invalid plan is rejected as by dsa_fwd_opts
    assert _fake_call(lib, _lib.DsaPlan(48, 64, 1, 1, 2, 16, 0)) < 0
    # the size in the message is the header's: rows * 512 * 4 + 2 * rows * 4
    # bytes, each array rounded up to 256 bytes
    rows = 64 * 16 * 128
    need = -(-rows * 2048 // 256) * 256 + 2 * (-(-rows * 4 // 256) * 256)
    assert _fake_call(lib, big, shape=(64, 1, 128, 32768, 2048)) < 0
    assert need > CAP and str(need).encode() in lib.dsa_last_error()


def _case(seed, B, SQ, H, L, K):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, SQ, H, 512, generator=g).bfloat16()
    kv = torch.randn(B, L, 1, 512, generator=g).bfloat16()
    qr = torch.randn(B, SQ, H, 64, generator=g).bfloat16()
    kr = torch.randn(B, L, 1, 64, generator=g).bfloat16()
    ids = torch.randint(0, L, (B, SQ, 1, K), generator=g, dtype=torch.int32)
    ids[torch.rand(ids.shape, generator=g) < 0.05] = -1
    ids[..., :1] = torch.randint(0, L, (B, SQ, 1, 1), generator=g, dtype=torch.int32)
    return [t.cuda() for t in (q, kv, qr, kr, ids.contiguous())]


def _outputs(q):
    B, SQ, H, _ = q.shape
    return (torch.empty_like(q), torch.empty((B, 1, SQ, H), device=q.device, dtype=torch.float32),
            torch.empty((B, 1, SQ, H), device=q.device, dtype=torch.float32))


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _noalloc(lib, data, plan, stream):
    q, kv, qr, kr, ids = data
    B, SQ, H, _ = q.shape
    out = _outputs(q)
    rc = lib.dsa_fwd_noalloc(*map(_p, data), *map(_p, out), B, SQ, H, kv.shape[1], ids.shape[-1], None,
                             None if plan is None else ctypes.byref(plan.to_c()), stream)
    _lib.check(rc, "dsa_fwd_noalloc")
    return out


def _with_buffers(lib, data, plan, stream):
    """dsa_fwd_opts with caller-allocated partials and arrival counters."""
    q, kv, qr, kr, ids = data
    B, SQ, H, _ = q.shape
    out = _outputs(q)
    split = plan.split
    po = torch.empty((B, SQ, split, H, 512), device=q.device, dtype=torch.float32)
    pm = torch.empty((B, SQ, split, H), device=q.device, dtype=torch.float32)
    pl = torch.empty_like(pm)
    counters = torch.zeros(B * SQ * (H // plan.bm), device=q.device, dtype=torch.int32)
    opts = _lib.DsaFwdOptions(arrivals=counters.data_ptr())
    rc = lib.dsa_fwd_opts(*map(_p, data), *map(_p, out), _p(po), _p(pm), _p(pl), B, SQ, H, kv.shape[1],
                          ids.shape[-1], ctypes.byref(opts), ctypes.byref(plan.to_c()), stream)
    _lib.check(rc, "dsa_fwd_opts")
    return out


# (first shape, second smaller shape) as (B, SQ, H, L, K), and the plan
CASES = [
    (((8, 1, 128, 8192, 2048), (3, 1, 128, 4096, 1024)), Tuning(32, 64, 8, kv_waves=2, mfma=16)),   # merge kernel
    (((16, 2, 16, 8192, 2048), (5, 2, 16, 4096, 2000)), Tuning(16, 64, 2, kv_waves=4, mfma=16, fused_merge=True)),
    (((4, 2, 64, 8192, 2048), (2, 1, 64, 4096, 700)), Tuning(64, 64, 4, kv_waves=2)),               # wide, split 4
    (((2, 40, 128, 8192, 2048), (1, 7, 128, 2048, 512)), Tuning(128, 32, 1, stages=4)),              # no split
    (((2, 16, 128, 8192, 2048), (1, 5, 128, 4096, 700)),
     Tuning(128, 32, 2, kv_waves=1, stages=4, mfma=16, pv_cols=128)),                                # ping-pong, split 2
    (((8, 1, 128, 32768, 2048), (3, 1, 128, 4096, 1024)),
     Tuning(32, 32, 8, kv_waves=2, stages=4, mfma=16, pv_cols=128)),                                 # specialised waves (C2's)
    (((16, 2, 16, 8192, 2048), (5, 2, 16, 4096, 2000)),
     Tuning(16, 32, 2, kv_waves=2, stages=4, mfma=16, pv_cols=128, fused_merge=True)),               # ... merged in the kernel
]


@pytest.mark.gpu
@pytest.mark.parametrize("shapes,plan", CASES, ids=lambda v: str(v))
def test_noalloc_equals_caller_buffers_twice(shapes, plan):
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for i, shape in enumerate(shapes):
        data = _case(100 + i, *shape)
        print(f"[noalloc {plan}] call {i} shape={shape}", flush=True)
        got = _noalloc(lib, data, plan, stream)
        want = _with_buffers(lib, data, plan, stream)
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b), (plan, i, shape)


@pytest.mark.gpu
def test_noalloc_plans_within_the_scratch():
    """plan NULL: the planner keeps to splits whose partials fit.  64 decode
    tokens of 128 heads: checked against the oracle, twice in a row."""
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for i, shape in enumerate(((64, 1, 128, 8192, 2048), (16, 1, 128, 8192, 1536))):
        data = _case(200 + i, *shape)
        print(f"[noalloc planner] call {i} shape={shape}", flush=True)
        out, mx, sm = _noalloc(lib, data, None, stream)
        torch.cuda.synchronize()
        check(f"noalloc planner {shape}", out, mx, sm, O.reference(*[t.cpu() for t in data]))


def _paged(data, block_size, seed):
    """The same logical inputs with kv / k_rope in block pools under a random
    block permutation: (data with pools, options with the block table)."""
    q, kv, qr, kr, ids = data
    B, L = kv.shape[:2]
    per = L // block_size
    perm = torch.randperm(B * per, generator=torch.Generator().manual_seed(seed)).cuda()
    kv_pool = torch.empty((B * per, block_size, 1, 512), device="cuda", dtype=kv.dtype)
    kr_pool = torch.empty((B * per, block_size, 1, 64), device="cuda", dtype=kr.dtype)
    kv_pool[perm] = kv.view(B * per, block_size, 1, 512)
    kr_pool[perm] = kr.view(B * per, block_size, 1, 64)
    table = perm.view(B, per).int().contiguous()
    opts = dict(block_size=block_size, max_blocks=per, num_blocks=B * per, block_table=table.data_ptr())
    return [q, kv_pool, qr, kr_pool, ids], opts, table


def _call(lib, name, data, plan, length, opts, stream, out, part=None):
    """One dsa_fwd_noalloc or dsa_fwd_opts call into preallocated outputs."""
    q, kv, qr, kr, ids = data
    B, SQ, H, _ = q.shape
    o = None if opts is None else ctypes.byref(opts)
    if name == "noalloc":
        rc = lib.dsa_fwd_noalloc(*map(_p, data), *map(_p, out), B, SQ, H, length, ids.shape[-1], o,
                                 ctypes.byref(plan.to_c()), stream)
    else:
        rc = lib.dsa_fwd_opts(*map(_p, data), *map(_p, out), *map(_p, part), B, SQ, H, length, ids.shape[-1], o,
                              ctypes.byref(plan.to_c()), stream)
    _lib.check(rc, f"dsa_fwd_{name}")


GRAPH_CASES = [  # (B, SQ, H, L, K), plan, paged block size (0: contiguous kv)
    ((8, 1, 128, 8192, 2048), Tuning(32, 32, 8, kv_waves=2, stages=4, mfma=16, pv_cols=128), 0),  # + merge kernel
    ((16, 2, 16, 8192, 2048), Tuning(16, 64, 2, kv_waves=4, mfma=16, fused_merge=True), 0),       # merged in kernel
    ((16, 2, 16, 8192, 2048), Tuning(16, 64, 2, kv_waves=4, mfma=16, pv_cols=128, fused_merge=True), 64),  # paged
]


@pytest.mark.gpu
@pytest.mark.parametrize("shape,plan,block", GRAPH_CASES, ids=lambda v: str(v))
def test_noalloc_captured_replays_equal_caller_buffers(shape, plan, block):
    """dsa_fwd_noalloc captured in a HIP graph on a side stream: the capture
    and every replay allocate nothing (torch.cuda.memory_allocated stays put),
    and each replay -- the inputs rewritten in place between replays, eager
    calls and synchronisations in between -- equals dsa_fwd_opts with
    caller-allocated partials and counters, bit for bit."""
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    lib = _lib.load()
    B, SQ, H, L, K = shape
    tag = f"noalloc graph {shape} {plan} block={block}"
    data = _case(300 + H + block, *shape)
    opts_kw, table = {}, None
    if block:
        data, opts_kw, table = _paged(data, block, 7)
    split = plan.split
    part = (torch.empty((B, SQ, split, H, 512), device="cuda", dtype=torch.float32),
            torch.empty((B, SQ, split, H), device="cuda", dtype=torch.float32),
            torch.empty((B, SQ, split, H), device="cuda", dtype=torch.float32))
    counters = torch.zeros(B * SQ * (H // plan.bm), device="cuda", dtype=torch.int32)
    want_opts = _lib.DsaFwdOptions(arrivals=counters.data_ptr(), **opts_kw)
    got_opts = _lib.DsaFwdOptions(**opts_kw) if block else None
    got, want = _outputs(data[0]), _outputs(data[0])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    print(f"[{tag}] eager call, then capture", flush=True)
    with torch.cuda.stream(side):
        _call(lib, "noalloc", data, plan, L, got_opts, ctypes.c_void_p(side.cuda_stream), got)
    side.synchronize()
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    # (torch's capture itself allocates its RNG seed and offset tensors, so
    # the count is taken around the library call inside the capture)
    with torch.cuda.graph(graph, stream=side):
        before = torch.cuda.memory_allocated()
        _call(lib, "noalloc", data, plan, L, got_opts, ctypes.c_void_p(side.cuda_stream), got)
        during = torch.cuda.memory_allocated()
    assert during == before, tag
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    gen = torch.Generator(device="cuda").manual_seed(11)
    for replay in range(4):
        if replay:  # new values in the same tensors: q, the kv pool, the indices
            data[0].copy_(torch.randn(data[0].shape, device="cuda", generator=gen).bfloat16())
            data[1].copy_(torch.randn(data[1].shape, device="cuda", generator=gen).bfloat16())
            data[4].copy_(torch.randint(0, L, data[4].shape, device="cuda", generator=gen, dtype=torch.int32))
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated() == before, (tag, replay)
        _call(lib, "opts", data, plan, L, want_opts, stream, want, part)
        torch.cuda.synchronize()
        print(f"[{tag}] replay {replay}", flush=True)
        for a, b in zip(got, want):
            assert torch.equal(a, b), (tag, replay)
    del table


_FIRST_CALL = "--first-call-under-capture"


@pytest.mark.gpu
def test_noalloc_first_call_under_capture_in_a_fresh_process():
    """A process whose very first dsa_fwd_noalloc call is made under graph
    capture on a fresh stream: the scratch set-up (hipGetSymbolAddress and
    the counters' zero-fill kernel) is recorded into the graph, and three
    replays of that graph equal dsa_fwd_opts bit for bit (the child process
    runs this file with the flag below)."""
    import os
    import subprocess
    import sys
    from pathlib import Path

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    print("[noalloc first call under capture] child process", flush=True)
    root = str(Path(__file__).resolve().parents[1])
    env = dict(os.environ, PYTHONPATH=os.pathsep.join(filter(None, (root, os.environ.get("PYTHONPATH")))))
    res = subprocess.run([sys.executable, __file__, _FIRST_CALL], capture_output=True, text=True, timeout=300,
                         env=env)
    print(res.stdout[-2000:], res.stderr[-2000:], flush=True)
    assert res.returncode == 0 and "first call under capture: ok" in res.stdout


def _first_call_under_capture():
    lib = _lib.load()
    plan = Tuning(16, 64, 2, kv_waves=4, mfma=16, fused_merge=True)
    B, SQ, H, L, K = 16, 2, 16, 8192, 2048
    data = _case(400, B, SQ, H, L, K)
    got, want = _outputs(data[0]), _outputs(data[0])
    part = (torch.empty((B, SQ, 2, H, 512), device="cuda", dtype=torch.float32),
            torch.empty((B, SQ, 2, H), device="cuda", dtype=torch.float32),
            torch.empty((B, SQ, 2, H), device="cuda", dtype=torch.float32))
    counters = torch.zeros(B * SQ, device="cuda", dtype=torch.int32)
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        before = torch.cuda.memory_allocated()
        _call(lib, "noalloc", data, plan, L, None, ctypes.c_void_p(side.cuda_stream), got)
        during = torch.cuda.memory_allocated()
    assert during == before
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for replay in range(3):
        graph.replay()
        torch.cuda.synchronize()
        _call(lib, "opts", data, plan, L, _lib.DsaFwdOptions(arrivals=counters.data_ptr()), stream, want, part)
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b), replay
        print(f"replay {replay} equal", flush=True)
    print("first call under capture: ok", flush=True)


if __name__ == "__main__" and _FIRST_CALL in __import__("sys").argv:
    _first_call_under_capture()
