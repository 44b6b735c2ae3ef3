"""forward() captured in a HIP graph (torch.cuda.CUDAGraph) and replayed.

The library allocates and synchronises nothing, clears nothing with
hipMemsetAsync, and the in-kernel merge leaves its arrival counters at zero
after every call, so a captured call must replay exactly: every replay is
compared bit for bit with the eager result, with the program's own eager
calls and synchronisations between the replays, and the inputs are changed
in place between replays to show that the graph reads them afresh.  Calls of
256 tokens or more also run the row bucketing, into an index buffer that
forward() allocates (from the graph's private pool under capture).
"""
import pytest
import torch

import dsa_amd
from dsa_amd import Tuning

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    torch.cuda.init()


def _case(seed, B, SQ, H, L=4096, K=2048):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, SQ, H, 512, generator=g).bfloat16()
    kv = torch.randn(B, L, 1, 512, generator=g).bfloat16()
    qr = torch.randn(B, SQ, H, 64, generator=g).bfloat16()
    kr = torch.randn(B, L, 1, 64, generator=g).bfloat16()
    ids = torch.randint(0, L, (B, SQ, 1, K), generator=g, dtype=torch.int32)
    ids[torch.rand(ids.shape, generator=g) < 0.05] = -1
    ids[..., :1] = torch.randint(0, L, (B, SQ, 1, 1), generator=g, dtype=torch.int32)
    return [t.cuda() for t in (q, kv, qr, kr, ids.contiguous())]


CASES = [  # (B, SQ, H), plan, W_UV value dim (0: none)
    ((2, 1, 128), Tuning(32, 64, 8, kv_waves=2, mfma=16), 0),                    # main + merge kernel
    ((4, 2, 16), Tuning(16, 64, 2, kv_waves=4, mfma=16, fused_merge=True), 0),   # one launch, arrival counters
    ((1, 40, 128), Tuning(128, 32, 1, stages=4), 0),                              # wide kernel, no split
    ((1, 40, 128), Tuning(128, 32, 1, kv_waves=1, stages=4, mfma=16, pv_cols=128), 0),   # ping-pong, no split
    ((2, 2, 128), Tuning(128, 32, 3, kv_waves=1, stages=4, mfma=16, pv_cols=128), 0),    # ping-pong + merge kernel
    ((8, 1, 128), Tuning(32, 32, 8, kv_waves=2, stages=4, mfma=16, pv_cols=128), 0),     # specialised waves + merge
    ((2, 1, 128), Tuning(32, 64, 4, kv_waves=2, mfma=16), 128),                   # main + merge_uv
    ((2, 3, 16), Tuning(16, 64, 1, kv_waves=4, mfma=16), 128),                    # main + project_uv
    # 256 tokens or more: the row bucketing runs first, into a buffer the
    # capture allocates from the graph's pool
    ((1, 260, 16), Tuning(16, 64, 1, kv_waves=4, mfma=16, pv_cols=128), 0),      # bucketing + column-split
    ((2, 130, 128), Tuning(128, 32, 1, kv_waves=1, stages=4, mfma=16, pv_cols=128), 0),  # bucketing + ping-pong
    ((1, 256, 16), Tuning(16, 64, 1, kv_waves=4, mfma=16, pv_cols=128), 128),    # bucketing + project_uv
]


@pytest.mark.parametrize("shape,config,dv", CASES, ids=str)
def test_captured_forward_replays_bitwise(shape, config, dv):
    B, SQ, H = shape
    data = _case(B * 31 + H, B, SQ, H)
    w = None
    if dv:
        w = (torch.randn(H, dv, 512, generator=torch.Generator().manual_seed(H)) / 512 ** 0.5).bfloat16().cuda()
    kw = {"config": config, "w_uv": w}
    tag = f"graph {shape} {config} dv={dv}"
    print(f"[{tag}] warm-up and capture", flush=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        dsa_amd.forward(*data, **kw)  # warm-up: library loaded, plan cached
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = dsa_amd.forward(*data, **kw)
    torch.cuda.synchronize()
    for rep in range(4):
        if rep == 2:  # new inputs, written in place: the graph must read them afresh
            fresh = _case(B * 31 + H + 1000, B, SQ, H)
            for dst, src in zip(data, fresh):
                dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        eager = dsa_amd.forward(*data, **kw)
        torch.cuda.synchronize()
        print(f"[{tag}] replay {rep}", flush=True)
        for a, b in zip(static_out, eager):
            assert torch.equal(a, b), (tag, rep)


def test_two_fused_graphs_replayed_out_of_order():
    """Two fused-merge calls captured into two graphs (on torch's shared
    capture stream), then the second graph replayed first and both replayed
    in turn: each captured call has counters of its own, zero-filled by a
    kernel recorded in its own graph, so neither replay depends on the other
    graph having run.  Every replay equals the eager call bit for bit."""
    config = Tuning(16, 64, 2, kv_waves=4, mfma=16, fused_merge=True)
    cases = [_case(501, 4, 2, 16), _case(502, 3, 2, 32)]
    for data in cases:
        dsa_amd.forward(*data, config=config)
    torch.cuda.synchronize()
    graphs, outs = [], []
    for i, data in enumerate(cases):
        print(f"[two fused graphs] capture {i}", flush=True)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs.append(dsa_amd.forward(*data, config=config))
        graphs.append(g)
    torch.cuda.synchronize()
    eager = [dsa_amd.forward(*data, config=config) for data in cases]
    torch.cuda.synchronize()
    for rep, order in enumerate(([1, 0], [1, 1, 0, 0], [0, 1])):
        for i in order:
            graphs[i].replay()
            torch.cuda.synchronize()
            print(f"[two fused graphs] round {rep} graph {i}", flush=True)
            for a, b in zip(outs[i], eager[i]):
                assert torch.equal(a, b), (rep, i)


def test_caller_owned_arrivals():
    """forward(arrivals=...): the caller's counters are used (and left zero),
    and a too-small tensor is rejected before anything is enqueued."""
    config = Tuning(16, 64, 2, kv_waves=4, mfma=16, fused_merge=True)
    data = _case(503, 4, 2, 16)
    ref = dsa_amd.forward(*data, config=config)
    own = torch.zeros(4 * 2 * 1, device="cuda", dtype=torch.int32)
    for _ in range(3):
        got = dsa_amd.forward(*data, config=config, arrivals=own)
        torch.cuda.synchronize()
        for a, b in zip(ref, got):
            assert torch.equal(a, b)
        assert int(own.abs().sum()) == 0
    with pytest.raises(ValueError, match="arrivals"):
        dsa_amd.forward(*data, config=config, arrivals=own[:7])
