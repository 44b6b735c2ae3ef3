"""W_UV output projection after the attention (no reference counterpart; the
reference returns the 512-wide latent output, README.md:81-83).

* ``project_uv`` against the FP64 oracle projection of the same bf16 latent:
  |out - ref| <= 2^-8 |ref| + 2^-16 sum_c |x_c w_c| (one bf16 rounding plus
  FP32 accumulation), on every launch shape (one tile or many per chunk,
  d split in 1, 2, 3 or 4, heads a multiple of 8 or not, ragged last
  tiles, strided weights, dv 64..256).
* ``merge_uv`` equals ``project_uv(merge(...))`` bit for bit, and its max and
  sum equal ``merge``'s, including more than 16 splits (two merge batches)
  and masked splits.
* ``forward(w_uv=)`` equals ``project_uv(forward(...)[0])`` bit for bit on
  every path (no split: a projection launch; split, fused-merge plans
  included: merged in the W_UV launch), and is checked end to end against
  the FP32 oracle attention
  followed by the FP64 projection (max-normalised error <= 1e-2, the
  attention's own gate).
"""
import pytest
import torch

import dsa_amd
from dsa_amd import Tuning
from dsa_amd import api as A
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu

OUT_TOL = 1e-2


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    torch.cuda.init()


def _weights(seed, heads, dv, parent=None):
    """bf16 [H, dv, 512] at about the scale of a trained up-projection; with
    ``parent`` rows per head, the last dv rows of a [H, parent, 512] tensor
    (wkv_b's value rows)."""
    g = torch.Generator().manual_seed(seed)
    rows = parent or dv
    w = (torch.randn(heads, rows, 512, generator=g) / 512 ** 0.5).bfloat16().cuda()
    return w[:, rows - dv:] if parent else w


def _check_projection(tag, out, x, w):
    ref = O.project_uv_ref(x, w)
    mag = O.project_uv_ref(x.float().abs(), w.float().abs())
    err = (out.double().cpu() - ref).abs()
    bound = ref.abs() * 2.0 ** -8 + mag * 2.0 ** -16
    worst = float((err - bound).max())
    print(f"[{tag}] max err {float(err.max()):.3e}, worst margin {worst:.3e}", flush=True)
    assert torch.isfinite(out).all(), tag
    assert bool((err <= bound).all()), (tag, worst)


SHAPES = [  # tokens, heads, dv, parent rows
    (8, 128, 128, None),      # decode_b8: 16-token block, d split 2
    (128, 16, 128, None),     # MTP decode, 16 heads
    (1, 16, 64, None),        # one token, dv 64: no d split
    (37, 16, 192, None),      # ragged block, dv 192
    (3, 24, 256, None),       # heads not a multiple of 8, d split 4
    (1000, 128, 128, None),   # two chunks of 16 tiles, ragged last tile
    (4096, 16, 128, 256),     # prefill: 16 chunks of 8 tiles, strided weights
    (20, 16, 128, 256),       # strided weights, 16-token blocks
]


@pytest.mark.parametrize("tokens,heads,dv,parent", SHAPES, ids=str)
def test_project_uv_against_oracle(tokens, heads, dv, parent):
    g = torch.Generator().manual_seed(tokens * 7 + heads)
    x = torch.randn(tokens, heads, 512, generator=g).bfloat16().cuda()
    w = _weights(heads + dv, heads, dv, parent)
    tag = f"project_uv T={tokens} H={heads} dv={dv} parent={parent}"
    print(f"[{tag}] launching {A._uv_launch(tokens, heads, dv, False)}", flush=True)
    out = dsa_amd.project_uv(x, w)
    torch.cuda.synchronize()
    assert out.shape == (tokens, heads, dv)
    _check_projection(tag, out, x, w)


def test_project_uv_block_shape_does_not_change_bits():
    # 1000 tokens run as two chunks of 16 tiles with two d tiles per wave;
    # an 8-token slice runs as one tile with the d range split in 2: the
    # same bits.
    x = torch.randn(1000, 128, 512, generator=torch.Generator().manual_seed(3)).bfloat16().cuda()
    w = _weights(4, 128, 128)
    full = dsa_amd.project_uv(x, w)
    for t0 in (0, 8, 992):
        part = dsa_amd.project_uv(x[t0:t0 + 8].contiguous(), w)
        assert torch.equal(part, full[t0:t0 + 8]), t0


def _partials(seed, tokens, split, heads, dead=0.0):
    g = torch.Generator().manual_seed(seed)
    part_o = torch.randn(tokens, 1, split, heads, 512, generator=g) * 3
    part_m = torch.randn(tokens, 1, split, heads, generator=g) * 4
    part_l = torch.rand(tokens, 1, split, heads, generator=g) * 50 + 1
    if dead:
        off = torch.rand(tokens, 1, split, heads, generator=g) < dead
        off[:, :, 0] = False  # every row keeps a live split
        part_m[off] = -torch.finfo(torch.float32).max
        part_l[off] = 0
        part_o[off] = 0
    return [t.cuda().contiguous() for t in (part_o, part_m, part_l)]


@pytest.mark.parametrize("tokens,split,heads,dv,dead", [
    (8, 8, 128, 128, 0.0), (8, 8, 128, 128, 0.4), (128, 2, 16, 128, 0.0), (17, 5, 16, 64, 0.3),
    (3, 20, 32, 256, 0.2), (40, 16, 24, 192, 0.0), (1, 1, 16, 128, 0.0)], ids=str)
def test_merge_uv_equals_merge_then_project_bitwise(tokens, split, heads, dv, dead):
    po, pm, pl = _partials(tokens + split, tokens, split, heads, dead)
    w = _weights(split, heads, dv)
    tag = f"merge_uv T={tokens} S={split} H={heads} dv={dv} dead={dead}"
    print(f"[{tag}] launching {A._uv_launch(tokens, heads, dv, True)}", flush=True)
    out_v, mx, sm = dsa_amd.merge_uv(po, pm, pl, w)
    lat, mx2, sm2 = dsa_amd.merge(po, pm, pl)
    two = dsa_amd.project_uv(lat, w)
    torch.cuda.synchronize()
    assert torch.equal(out_v, two), tag
    assert torch.equal(mx, mx2) and torch.equal(sm, sm2), tag
    _check_projection(tag, out_v.view(tokens, heads, dv), lat.view(tokens, heads, 512), w)


def _case(seed, B, SQ, H, L=4096, K=2048):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, SQ, H, 512, generator=g).bfloat16()
    kv = torch.randn(B, L, 1, 512, generator=g).bfloat16()
    qr = torch.randn(B, SQ, H, 64, generator=g).bfloat16()
    kr = torch.randn(B, L, 1, 64, generator=g).bfloat16()
    ids = torch.randint(0, L, (B, SQ, 1, K), generator=g, dtype=torch.int32)
    ids[torch.rand(ids.shape, generator=g) < 0.05] = -1
    ids[..., :1] = torch.randint(0, L, (B, SQ, 1, 1), generator=g, dtype=torch.int32)
    return q, kv, qr, kr, ids.contiguous()


FORWARD = [  # (B, SQ, H), plan, expected W_UV launch
    ((2, 3, 16), Tuning(16, 64, 1, kv_waves=4, mfma=16), "project_uv"),
    ((2, 1, 128), Tuning(32, 64, 4, kv_waves=2, mfma=16), "merge_uv"),
    ((4, 2, 16), Tuning(16, 64, 2, kv_waves=4, mfma=16, fused_merge=True), "merge_uv"),
    ((2, 2, 16), Tuning(16, 64, 16, kv_waves=4, mfma=16), "merge_uv"),
    ((1, 20, 128), Tuning(128, 32, 1, stages=4), "project_uv"),
]


@pytest.mark.parametrize("shape,config,launch", FORWARD, ids=str)
def test_forward_w_uv_equals_project_of_output(shape, config, launch):
    B, SQ, H = shape
    data = [t.cuda() for t in _case(B * 100 + H, B, SQ, H)]
    w = _weights(H, H, 128, parent=256)
    tag = f"forward w_uv {shape} {config}"
    print(f"[{tag}] launching", flush=True)
    (out_v, mx, sm), launches = dsa_amd.forward(*data, config=config, w_uv=w, return_kernels=True)
    out, mx2, sm2 = dsa_amd.forward(*data, config=config)
    two = dsa_amd.project_uv(out, w)
    torch.cuda.synchronize()
    assert launches[-1].name == launch, launches
    assert out_v.shape == (B, SQ, H, 128)
    assert torch.equal(out_v, two), tag
    assert torch.equal(mx, mx2) and torch.equal(sm, sm2), tag
    # end to end: FP32 oracle attention, then the FP64 projection
    ref = O.project_uv_ref(O.reference(*[t.cpu() for t in data])[0], w)
    acc = O.accuracy(out_v.cpu(), ref)
    print(f"[{tag}] vs oracle N={acc['max_normalized']:.3e} row N={acc['max_row_normalized']:.3e}", flush=True)
    assert acc["finite"] and acc["max_normalized"] <= OUT_TOL, (tag, acc)
    assert acc["max_row_normalized"] <= OUT_TOL, (tag, acc)


def test_forward_w_uv_with_scale_paged_and_fp8():
    B, SQ, H, L = 2, 2, 16, 2048
    q, kv, qr, kr, ids = [t.cuda() for t in _case(9, B, SQ, H, L=L, K=1024)]
    w = _weights(9, H, 128)
    rows = dsa_amd.quantize_kv_fp8(kv, kr)
    for kw in ({"scale": 192 ** -0.5}, {"kv": rows, "k_rope": None}):
        args = {"kv": kv, "k_rope": kr, **kw}
        (out_v, mx, sm), launches = dsa_amd.forward(q, args["kv"], qr, args["k_rope"], ids, w_uv=w,
                                                    scale=kw.get("scale"), return_kernels=True)
        assert launches[-1].name == "merge_uv", launches  # the planner splits this shape
        out, mx2, sm2 = dsa_amd.forward(q, args["kv"], qr, args["k_rope"], ids, scale=kw.get("scale"))
        torch.cuda.synchronize()
        assert torch.equal(out_v, dsa_amd.project_uv(out, w)), sorted(kw)
        assert torch.equal(mx, mx2) and torch.equal(sm, sm2), sorted(kw)
    # paged kv: a permuted block table over a pool
    bs = 64
    nblk = L // bs
    perm = torch.randperm(B * nblk, generator=torch.Generator().manual_seed(1)).int().cuda()
    table = perm.view(B, nblk).contiguous()
    kv_pool = torch.empty(B * nblk, bs, 1, 512, dtype=torch.bfloat16, device="cuda")
    kr_pool = torch.empty(B * nblk, bs, 1, 64, dtype=torch.bfloat16, device="cuda")
    kv_pool[table.view(-1).long()] = kv.view(B * nblk, bs, 1, 512)
    kr_pool[table.view(-1).long()] = kr.view(B * nblk, bs, 1, 64)
    out_v, _, _ = dsa_amd.forward(q, kv_pool, qr, kr_pool, ids, block_table=table, w_uv=w)
    out, _, _ = dsa_amd.forward(q, kv, qr, kr, ids)
    torch.cuda.synchronize()
    assert torch.equal(out_v, dsa_amd.project_uv(out, w))
