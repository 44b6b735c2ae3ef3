"""Host contract of dsa_amd.forward without a GPU.

Mirrors the reference's CPU-only host checks (tools/check_host_api.py:88-129):
every rejection is raised before any allocation or launch, with the
reference's exception types (ValueError for shapes/devices/dtypes/plans,
TypeError for a config of the wrong type).  Planning runs in the C library,
which loads and plans without touching a device.
"""
import pytest
import torch

import dsa_amd
from dsa_amd import CASE_SHAPES, SELECTED, Tuning, plan_call
from dsa_amd import api as A
from dsa_amd.api import _check_inputs
from dsa_amd.config import check_tuning, plan_for
from dsa_amd.workloads import BASELINE_CONFIGS


def _tensors(B=2, SQ=3, H=16, L=40, K=24, device="cpu"):
    return (torch.zeros(B, SQ, H, 512, dtype=torch.bfloat16, device=device),
            torch.zeros(B, L, 1, 512, dtype=torch.bfloat16, device=device),
            torch.zeros(B, SQ, H, 64, dtype=torch.bfloat16, device=device),
            torch.zeros(B, L, 1, 64, dtype=torch.bfloat16, device=device),
            torch.zeros(B, SQ, 1, K, dtype=torch.int32, device=device))


SHAPE_MUTATIONS = {
    "q rank": lambda t: (t[0][0],) + t[1:],
    "kv rank": lambda t: (t[0], t[1][0]) + t[2:],
    "ids rank": lambda t: t[:4] + (t[4][0],),
    "q width": lambda t: (torch.zeros(2, 3, 16, 256, dtype=torch.bfloat16),) + t[1:],
    "kv width": lambda t: (t[0], torch.zeros(2, 40, 1, 256, dtype=torch.bfloat16)) + t[2:],
    "kv heads": lambda t: (t[0], torch.zeros(2, 40, 2, 512, dtype=torch.bfloat16)) + t[2:],
    "kv batch": lambda t: (t[0], torch.zeros(3, 40, 1, 512, dtype=torch.bfloat16)) + t[2:],
    "q_rope width": lambda t: t[:2] + (torch.zeros(2, 3, 16, 32, dtype=torch.bfloat16),) + t[3:],
    "q_rope heads": lambda t: t[:2] + (torch.zeros(2, 3, 8, 64, dtype=torch.bfloat16),) + t[3:],
    "k_rope length": lambda t: t[:3] + (torch.zeros(2, 41, 1, 64, dtype=torch.bfloat16),) + t[4:],
    "ids queries": lambda t: t[:4] + (torch.zeros(2, 4, 1, 24, dtype=torch.int32),),
    "ids heads": lambda t: t[:4] + (torch.zeros(2, 3, 2, 24, dtype=torch.int32),),
    "zero length": lambda t: _tensors(L=0),
    "zero topk": lambda t: _tensors(K=0),
    "heads not multiple of 16": lambda t: _tensors(H=24),
}


@pytest.mark.parametrize("name", sorted(SHAPE_MUTATIONS))
def test_shape_rejections(name):
    bad = SHAPE_MUTATIONS[name](_tensors())
    with pytest.raises(ValueError):
        _check_inputs(*bad)
    with pytest.raises(ValueError):
        dsa_amd.forward(*bad)


def test_cpu_tensors_rejected_as_device_error():
    with pytest.raises(ValueError, match="ROCm GPU"):
        dsa_amd.forward(*_tensors())


def test_meta_tensors_rejected():
    with pytest.raises(ValueError, match="ROCm GPU"):
        dsa_amd.forward(*_tensors(device="meta"))


def test_exports_match_reference_surface():
    for name in ("forward", "Tuning", "CASE_SHAPES", "SELECTED"):
        assert hasattr(dsa_amd, name)
    assert set(SELECTED) == set(CASE_SHAPES)


@pytest.mark.parametrize("name", sorted(CASE_SHAPES))
def test_selected_plans_are_valid(name):
    check_tuning(SELECTED[name], CASE_SHAPES[name])


@pytest.mark.parametrize("name", sorted(BASELINE_CONFIGS))
def test_baseline_configs_in_table(name):
    assert CASE_SHAPES[name] == BASELINE_CONFIGS[name]
    assert dsa_amd.select(CASE_SHAPES[name]) == SELECTED[name]


def test_bench_reference_cases_cover_the_table():
    """bench.py --cases times exactly the reference's 16 validated cases, each
    with a published span to compare against."""
    import importlib.util
    from pathlib import Path
    spec = importlib.util.spec_from_file_location("bench", Path(__file__).resolve().parents[1] / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    ref = {n for n in CASE_SHAPES if n[:2] not in ("c1", "c2", "c3", "c4", "c5")}
    assert set(bench.REF_CASES) == ref == set(bench.REF_CASE_SPAN_US)
    assert len(bench.REF_CASES) == 16 and all(v > 0 for v in bench.REF_CASE_SPAN_US.values())


def test_case_inputs_distribution():
    """The device-side draw of the review recipe (bench.py --cases): shapes,
    dtypes, TOPK distinct indices per token inside [0, L), reproducible per
    seed."""
    from dsa_amd.workloads import case_inputs
    shape = (2, 3, 16, 300, 40)
    q, kv, qr, kr, ids = case_inputs(shape, seed=7, device="cpu")
    assert q.shape == (2, 3, 16, 512) and kv.shape == (2, 300, 1, 512)
    assert qr.shape == (2, 3, 16, 64) and kr.shape == (2, 300, 1, 64)
    assert ids.shape == (2, 3, 1, 40) and ids.dtype == torch.int32
    assert {t.dtype for t in (q, kv, qr, kr)} == {torch.bfloat16}
    rows = ids.reshape(6, 40)
    assert int(rows.min()) >= 0 and int(rows.max()) < 300
    assert all(len(set(r.tolist())) == 40 for r in rows)
    assert len({tuple(r.tolist()) for r in rows}) == 6
    assert abs(float(q.float().std()) - 1.0) < 0.05
    again = case_inputs(shape, seed=7, device="cpu")
    assert all(torch.equal(a, b) for a, b in zip((q, kv, qr, kr, ids), again))


@pytest.mark.parametrize("shape", [(1, 1, 16, 1, 1), (3, 5, 48, 1000, 777), (2, 7, 32, 9, 4097),
                                   (1, 1, 128, 65536, 8192), (64, 2, 16, 65536, 2048)])
def test_planner_covers_any_shape(shape):
    plan = plan_for(shape)
    check_tuning(plan, shape)
    topk = shape[-1]
    ntiles = -(-topk // plan.bn)
    assert 1 <= plan.split <= ntiles
    assert -(-ntiles // plan.split) * plan.bn <= 2048  # index cache of one workgroup
    assert shape[2] % plan.bm == 0
    if plan.pv_cols == 128 and plan.bn == 32 and plan.bm < 128:  # specialised waves: 16 or 32 heads
        assert plan.kv_waves == 2 and plan.stages == 4 and plan.mfma == 16 and plan.bm in (16, 32)
        assert not plan.fused_merge or plan.bm == 16  # in-kernel merge: 16 heads only
    elif plan.pv_cols == 128 and plan.bm < 128:  # column-split PV: four waves share every head block
        assert plan.kv_waves == 4 and plan.mfma == 16 and plan.bm in (16, 32, 64)
    elif plan.pv_cols == 128:  # ping-pong
        assert plan.kv_waves == 1 and plan.stages == 4 and plan.mfma == 16 and plan.bn == 32
    else:
        assert plan.bm // plan.mfma * plan.kv_waves == 4


def test_plan_call_allocations_and_launches():
    shape = CASE_SHAPES["decode_b8"]
    config, partials, launches = plan_call(shape, cores=256)
    assert config == SELECTED["decode_b8"]
    assert partials == ((8, 1, config.split, 128, 512), (8, 1, config.split, 128))
    assert [l.name for l in launches] == [launches[0].name, "merge_partials"]
    assert launches[0].grid == 8 * config.split * (128 // config.bm)
    # 32 heads, specialised waves: two QK, two PV and four gather waves
    assert launches[0].name.startswith("sparse_mla_fwd_xs_h32") and launches[0].block == 512
    assert launches[0].lds_bytes == 4 * 32 * 1152 + 2048 * 4 + 2 * 32 * 64 + 3 * 32 * 4 + 16
    # 16 heads, column-split PV: four compute waves and four gather waves
    _, _, launches = plan_call(shape, config=Tuning(16, 64, 4, kv_waves=4, mfma=16, pv_cols=128), cores=256)
    assert launches[0].name.startswith("sparse_mla_fwd_xp_h16") and launches[0].block == 512
    # XpLds<HB>: two 64-row stages, the index cache (1024 slots for 64 heads),
    # P at 144 bytes a head, four waves' maxima, the vote flag
    for bm, idx_cap in ((16, 2048), (32, 2048), (64, 1024)):
        _, _, launches = plan_call(shape, config=Tuning(bm, 64, 4, kv_waves=4, mfma=16, pv_cols=128), cores=256)
        assert launches[0].lds_bytes == 2 * 64 * 1152 + idx_cap * 4 + bm * 144 + 4 * bm * 4 + 16
        assert launches[0].lds_bytes <= 160 * 1024
    assert launches[0].lds_bytes == 161808
    # 16 heads, specialised waves: one QK wave, two PV and four gather waves
    _, _, launches = plan_call(shape, config=Tuning(16, 32, 4, kv_waves=2, stages=4, mfma=16, pv_cols=128), cores=256)
    assert launches[0].name.startswith("sparse_mla_fwd_xs_h16") and launches[0].block == 448
    config, partials, launches = plan_call(CASE_SHAPES["c5_prefill_h128"], cores=256)
    assert config.split == 1 and partials is None and [l.name for l in launches][0] == "bucket_rows"
    # 128 heads, column-split PV: the eight-wave ping-pong kernel after the row bucketing
    assert len(launches) == 2 and launches[1].name.startswith("sparse_mla_fwd_pp") and launches[1].block == 512
    assert launches[1].lds_bytes == 160 * 1024


def test_prefill_calls_bucket_their_rows_first():
    from dsa_amd import api as A
    # 256 tokens or more, TOPK up to 4096: a row bucketing before the main kernel
    assert A.buckets_rows(CASE_SHAPES["c4_prefill_h16"]) and A.buckets_rows(CASE_SHAPES["c5_prefill_h128"])
    assert not A.buckets_rows(CASE_SHAPES["c2_decode_b8"]) and not A.buckets_rows(CASE_SHAPES["c3_decode_h16_mtp"])
    assert not A.buckets_rows((1, 4096, 16, 8192, 8192)) and A.buckets_rows((2, 128, 16, 8192, 4096))
    _, _, launches = plan_call(CASE_SHAPES["c4_prefill_h16"], cores=256)
    # 32 chunks x 65 counts, 65 bases, the 2048-entry row
    assert launches[0] == A.Launch("bucket_rows", 4096, 256, 4 * (32 * 65 + 65 + 2048)) and len(launches) == 2
    assert A.bucket_lds_bytes(4096) == 4 * (64 * 65 + 65 + 4096) and A.bucket_lds_bytes(1) == 4 * (65 + 65 + 1)
    _, _, launches = plan_call(CASE_SHAPES["c2_decode_b8"], cores=256)
    assert all(l.name != "bucket_rows" for l in launches)


def test_plan_call_fused_merge_is_one_launch():
    shape = CASE_SHAPES["c3_decode_h16_mtp"]
    config, partials, launches = plan_call(shape, cores=256)
    assert config.fused_merge and config.split == 2
    # partials are still written (and read back by the last workgroup); no merge launch
    assert partials == ((64, 2, 2, 16, 512), (64, 2, 2, 16))
    assert len(launches) == 1 and launches[0].name.startswith("sparse_mla_fwd_xp")  # column-split PV
    # a fused plan goes through the same library check as any other
    with pytest.raises(ValueError, match="fused_merge"):
        plan_call(CASE_SHAPES["c2_decode_b8"], Tuning(64, 64, 2, kv_waves=2, mfma=32, fused_merge=True))
    with pytest.raises(ValueError, match="fused_merge"):  # specialised waves: 16 heads only
        plan_call(CASE_SHAPES["c2_decode_b8"],
                  Tuning(32, 32, 8, kv_waves=2, stages=4, mfma=16, pv_cols=128, fused_merge=True))
    config, _, launches = plan_call(CASE_SHAPES["c3_decode_h16_mtp"],
                                    Tuning(16, 32, 2, kv_waves=2, stages=4, mfma=16, pv_cols=128, fused_merge=True))
    assert len(launches) == 1 and launches[0].name.startswith("sparse_mla_fwd_xs_h16")
    with pytest.raises(ValueError, match="bool"):
        plan_call(shape, Tuning(16, 64, 2, kv_waves=4, mfma=16, fused_merge=1))


def test_plan_call_explicit_tuning_and_errors():
    shape = (1, 1, 128, 8192, 2048)
    config, partials, _ = plan_call(shape, Tuning(32, 64, 4, kv_waves=2, mfma=16))
    assert config.split == 4 and partials[0][2] == 4
    with pytest.raises(ValueError):
        plan_call(shape, cores=0)
    with pytest.raises(ValueError):
        plan_call(shape, cores=2.0)


TUNING_MUTATIONS = {
    "bm not dividing H": Tuning(64, 64, 1, kv_waves=2),
    "bm 48": Tuning(48, 64, 1, mfma=16),
    "bn 128": Tuning(16, 128, 1, kv_waves=4, mfma=16),
    "narrow bn 32": Tuning(16, 32, 1, kv_waves=4, mfma=16),
    "split 0": Tuning(16, 64, 0, kv_waves=4, mfma=16),
    "split > tiles": Tuning(16, 64, 2, kv_waves=4, mfma=16),
    "kv_waves mismatch": Tuning(16, 64, 1, kv_waves=1, mfma=16),
    "stages 3": Tuning(16, 64, 1, kv_waves=4, stages=3, mfma=16),
    "mfma 8": Tuning(16, 64, 1, kv_waves=4, mfma=8),
    "wide with 16 heads": Tuning(16, 64, 1, kv_waves=4, mfma=32),
    "wide 128 heads": Tuning(128, 64, 1, kv_waves=1, mfma=32),
}


@pytest.mark.parametrize("name", sorted(TUNING_MUTATIONS))
def test_tuning_rejections(name):
    shape = (1, 1, 16, 100, 64)  # one tile of 64 slots
    with pytest.raises(ValueError):
        check_tuning(TUNING_MUTATIONS[name], shape)


def test_tuning_type_error():
    with pytest.raises(TypeError):
        check_tuning((64, 64, 1), (1, 1, 64, 10, 10))
    with pytest.raises(ValueError):
        check_tuning(Tuning(64.0, 64, 1), (1, 1, 64, 10, 10))


def test_index_cache_limit_forces_split():
    # TOPK 8192 = 128 tiles; one workgroup holds at most 2048 slots -> split >= 4
    with pytest.raises(ValueError):
        check_tuning(Tuning(64, 64, 2, kv_waves=2), (1, 1, 64, 100000, 8192))
    check_tuning(Tuning(64, 64, 4, kv_waves=2), (1, 1, 64, 100000, 8192))


# ------------------------------------------------------- options beyond the reference
@pytest.mark.parametrize("bad,exc", [("0.1", TypeError), (True, TypeError), (0.0, ValueError), (-0.5, ValueError),
                                     (float("inf"), ValueError), (float("nan"), ValueError)])
def test_scale_rejections(bad, exc):
    with pytest.raises(exc):
        dsa_amd.forward(*_tensors(), scale=bad)


def _paged_tensors(B=2, SQ=3, H=16, blocks=9, bs=8, M=5, K=24, device="cpu"):
    return (torch.zeros(B, SQ, H, 512, dtype=torch.bfloat16, device=device),
            torch.zeros(blocks, bs, 1, 512, dtype=torch.bfloat16, device=device),
            torch.zeros(B, SQ, H, 64, dtype=torch.bfloat16, device=device),
            torch.zeros(blocks, bs, 1, 64, dtype=torch.bfloat16, device=device),
            torch.zeros(B, SQ, 1, K, dtype=torch.int32, device=device),
            torch.zeros(B, M, dtype=torch.int32, device=device))


def test_paged_shape_contract():
    q, kv, qr, kr, ids, table = _paged_tensors()
    # the logical length is max_blocks * block_size; the pool shape is free
    with pytest.raises(ValueError, match="ROCm GPU"):  # shapes pass; CPU tensors fail the device check
        _check_inputs(q, kv, qr, kr, ids, table)
    bad = {
        "table rank": (q, kv, qr, kr, ids, table[0]),
        "table batch": (q, kv, qr, kr, ids, torch.zeros(3, 5, dtype=torch.int32)),
        "rope pool": (q, kv, qr, torch.zeros(9, 4, 1, 64, dtype=torch.bfloat16), ids, table),
        "kv width": (q, torch.zeros(9, 8, 1, 256, dtype=torch.bfloat16), qr, kr, ids, table),
    }
    for name, args in bad.items():
        with pytest.raises(ValueError):
            _check_inputs(*args)
        with pytest.raises(ValueError):
            dsa_amd.forward(*args[:5], block_table=args[5])


# ------------------------------------------------------------ lightning indexer
def _idx_inputs(B=2, SQ=3, HI=64, L=100):
    return (torch.zeros(B, SQ, HI, 128, dtype=torch.bfloat16), torch.zeros(B, L, 128, dtype=torch.bfloat16),
            torch.zeros(B, SQ, HI), torch.full((B, SQ), L, dtype=torch.int32))


@pytest.mark.parametrize("name,mutate", [
    ("q rank", lambda a: (a[0][0],) + a[1:]),
    ("head dim", lambda a: (a[0][..., :64],) + a[1:]),
    ("heads 48", lambda a: (a[0][:, :, :48].contiguous(), a[1], a[2][:, :, :48].contiguous(), a[3])),
    ("k batch", lambda a: (a[0], a[1][:1], a[2], a[3])),
    ("weights shape", lambda a: (a[0], a[1], a[2][:, :, :32], a[3])),
    ("lengths shape", lambda a: a[:3] + (a[3][:, :1],)),
    ("lengths dtype", lambda a: a[:3] + (a[3].long(),)),
    ("q dtype", lambda a: (a[0].float(),) + a[1:]),
    ("cpu tensors", lambda a: a),
])
def test_indexer_logits_rejections(name, mutate):
    with pytest.raises(ValueError):
        dsa_amd.indexer_logits(*mutate(_idx_inputs()))


def test_indexer_topk_rejections():
    logits, lengths = torch.zeros(2, 3, 100), torch.full((2, 3), 100, dtype=torch.int32)
    for bad in (0, -1, 2.0, True):
        with pytest.raises(ValueError):
            dsa_amd.indexer_topk(logits, lengths, bad)
    with pytest.raises(ValueError):
        dsa_amd.indexer_topk(logits[0], lengths, 10)
    with pytest.raises(ValueError):
        dsa_amd.indexer_topk(logits, lengths[:, :2], 10)
    with pytest.raises(ValueError):
        dsa_amd.indexer_topk(logits.double(), lengths, 10)
    with pytest.raises(ValueError):  # CPU tensors: the selection runs on a ROCm GPU only
        dsa_amd.indexer_topk(logits, lengths, 10)


# ------------------------------------------------------------ fp8 kv rows
def test_fp8_rows_shape_contract():
    q = torch.zeros(2, 3, 16, 512, dtype=torch.bfloat16)
    qr = torch.zeros(2, 3, 16, 64, dtype=torch.bfloat16)
    ids = torch.zeros(2, 3, 1, 64, dtype=torch.int32)
    rows = torch.zeros(2, 100, 1, 656, dtype=torch.uint8)
    kr = torch.zeros(2, 100, 1, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="k_rope must be None"):
        _check_inputs(q, rows, qr, kr, ids)
    with pytest.raises(ValueError, match="k_rope is required"):
        _check_inputs(q, torch.zeros(2, 100, 1, 512, dtype=torch.bfloat16), qr, None, ids)
    with pytest.raises(ValueError, match="656"):
        _check_inputs(q, torch.zeros(3, 100, 1, 656, dtype=torch.uint8), qr, None, ids)
    # shapes pass; the CPU device is then rejected like any other input
    with pytest.raises(ValueError, match="ROCm GPU"):
        _check_inputs(q, rows, qr, None, ids)


def test_fp8_plans_are_narrow():
    for shape in ((8, 1, 128, 32768, 2048), (1, 4096, 128, 32768, 2048)):
        config, _, _ = plan_call(shape, None, 256, kv_fp8=True)
        assert config.mfma == 16
    with pytest.raises(ValueError, match="narrow"):
        plan_call((1, 1, 128, 8192, 2048), Tuning(128, 32, 1, stages=4), 256, kv_fp8=True)


def test_quantize_kv_fp8_rows():
    g = torch.Generator().manual_seed(5)
    kv = (torch.randn(2, 7, 1, 512, generator=g) * 3).bfloat16()
    kv[0, 0, 0, 128:256] = 0  # an all-zero block keeps scale 1
    kr = torch.randn(2, 7, 1, 64, generator=g).bfloat16()
    rows = dsa_amd.quantize_kv_fp8(kv, kr, pow2_scales=False)
    assert rows.shape == (2, 7, 1, 656) and rows.dtype == torch.uint8
    scales = rows[..., 512:528].contiguous().view(torch.float32)
    amax = kv.float().reshape(2, 7, 1, 4, 128).abs().amax(-1)
    expect = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    assert torch.equal(scales, expect)
    # default: the smallest power of two with amax / scale <= 448
    p2 = dsa_amd.quantize_kv_fp8(kv, kr)[..., 512:528].contiguous().view(torch.float32)
    m, _ = torch.frexp(p2)
    assert (m == 0.5).all()
    assert (amax / p2 <= 448.0).all() and ((amax == 0) | (amax / p2 > 224.0)).all()
    assert torch.equal(rows[..., 528:].contiguous().view(torch.bfloat16), kr)
    codes = rows[..., :512].contiguous().view(torch.float8_e4m3fn).float().reshape(2, 7, 1, 4, 128)
    assert codes.abs().max() <= 448.0
    back = (codes * scales[..., None]).reshape(2, 7, 1, 512)
    # e4m3 keeps 3 mantissa bits: each value within 2^-4 of its block maximum's scale step
    err = (back - kv.float()).abs().reshape(2, 7, 1, 4, 128).amax(-1)
    assert (err <= amax / 16 + 1e-30).all()
    with pytest.raises(ValueError):
        dsa_amd.quantize_kv_fp8(kv.float(), kr)
    with pytest.raises(ValueError):
        dsa_amd.quantize_kv_fp8(kv, kr[..., :32])


def test_plan_call_w_uv_launches():
    # split without the in-kernel merge: the merge runs inside the W_UV launch
    cfg = Tuning(32, 64, 8, kv_waves=2, mfma=16)
    _, partials, launches = A.plan_call((8, 1, 128, 32768, 2048), cfg, w_uv_dim=128)
    assert partials is not None
    assert [l.name for l in launches][1:] == ["merge_uv"]
    assert launches[1].grid == 128 * 2 and launches[1].lds_bytes == 16 * 1024   # d split in 2
    # a fused-merge plan also merges in the W_UV launch; no split: a projection follows
    _, _, launches = A.plan_call((64, 2, 16, 65536, 2048), Tuning(16, 64, 2, kv_waves=4, mfma=16, fused_merge=True),
                                 w_uv_dim=128)
    assert [l.name for l in launches][1:] == ["merge_uv"]
    _, _, launches = A.plan_call((1, 4096, 128, 32768, 2048), Tuning(128, 32, 1, stages=4), w_uv_dim=128)
    assert [l.name for l in launches][0] == "bucket_rows" and [l.name for l in launches][2:] == ["project_uv"]
    # prefill: two chunks of 2048 tokens per head, 32-token tiles in four LDS buffers
    assert launches[2].grid == 128 * 2 and launches[2].lds_bytes == 4 * 32 * 1024
    _, _, launches = A.plan_call((1, 4096, 16, 8192, 2048), None, w_uv_dim=128)
    assert launches[-1].grid == 16 * 16
    # 128 tokens, 256-wide values, split plan: 8 blocks of 16 tokens, d split in 2
    _, _, launches = A.plan_call((64, 2, 16, 65536, 2048), None, w_uv_dim=256)
    assert launches[-1].name == "merge_uv" and launches[-1].grid == 16 * 8 * 2
    # the same without a split: 4 chunks of one 32-token tile, d split in 4
    _, _, launches = A.plan_call((64, 2, 16, 65536, 2048), Tuning(16, 64, 1, kv_waves=4, mfma=16), w_uv_dim=256)
    assert launches[-1].grid == 16 * 4 * 4 and launches[-1].lds_bytes == 4 * 32 * 1024


@pytest.mark.parametrize("mutate,msg", [
    (lambda w: w[:, :100], "multiple of 64"),
    (lambda w: w[:8], "w_uv must be"),
    (lambda w: w.float(), "bfloat16"),
    (lambda w: w.transpose(1, 2)[:, :128, :], "w_uv must be"),
    (lambda w: w[:, :, :].as_strided((16, 64, 512), (64 * 512 + 4, 512, 1)), "head stride"),
], ids=["dv", "heads", "dtype", "transposed", "stride"])
def test_w_uv_rejections(mutate, msg):
    w = torch.zeros(16, 128, 512, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match=msg):
        A._check_w_uv(mutate(w), 16, torch.device("cpu"))


def test_w_uv_strided_value_rows_accepted():
    wkv_b = torch.zeros(16, 128 + 128, 512, dtype=torch.bfloat16)
    assert A._check_w_uv(wkv_b[:, -128:], 16, torch.device("cpu")) == (128, 256 * 512)


def test_reference_import_name_is_the_same_operator():
    # reference callers write `from dsa import forward` (README.md:70 of the reference)
    import dsa
    from dsa import CASE_SHAPES as shapes, SELECTED as selected, Tuning as tuning, forward as fwd

    assert fwd is dsa_amd.forward and tuning is dsa_amd.Tuning
    assert shapes is dsa_amd.CASE_SHAPES and selected is dsa_amd.SELECTED
    assert set(dsa.__all__) == set(dsa_amd.__all__)
