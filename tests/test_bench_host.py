"""Host logic of bench.py on the CPU: the record's scalar leg fields, the
per-call algorithmic units (pinned by the MFMA-instruction counters in
profiles/), the input-set rotation, and the refusal of more than one GPU."""
import importlib.util
import os
import subprocess
import sys
from pathlib import Path

import pytest

from dsa_amd import Tuning

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench", ROOT / "bench.py")
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def test_algorithmic_units(bench):
    # C2: 8 tokens x 2048 slots x 1152 bytes; MFMA FLOPs as counted on the
    # device (SQ_INSTS_MFMA x 16384 = 4.563e9 for C2, 2.921e11 for C4)
    assert bench.algorithmic_units((8, 1, 128, 32768, 2048)) == (18874368, 4563402752)
    assert bench.algorithmic_units((1, 4096, 16, 8192, 2048)) == (9663676416, 292057776128)
    # fp8 rows: 656 bytes a slot, the same MFMA work
    assert bench.algorithmic_units((8, 1, 128, 32768, 2048), fp8=True) == (8 * 2048 * 656, 4563402752)


def test_leg_fields_are_flat_scalars(bench):
    line = {"value": 63.9, "config": {"plan": "bm=16 bn=64 split=2"},
            "roofline": {"bound": "hbm", "achieved": 4724.1, "unit": "GB/s", "frac": 0.59, "frac_span": 0.59,
                         "traffic": 327593135},
            "breakdown": {"span_min_us": 63.8, "span_max_us": 64.0, "main_us": 63.9, "merge_us": 0.2,
                          "fixed_chain_us": 13.7},
            "cpu_baseline": {"value": 63962.2, "sample": "full call"}}
    line["config"]["rotating_input_sets"] = 2
    leg = bench.leg("c3", line)
    assert all(k.startswith("c3_") for k in leg)
    assert all(not isinstance(v, (dict, list)) for v in leg.values())
    assert leg["c3_span_us"] == 63.9 and leg["c3_frac"] == 0.59 and leg["c3_cpu_us"] == 63962.2
    assert leg["c3_fixed_chain_us"] == 13.7 and leg["c3_plan"] == "bm=16 bn=64 split=2"


def test_plan_text_and_spread(bench):
    text = bench.plan_text(Tuning(32, 32, 8, kv_waves=2, stages=4, mfma=16, pv_cols=128))
    assert text == "bm=32 bn=32 split=8 kv_waves=2 stages=4 mfma=16 pv_cols=128 fused_merge=0"
    assert bench.spread([3.0, 1.0, 2.0]) == (2.0, 1.0, 3.0)


def test_rotation_is_one_continuous_cycle(bench):
    rot = bench.Rotation(["a", "b", "c"])
    assert [rot.take() for _ in range(7)] == ["a", "b", "c", "a", "b", "c", "a"]


def test_more_than_one_gpu_is_refused():
    env = dict(os.environ, WORLD_SIZE="1")
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         env=env, timeout=300)
    assert res.returncode == 2 and "one GPU" in res.stderr and res.stdout == ""
