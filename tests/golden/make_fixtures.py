"""Write tests/golden/reference_stats.json from the reference's validation records.

Reads (as JSON data, nothing is imported or executed) the accuracy records the
reference keeps for its FP32 oracle:

* validation/accuracy-all16/<case>-normal-20261102/result.json
  -> accuracy.metrics.refactored.{output,maximum,denominator}
* validation/public/<case>[-family]/result.json
  -> accuracy.metrics.public.{output,maximum,denominator}

For every record it keeps the case, shape, seed, family, the oracle statistics
(reference_max, ref_sq, elements) and the device kernel's own errors against
that oracle (max_normalized, relative_rms) for comparison.  Run from a
checkout that has the reference at ``--reference`` (default /root/reference).
The tutorial known-answer tests (DSA从原理到实现.md:159-217) are copied as
numbers.
"""
from __future__ import annotations

import argparse
import json
from pathlib import Path

HERE = Path(__file__).resolve().parent


def extract(ref: Path) -> dict:
    records = []
    sources = [(p, "refactored") for p in sorted((ref / "validation/accuracy-all16").glob("*/result.json"))]
    sources += [(p, "public") for p in sorted((ref / "validation/public").glob("*/result.json"))]
    for path, model in sources:
        data = json.loads(path.read_text())
        metrics = data["accuracy"]["metrics"][model]
        rec = {
            "source": str(path.relative_to(ref)),
            "case": data["case"],
            "shape": data["shape"],
            "seed": data["seed"],
            "family": data["family"],
            "oracle": {},
            "ascend_kernel_error": {},
        }
        for key in ("output", "maximum", "denominator"):
            m = metrics[key]
            rec["oracle"][key] = {k: m[k] for k in ("reference_max", "ref_sq", "elements")}
            rec["ascend_kernel_error"][key] = {k: m[k] for k in ("max_normalized", "relative_rms")}
        records.append(rec)
    kats = {
        "online_softmax": {
            "source": "DSA从原理到实现.md:159-199",
            "scores": [1.0, 2.0, 3.0],
            "values": [10.0, 20.0, 40.0],
            "chunks": [[0, 2], [2, 3]],
            "state_after_first_chunk": [2.0, 1.367879441, 23.678794412],
            "l": 1.503214724,
            "u": 48.710941656,
            "output": 32.40451338379263,
            "weights": [0.090030573, 0.244728471, 0.665240956],
        },
        "split_merge": {
            "source": "DSA从原理到实现.md:211-217",
            "a": [2.0, 1.367879441, 23.678794412],
            "b": [3.0, 1.0, 40.0],
            "output": 32.404513384,
            "wrong_average": 28.655292893,
        },
    }
    return {"records": records, "kats": kats}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    ap.add_argument("--out", default=str(HERE / "reference_stats.json"))
    args = ap.parse_args()
    data = extract(Path(args.reference))
    Path(args.out).write_text(json.dumps(data, indent=1, ensure_ascii=False) + "\n")
    print(f"wrote {len(data['records'])} records to {args.out}")


if __name__ == "__main__":
    main()
