"""Shared parity gate of the GPU tests: one kernel result against the CPU
oracle (oracle/dsa_oracle.py), at the BASELINE bounds.

* output: max-normalised error max|out - ref| / max|ref| <= 1e-2, and the
  reference's per-row error (tools/review.py:160-161: per (token, head) over
  the 512 columns) <= 1e-2;
* softmax_max / softmax_sum: elementwise relative error <= 1e-4 (which also
  bounds their per-query row metric).
"""
from oracle import dsa_oracle as O

OUT_TOL = 1e-2
STAT_RTOL = 1e-4


def check(tag, out, mx, sm, ref):
    """Compare (out, mx, sm) with the oracle's ``ref`` triple; print and
    assert.  Returns the output's accuracy record."""
    acc = O.accuracy(out.cpu(), ref[0])
    em, es = O.rel_error(mx.cpu(), ref[1]), O.rel_error(sm.cpu(), ref[2])
    print(f"[{tag}] output N={acc['max_normalized']:.3e} row N={acc['max_row_normalized']:.3e} "
          f"({acc['rows']} rows) max rel={em:.2e} sum rel={es:.2e}", flush=True)
    assert acc["finite"], tag
    assert acc["max_normalized"] <= OUT_TOL, (tag, acc)
    assert acc["max_row_normalized"] <= OUT_TOL, (tag, acc)
    assert em <= STAT_RTOL and es <= STAT_RTOL, (tag, em, es)
    return acc
