"""MI355X-native DSA sparse-MLA attention forward (drop-in for ``dsa.forward``).

Public surface mirrors the reference package (dsa/__init__.py:2-5):
``forward``, ``Tuning``, ``CASE_SHAPES``, ``SELECTED``; plus ``merge`` (the
standalone FP32 split merge), ``select`` (the plan for a shape) and the
lightning indexer that produces the indices (``indexer``, ``indexer_logits``,
``indexer_topk``), the fp8 kv cache row writer (``quantize_kv_fp8``) and the
W_UV output projection after the attention (``project_uv``, ``merge_uv``,
``forward(w_uv=)``) and the row-range bucketing of prefill-sized calls'
indices (``bucket_indices``).
"""
from .api import bucket_indices, forward, merge, merge_uv, plan_call, project_uv
from .config import CASE_SHAPES, SELECTED, Tuning, select
from .indexer import indexer, indexer_logits, indexer_topk
from .kvcache import quantize_kv_fp8

__all__ = ["forward", "merge", "merge_uv", "project_uv", "plan_call", "bucket_indices", "Tuning", "CASE_SHAPES",
           "SELECTED", "select", "indexer", "indexer_logits", "indexer_topk", "quantize_kv_fp8"]
