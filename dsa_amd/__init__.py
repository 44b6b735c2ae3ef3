"""MI355X-native DSA sparse-MLA attention forward (drop-in for ``dsa.forward``).

Public surface mirrors the reference package (dsa/__init__.py:2-5):
``forward``, ``Tuning``, ``CASE_SHAPES``, ``SELECTED``; plus ``merge`` (the
standalone FP32 split merge) and ``select`` (the plan for a shape).
"""
from .api import forward, merge, plan_call
from .config import CASE_SHAPES, SELECTED, Tuning, select

__all__ = ["forward", "merge", "plan_call", "Tuning", "CASE_SHAPES", "SELECTED", "select"]
