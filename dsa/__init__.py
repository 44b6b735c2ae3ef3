"""The reference's import name for this operator, so that reference callers
switch without edits: ``from dsa import forward`` (reference README.md:70,
tools/review.py:81, tools/check_bitwise.py:13) and ``dsa.Tuning``,
``dsa.CASE_SHAPES``, ``dsa.SELECTED`` (dsa/__init__.py:2-5) resolve to the
MI355X implementation in ``dsa_amd``.  Nothing else lives here.
"""
from dsa_amd import *  # noqa: F401,F403
from dsa_amd import __all__  # noqa: F401
