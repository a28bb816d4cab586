"""MiniPrefix CPU oracle -- test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, and only to check results against it. The product path never
does.
"""
from .oracle import Oracle, OracleModel, load, ref_library  # noqa: F401
