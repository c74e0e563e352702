"""TEST INFRASTRUCTURE: ctypes binding of the scalar C oracle (liboracle.so).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this package. It restates the reference's shader semantics on the CPU and is
never part of the product path.
"""
from .binding import ORACLE_LIB, Oracle, oracle  # noqa: F401
