"""CPU oracle for KORE's fused layer ops -- TEST INFRASTRUCTURE ONLY.

A C restatement of the reference Rust CPU functions (kore_oracle.c), loaded
through ctypes.  Only tests/, ``__graft_entry__.smoke()`` and bench.py's
``cpu_baseline`` leg may import this package; the product never does.
"""
from .oracle import *  # noqa: F401,F403
