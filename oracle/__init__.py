"""CPU oracle for gorelaxor's Q8_0 hot path (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker. The product
(gorelaxor_amd) never imports it.
"""
from .oracle import *  # noqa: F401,F403
