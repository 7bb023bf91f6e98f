"""CPU oracle for the quantized matmul path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import this package. The product path (``brimkern_amd``) never does.
"""
from .brik_oracle import *  # noqa: F401,F403
