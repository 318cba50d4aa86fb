"""CPU oracle for the gstar_evict eviction path (test infrastructure only).

Nothing in the product imports this package. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg use it, and
only as the checker or as the timed CPU baseline, never as a fallback for the
HIP path.
"""
from .evict_oracle import *  # noqa: F401,F403
