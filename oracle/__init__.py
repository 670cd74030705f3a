"""CPU oracle for the MoE-layer hot path.

TEST INFRASTRUCTURE ONLY. This package is a checker, never part of the product:
only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import it. The HIP product path never routes through it and has no CPU
fallback.
"""

from .moe_oracle import *  # noqa: F401,F403
