"""ScatterMoE interface (reference scattermoe/__init__.py) on MI355X.

The compute runs in libzmoe_hip (hand-written gfx950 HIP); importing this
package patches nothing else.
"""

from .parallel_experts import flatten_sort_count, parallel_linear, ParallelExperts
from . import parallel_experts
from . import kernels
from . import mlp
from . import utils

__all__ = [
    "flatten_sort_count",
    "parallel_linear",
    "ParallelExperts",
    "parallel_experts",
    "kernels",
    "mlp",
    "utils",
]
