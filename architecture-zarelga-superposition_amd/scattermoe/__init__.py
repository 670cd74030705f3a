"""ScatterMoE interface (reference scattermoe/__init__.py) on MI355X.

The compute runs in libzmoe_hip (hand-written gfx950 HIP); importing this
package patches nothing else. The reference's ``utils`` subpackage (Hugging
Face class replacement) is not on the MoE-layer path and is not provided.
"""

from .parallel_experts import flatten_sort_count, parallel_linear, ParallelExperts
from . import parallel_experts
from . import kernels
from . import mlp

__all__ = [
    "flatten_sort_count",
    "parallel_linear",
    "ParallelExperts",
    "parallel_experts",
    "kernels",
    "mlp",
]
