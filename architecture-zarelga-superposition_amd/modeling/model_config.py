"""MoE fields of the reference's ModelConfig (modeling/model_config.py:45-185).

Only the fields the MoE layer reads are kept, with the same names, defaults,
derived values and validation; any object carrying these attributes (such as
the reference's own ModelConfig) can be passed to MoEGate / MoELayer.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field


@dataclass
class ModelConfig:
    hidden_size: int = 512
    # fine-grained MoE: 32 routed + 2 shared experts, top-2 routed (model_config.py:53-58)
    intermediate_size: int = 160
    n_experts: int = 34
    n_shared_experts: int = 2
    n_experts_per_token: int = 2
    n_routed_experts: int = field(init=False)
    initializer_range: float = field(init=False)

    def __post_init__(self):
        self.n_routed_experts = self.n_experts - self.n_shared_experts          # :135
        self.initializer_range = 1.0 / math.sqrt(self.hidden_size)              # :138
        if self.n_routed_experts <= 0:
            raise ValueError("n_experts must be greater than n_shared_experts.")
        if self.n_experts_per_token <= 0:
            raise ValueError("n_experts_per_token must be positive.")
        if self.n_experts_per_token > self.n_routed_experts:
            raise ValueError("n_experts_per_token cannot exceed n_routed_experts.")
