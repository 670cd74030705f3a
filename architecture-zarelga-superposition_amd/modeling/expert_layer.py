"""Shared expert (reference modeling/expert_layer.py:5-24): dense SwiGLU.

Its three bias-free projections are plain dense GEMMs and run on torch
(hipBLASLt); state-dict keys gate_proj / up_proj / down_proj are unchanged.
"""

import torch.nn as nn


class ExpertMLP(nn.Module):
    def __init__(self, config, intermediate_size=None):
        super().__init__()
        self.config = config
        self.hidden_size = config.hidden_size
        self.intermediate_size = intermediate_size or config.intermediate_size
        self.initializer_range = config.initializer_range
        self.gate_proj = nn.Linear(self.hidden_size, self.intermediate_size, bias=False)
        self.up_proj = nn.Linear(self.hidden_size, self.intermediate_size, bias=False)
        self.down_proj = nn.Linear(self.intermediate_size, self.hidden_size, bias=False)
        self.act_fn = nn.SiLU()
        self.reset_parameters()

    def reset_parameters(self):
        nn.init.normal_(self.gate_proj.weight, mean=0.0, std=self.initializer_range)
        nn.init.normal_(self.up_proj.weight, mean=0.0, std=self.initializer_range)
        nn.init.normal_(self.down_proj.weight, mean=0.0, std=self.initializer_range)

    def forward(self, x):
        return self.down_proj(self.act_fn(self.gate_proj(x)) * self.up_proj(x))
