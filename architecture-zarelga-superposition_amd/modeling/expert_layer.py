"""Shared expert (reference modeling/expert_layer.py:5-24): dense SwiGLU.

Its three bias-free projections are dense GEMMs (hipBLASLt through torch; the up
and gate projections as one GEMM), the SwiGLU is a fused HIP pass and the weight
grads are split-K HIP GEMMs (zmoe.functional.swiglu_mlp). State-dict keys
gate_proj / up_proj / down_proj are unchanged.
"""

import torch.nn as nn

from zmoe import functional as _zf


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
        # down_proj(act_fn(gate_proj(x)) * up_proj(x)), expert_layer.py:23-24
        return _zf.swiglu_mlp(x, self.gate_proj.weight, self.up_proj.weight, self.down_proj.weight)
