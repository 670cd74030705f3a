"""MoE sublayer (reference modeling/moe_layer.py:11-59) on MI355X.

Same submodules, parameters and state-dict keys as the reference:
``gate`` (MoEGate), ``shared_experts`` (ExpertMLP), ``routed_experts`` (GLUMLP).
The optional unpad around the layer (the reference uses flash-attn's
index_first_axis) is a torch gather; the re-pad of the output (pad_input) is folded
into the routed experts' combine pass, which writes the padded layout directly.
"""

import torch
import torch.nn as nn

from scattermoe.mlp import GLUMLP

from .expert_layer import ExpertMLP
from .moe_gate import MoEGate


def index_first_axis(x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """Rows ``indices`` of ``x`` [N, ...] (flash_attn.bert_padding.index_first_axis)."""
    return x.index_select(0, indices)


def pad_input(x: torch.Tensor, indices: torch.Tensor, batch: int, seqlen: int) -> torch.Tensor:
    """Scatter rows back into a zero [batch, seqlen, ...] tensor (flash_attn pad_input)."""
    out = torch.zeros((batch * seqlen, *x.shape[1:]), dtype=x.dtype, device=x.device)
    out[indices] = x
    return out.view(batch, seqlen, *x.shape[1:])


class MoELayer(nn.Module):
    def __init__(self, config):
        super().__init__()
        self.config = config
        self.n_experts_per_token = config.n_experts_per_token
        self.gate = MoEGate(config)

        shared_intermediate = config.intermediate_size * config.n_shared_experts
        # As in the reference, n_shared_experts = 0 still yields a shared expert:
        # ExpertMLP treats intermediate_size=0 as "use config.intermediate_size"
        # (expert_layer.py:10), and forward always adds its output (moe_layer.py:47-53).
        self.shared_experts = ExpertMLP(config, intermediate_size=shared_intermediate)

        self.routed_experts = GLUMLP(
            input_size=config.hidden_size,
            hidden_size=config.intermediate_size,
            num_experts=config.n_routed_experts,
            top_k=config.n_experts_per_token,
            activation=nn.SiLU(),
        )
        # GLUMLP's ParallelExperts init at std 0.02; re-init at the config's 1/sqrt(d)
        # (moe_layer.py:27-36).
        self.reset_routed_expert_parameters()

    def reset_routed_expert_parameters(self):
        std = self.config.initializer_range
        nn.init.normal_(self.routed_experts.experts.weight, mean=0.0, std=std)
        nn.init.normal_(self.routed_experts.output_experts.weight, mean=0.0, std=std)

    def forward(self, hidden_states, unpad_indices=None):
        if unpad_indices is not None:
            bsz, seq_len = hidden_states.shape[:2]
            flat = hidden_states.reshape(bsz * seq_len, hidden_states.shape[-1])
            x = index_first_axis(flat, unpad_indices).unsqueeze(0)
        else:
            x = hidden_states

        topk_idx, topk_weight = self.gate(x)
        shared_output = self.shared_experts(x)

        flat_topk_idx = topk_idx.reshape(-1, self.n_experts_per_token)
        flat_topk_weight = topk_weight.reshape(-1, self.n_experts_per_token)
        # out = shared_output + routed_output (moe_layer.py:48-53), the sum formed in the
        # routed experts' combine pass, which also writes the re-padded layout (:55-56)
        # directly when unpad_indices is given
        if unpad_indices is None:
            return self.routed_experts(x, flat_topk_weight, flat_topk_idx, residual=shared_output), topk_idx
        out = self.routed_experts(x, flat_topk_weight, flat_topk_idx, residual=shared_output,
                                  pad=(unpad_indices, bsz * seq_len))
        topk_idx = pad_input(topk_idx.squeeze(0), unpad_indices, bsz, seq_len)
        return out.view(bsz, seq_len, -1), topk_idx
