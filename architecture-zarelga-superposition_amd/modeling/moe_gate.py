"""Aux-loss-free sigmoid router (reference modeling/moe_gate.py:5-36) on MI355X.

The gate projection is a library GEMM (its weight grad the split-K HIP kernel,
zmoe.functional.linear); the rest of the routing — sigmoid, +bias for selection, top-k, gather of the unbiased
probabilities and L1 renormalisation — is one HIP kernel (zmoe_route_topk) whose
backward is the analytic gradient of the same expression.

Contract where the reference leaves order unspecified (topk(sorted=False)):
slots come in (biased score desc, expert asc) order and NaN ranks first, as in
torch.topk. Under bf16 logits the probabilities are rounded to bf16 before the
bias add, as the reference's bf16 sigmoid does under autocast.
"""

import torch
import torch.nn as nn

from zmoe import functional as _zf
from zmoe import library as _zl


class RouteTopK(torch.autograd.Function):
    """(logits [T, E], expert_biases [E], k) -> (topk_idx [T, k] int64, topk_weight [T, k] f32)."""

    @staticmethod
    def forward(ctx, logits, expert_biases, k: int):
        idx, w, p = _zl.route_topk(logits, expert_biases, k, logits.dtype == torch.bfloat16)
        ctx.save_for_backward(p, idx)
        ctx.num_experts = logits.shape[-1]
        ctx.like = logits.new_empty(0)                    # the logits' dtype and device
        ctx.mark_non_differentiable(idx)
        return idx, w

    @staticmethod
    def backward(ctx, d_idx, d_weight):
        if d_weight is None:
            return None, None, None
        p, idx = ctx.saved_tensors
        d_logits = _zl.route_topk_backward(d_weight, p, idx, ctx.num_experts, ctx.like)
        return d_logits, None, None


class MoEGate(nn.Module):
    def __init__(self, config):
        super().__init__()
        self.config = config
        self.top_k = config.n_experts_per_token
        self.n_routed_experts = config.n_routed_experts
        self.gating_dim = config.hidden_size
        self.weight = nn.Parameter(torch.empty((self.n_routed_experts, self.gating_dim)))
        self.register_buffer("expert_biases", torch.zeros(self.n_routed_experts))
        self.reset_parameters()

    def reset_parameters(self):
        nn.init.normal_(self.weight, mean=0.0, std=self.config.initializer_range)

    def forward(self, hidden_states):
        bsz, seq_len, h = hidden_states.shape
        hidden_states = hidden_states.view(-1, h)
        gate_output = _zf.linear(hidden_states, self.weight)                     # moe_gate.py:26
        topk_idx, topk_weight = RouteTopK.apply(gate_output, self.expert_biases, self.top_k)  # :27-34
        return topk_idx.view(bsz, seq_len, -1), topk_weight.view(bsz, seq_len, -1)
