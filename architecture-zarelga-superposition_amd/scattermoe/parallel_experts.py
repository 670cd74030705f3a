"""ParallelExperts on MI355X — the reference's scattermoe/parallel_experts.py
interface (names, signatures, parameters, autograd contract) over libzmoe_hip.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from zmoe import library as _zl
from zmoe import ops as _z

from . import kernels


@torch.library.custom_op("zmoe::bincount", mutates_args={})
def compileable_bincount(x: torch.Tensor, minlength: int) -> torch.Tensor:
    """Reference parallel_experts.py:6-15: per-expert counts without a host sync."""
    return _z.bincount(x, minlength)


@compileable_bincount.register_fake
def _(x: torch.Tensor, minlength: int) -> torch.Tensor:
    return torch.empty(minlength, dtype=torch.long, device=x.device)


def flatten_sort_count(expert_idxs: torch.Tensor, num_experts: int):
    """Reference parallel_experts.py:21-28 as one stable LDS counting sort.

    Returns (sorted_expert_idxs, sorted_scattered_idxs, expert_offsets); equal
    experts keep flat-slot order, offsets are inclusive ends.
    """
    se, ss, off, _ = _zl.flatten_sort_count(expert_idxs, num_experts)
    return se, ss, off


def flatten_sort_count_with_inverse(expert_idxs: torch.Tensor, num_experts: int):
    """flatten_sort_count plus inverse[slot] = sorted position (int32)."""
    return tuple(_zl.flatten_sort_count(expert_idxs, num_experts))


class ParallelLinear(torch.autograd.Function):
    """Reference parallel_experts.py:32-135, same saved tensors and 10-tuple grads."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, expert_weights: torch.Tensor, k: int, sorted_expert_idxs: torch.Tensor,
                sorted_scattered_idxs: torch.Tensor, expert_offsets: torch.Tensor,
                expert_biases: Optional[torch.Tensor] = None, gates: Optional[torch.Tensor] = None,
                grouped_in: bool = False, grouped_out: bool = False):
        output = kernels.ops.scatter2scatter(
            X=x, W=expert_weights, b=expert_biases, k=k, sorted_expert_idxs=sorted_expert_idxs,
            sorted_scattered_idxs=sorted_scattered_idxs, x_grouped=grouped_in, y_grouped=grouped_out,
            expert_offsets=expert_offsets)
        if gates is not None:
            output_expanded = output.view(gates.size(0), gates.size(1), output.size(-1))
            output = _zl.combine(output, gates, gates.size(1), None, None, 0)
        else:
            output_expanded = None
        ctx.save_for_backward(x, expert_weights, expert_biases, sorted_expert_idxs, sorted_scattered_idxs,
                              expert_offsets, gates, output_expanded)
        ctx.grouped_in = grouped_in
        ctx.grouped_out = grouped_out
        ctx.k = k
        return output

    @staticmethod
    def backward(ctx, grad_out: torch.Tensor):
        (x, expert_weights, expert_biases, sorted_expert_idxs, sorted_scattered_idxs, expert_offsets, gates,
         output_expanded) = ctx.saved_tensors
        k = ctx.k
        grouped_in, grouped_out = ctx.grouped_in, ctx.grouped_out
        grad_out = grad_out.to(x.dtype)

        if gates is not None:
            d_gates = kernels.ops.rowwise_sum_product(output_expanded, grad_out, dtype=gates.dtype)
            gates_flat = gates.flatten()
            gate_fan = gates.size(1)
            grouped_grad_out = output_expanded.flatten(0, 1)  # reuse the expanded buffer
        else:
            d_gates, gates_flat, gate_fan, grouped_grad_out = None, None, 1, None

        if grouped_out:
            grouped_grad_out = grad_out
        else:
            grouped_grad_out = kernels.ops.group(grad_out, sorted_scattered_idxs, fan_out=gate_fan,
                                                 coeff=gates_flat, out=grouped_grad_out)
        # dW: the x gather happens inside the wgrad kernel (no grouped copy of x).
        x_gather = None if grouped_in else sorted_scattered_idxs
        if expert_biases is None:
            DWt = _zl.group_bwd_w(grouped_grad_out, x, expert_offsets, expert_weights.size(0), x_gather, k)
            d_biases = None
        else:
            DWt, d_biases = _zl.group_bwd_w_bias(grouped_grad_out, x, expert_offsets, expert_weights.size(0),
                                                 x_gather, k)
        d_weights = DWt.permute(0, 2, 1)
        d_expanded_input = kernels.ops.scatter2scatter(
            X=grouped_grad_out, x_grouped=True, W=expert_weights.permute(0, 2, 1),
            sorted_expert_idxs=sorted_expert_idxs, sorted_scattered_idxs=sorted_scattered_idxs, k=1,
            y_grouped=grouped_in, expert_offsets=expert_offsets)
        if k == 1:
            d_input = d_expanded_input
        else:
            d_input = _zl.sum_k(d_expanded_input, k, None)
        return (d_input, d_weights, None, None, None, None, d_biases, d_gates, None, None)


def parallel_linear(inputs, expert_weights, k, sorted_expert_idxs, sorted_scattered_idxs, expert_offsets,
                    expert_biases=None, gates=None, grouped_in=False, grouped_out=False):
    """Reference parallel_experts.py:137-147."""
    return ParallelLinear.apply(inputs, expert_weights, k, sorted_expert_idxs, sorted_scattered_idxs, expert_offsets,
                                expert_biases, gates, grouped_in, grouped_out)


class ParallelExperts(nn.Module):
    """Reference parallel_experts.py:149-183: weight [E, out, in], optional bias [E, out]."""

    def __init__(self, num_experts, input_size, output_size, bias=False) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.empty(num_experts, output_size, input_size))
        if bias:
            self.bias = nn.Parameter(torch.empty(num_experts, output_size))
        else:
            self.bias = None
        self.num_experts = num_experts
        self.input_size = input_size
        self.output_size = output_size
        self.reset_parameters()

    def extra_repr(self):
        return "num_experts={}, input_size={}, output_size={}".format(self.num_experts, self.input_size,
                                                                     self.output_size)

    def reset_parameters(self) -> None:
        nn.init.normal_(self.weight, std=0.02)
        if self.bias is not None:
            nn.init.zeros_(self.bias)

    def compute_weight(self, dtype: torch.dtype) -> torch.Tensor:
        """The weight in the compute dtype (a cast copy when autocast asks for one)."""
        return self.weight if self.weight.dtype == dtype else self.weight.to(dtype)

    def forward(self, inputs, k, sorted_expert_idxs, sorted_scattered_idxs, expert_offsets, gates=None,
                grouped_in=False, grouped_out=False):
        dtype = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled() else inputs.dtype
        inputs = inputs.to(dtype)
        bias = None if self.bias is None else self.bias.to(dtype)
        return parallel_linear(inputs, self.compute_weight(dtype).permute(0, 2, 1), k, sorted_expert_idxs,
                               sorted_scattered_idxs, expert_offsets, expert_biases=bias, gates=gates,
                               grouped_in=grouped_in, grouped_out=grouped_out)
