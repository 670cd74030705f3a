"""Expert MLPs on MI355X — the reference's scattermoe/mlp.py interface.

``GLUMLP`` keeps the reference's modules and parameters (``experts`` W1
[E, 2f, d], ``output_experts`` W2 [E, d, f]) and, by default, runs them through
one fused autograd function over libzmoe_hip:

  forward : sort -> W1 GEMM with SwiGLU epilogue (H, A) -> W2 GEMM scattered to
            slot order (Y) -> weighted combine
  backward: combine backward (d_gates + grouped grad) -> W2 input-grad GEMM with
            SwiGLU-backward epilogue (dH) -> dW2, dW1 (x gathered in-kernel)
            -> W1 input-grad GEMM -> k-sum

which computes the same values as the reference's composition (mlp.py:74-95 via
ParallelLinear). ``fused=False`` runs that composition through ParallelExperts.
"""

from __future__ import annotations

import torch
from torch import nn

from zmoe import library as _zl

from .parallel_experts import ParallelExperts, flatten_sort_count


def _compute_dtype(x: torch.Tensor) -> torch.dtype:
    return torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled() else x.dtype


def _fused_widths_ok(d: int, f: int, dtype: torch.dtype) -> bool:
    """The fused GLU kernels move rows as 16-byte chunks: d and f must be multiples of 8
    (bf16) or 4 (fp32) elements. Other widths run the module composition, whose ops take
    any width (through zero-padded copies)."""
    v = 8 if dtype == torch.bfloat16 else 4
    return d % v == 0 and f % v == 0


class GLUExpertsFunction(torch.autograd.Function):
    """y = sum_j gates[:, j] * W2[e_j] silu(W1g[e_j] x) * (W1h[e_j] x) for every token.

    (x, gates, expert_idxs, W1, W2, k, num_experts, residual=None, pad_rows=None,
    pad_total=0) -> (y, expert_offsets). ``residual`` [T, d] is added in the combine pass
    (moe_layer.py:53 adds the shared expert's output); with ``pad_rows`` the output is the
    padded [pad_total, d] (moe_layer.py:55-56). ``expert_offsets`` is the sort's (not
    differentiable). Every launch is a ``zmoe::`` custom op, so torch.compile traces
    through this function without a graph break.
    """

    @staticmethod
    def forward(ctx, x, gates, expert_idxs, W1, W2, k: int, num_experts: int, residual=None, pad_rows=None,
                pad_total: int = 0):
        se, ss, off, inv = _zl.flatten_sort_count(expert_idxs, num_experts)
        H, A = _zl.glu_w1_forward(x, W1, se, ss, off, k, None)                   # mlp.py:80-86
        Y = _zl.grouped_mm(A, W2.permute(0, 2, 1), se, ss, 1, True, False, off,
                           "scatter2scatter")                                    # mlp.py:87-93
        out = _zl.combine(Y, gates, k, residual, pad_rows, pad_total)            # parallel_experts.py:50-52
        ctx.has_residual = residual is not None
        ctx.save_for_backward(x, gates, W1, W2, se, ss, off, inv, H, A, Y, pad_rows)
        ctx.k = k
        ctx.num_experts = num_experts
        ctx.mark_non_differentiable(off)
        ctx.set_materialize_grads(False)  # no zero-filled grad for off
        return out, off

    @staticmethod
    def backward(ctx, dout, d_off):
        if dout is None:  # out took no part in the loss
            return (None,) * 10
        x, gates, W1, W2, se, ss, off, inv, H, A, Y, pad_rows = ctx.saved_tensors
        k, E = ctx.k, ctx.num_experts
        dout = dout.to(x.dtype)
        d_gates, dYg = _zl.combine_backward(Y, dout, gates, inv, pad_rows)  # parallel_experts.py:80-97
        dH = _zl.glu_w2_backward_dh(dYg, W2, H, se, off)                        # :112-120 + silu*mul backward
        dW2 = _zl.group_bwd_w(dYg, A, off, E, None, 1)                           # :98-110 (W2)
        dW1 = _zl.group_bwd_w(dH, x, off, E, ss, k)                              # :98-110 (W1, x gathered)
        dXe = _zl.grouped_mm(dH, W1, se, ss, 1, True, False, off, "scatter2scatter")  # :112-120 (W1)
        dx = _zl.sum_k(dXe, k, None)                                             # :125
        d_res = None
        if ctx.has_residual and ctx.needs_input_grad[7]:
            d_res = dout if pad_rows is None else dout.index_select(0, pad_rows)
        return dx, d_gates.to(gates.dtype), None, dW1, dW2, None, None, d_res, None, None


class MLP(nn.Module):
    """Reference scattermoe/mlp.py:6-49 (non-GLU expert MLP)."""

    def __init__(self, input_size, hidden_size, num_experts, top_k, bias=False, activation=None):
        super(MLP, self).__init__()
        self.num_experts = num_experts
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.experts = ParallelExperts(num_experts, input_size, hidden_size, bias=bias)
        self.output_experts = ParallelExperts(num_experts, hidden_size, input_size, bias=bias)
        self.top_k = min(top_k, self.num_experts)
        self.activation = activation

    def extra_repr(self):
        return "k={}".format(self.top_k)

    def forward(self, x: torch.Tensor, expert_p: torch.Tensor, expert_idxs: torch.Tensor):
        x_shape = x.size()
        x = x.view(-1, x_shape[-1])
        sorted_expert_idxs, sorted_scattered_idxs, expert_offsets = flatten_sort_count(
            expert_idxs, num_experts=self.num_experts)
        h = self.experts(x, self.top_k, sorted_expert_idxs, sorted_scattered_idxs, expert_offsets,
                         grouped_out=True)
        h = self.activation(h)
        y = self.output_experts(h, 1, sorted_expert_idxs, sorted_scattered_idxs, expert_offsets,
                                grouped_in=True, gates=expert_p)
        y = y.view(*x_shape[:-1], y.size(-1))
        return y


class GLUMLP(nn.Module):
    """Reference scattermoe/mlp.py:51-95 (SwiGLU expert MLP)."""

    def __init__(self, input_size, hidden_size, num_experts, top_k, bias=False, activation=nn.SiLU(), fused=True):
        super(GLUMLP, self).__init__()
        self.num_experts = num_experts
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.experts = ParallelExperts(num_experts, input_size, 2 * hidden_size, bias=bias)
        self.output_experts = ParallelExperts(num_experts, hidden_size, input_size, bias=bias)
        self.top_k = min(top_k, self.num_experts)
        self.activation = activation
        # The fused kernels implement SiLU-gated units without expert biases.
        self.fused = fused and not bias and isinstance(activation, nn.SiLU)
        # expert_offsets of the last forward's sort (device tensor; not module state)
        self.last_expert_offsets = None

    def extra_repr(self):
        return "k={}".format(self.top_k)

    def forward(self, x: torch.Tensor, expert_p: torch.Tensor, expert_idxs: torch.Tensor, residual=None, pad=None):
        """mlp.py:74-95. Two arguments beyond the reference signature (their defaults keep its
        behaviour): ``residual`` is added to the output, in the combine pass on the fused
        path; ``pad = (rows, total)`` returns the padded [total, d] output whose row rows[t]
        is token t's (moe_layer.py:55-56), written by the combine in place."""
        x_shape = x.size()
        x = x.view(-1, x_shape[-1])
        if self.fused and _fused_widths_ok(x_shape[-1], self.hidden_size, _compute_dtype(x)):
            dtype = _compute_dtype(x)
            res = None if residual is None else residual.reshape(-1, residual.shape[-1]).to(dtype)
            rows, total = (None, 0) if pad is None else (pad[0], int(pad[1]))
            y, self.last_expert_offsets = GLUExpertsFunction.apply(
                x.to(dtype), expert_p, expert_idxs, self.experts.compute_weight(dtype),
                self.output_experts.compute_weight(dtype), self.top_k, self.num_experts, res, rows, total)
            return y if pad is not None else y.view(*x_shape[:-1], y.size(-1))
        sorted_expert_idxs, sorted_scattered_idxs, expert_offsets = flatten_sort_count(
            expert_idxs, num_experts=self.num_experts)
        self.last_expert_offsets = expert_offsets
        h, gates = self.experts(x, self.top_k, sorted_expert_idxs, sorted_scattered_idxs, expert_offsets,
                                grouped_out=True).chunk(2, dim=-1)
        h = self.activation(gates) * h
        y = self.output_experts(h, 1, sorted_expert_idxs, sorted_scattered_idxs, expert_offsets,
                                grouped_in=True, gates=expert_p)
        y = y.view(*x_shape[:-1], y.size(-1))
        y = y if residual is None else residual + y
        if pad is not None:
            rows, total = pad
            y = torch.zeros((int(total), y.size(-1)), dtype=y.dtype, device=y.device).index_copy(
                0, rows, y.reshape(-1, y.size(-1)))
        return y
