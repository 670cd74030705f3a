"""Autograd functions for the dense layers around the routed experts.

The reference computes the gate projection (modeling/moe_gate.py:26) and the shared
expert (modeling/expert_layer.py:23-24) as plain nn.Linear / F.linear under torch
autograd. Here the forward GEMMs and input grads stay library GEMMs (hipBLASLt
through torch), while the weight grads — small outputs reduced over all T tokens,
which one library launch spreads over only a few dozen tiles — run as the split-K
``zmoe_dense_wgrad`` (fp32 partials, fixed-order sum, one rounding). The shared
expert's SwiGLU is one fused HIP pass each way (``zmoe_swiglu`` /
``zmoe_swiglu_backward``) and its up and gate projections run as one GEMM.

bf16 CUDA tensors with 16-byte rows take these paths; other dtypes and widths use plain
torch ops, as the reference does.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from . import library as zl


def _fused(x, *ws) -> bool:
    """bf16 CUDA operands whose widths are whole 16-byte chunks (8 elements) take the HIP path:
    x's last dim and both dims of each [out, in] weight."""
    return (all(t.is_cuda and t.dtype == torch.bfloat16 for t in (x, *ws)) and x.shape[-1] % 8 == 0
            and all(w.shape[0] % 8 == 0 and w.shape[1] % 8 == 0 for w in ws))


class _Linear(torch.autograd.Function):
    """y = x W^T for x [M, K], W [N, K]."""

    @staticmethod
    def forward(ctx, x2, W):
        ctx.save_for_backward(x2, W)
        return F.linear(x2, W)

    @staticmethod
    def backward(ctx, dy):
        x2, W = ctx.saved_tensors
        dy = dy.contiguous()
        dx = dy @ W if ctx.needs_input_grad[0] else None
        dW = zl.dense_wgrad(dy, x2) if ctx.needs_input_grad[1] else None
        return dx, dW


def linear(x: torch.Tensor, W: torch.Tensor) -> torch.Tensor:
    """F.linear(x, W) without bias; the weight grad goes through the split-K kernel."""
    if not _fused(x, W):
        return F.linear(x, W)
    lead = x.shape[:-1]
    y = _Linear.apply(x.reshape(-1, x.shape[-1]), W)
    return y.view(*lead, W.shape[0])


class _SwiGLUMLP(torch.autograd.Function):
    """down(silu(gate(x)) * up(x)) (expert_layer.py:23-24) for x [M, d]."""

    @staticmethod
    def forward(ctx, x2, W_gate, W_up, W_down):
        f = W_up.shape[0]
        W_cat = torch.cat([W_up, W_gate], dim=0)     # [2f, d]: H = [up | gate], the GLU layout
        H = F.linear(x2, W_cat)
        A = zl.swiglu(H)                              # silu(gate) * up, one rounding
        y = F.linear(A, W_down)
        ctx.save_for_backward(x2, W_cat, W_down, H, A)
        ctx.f = f
        return y

    @staticmethod
    def backward(ctx, dy):
        x2, W_cat, W_down, H, A = ctx.saved_tensors
        f = ctx.f
        dy = dy.contiguous()
        dA = dy @ W_down                              # [M, f]
        dW_down = zl.dense_wgrad(dy, A)               # [d, f]
        dH = zl.swiglu_backward(dA, H)                # [M, 2f] = [d up | d gate]
        dx = dH @ W_cat
        dW_cat = zl.dense_wgrad(dH, x2)               # [2f, d]
        return dx, dW_cat[f:], dW_cat[:f], dW_down


def swiglu_mlp(x: torch.Tensor, W_gate: torch.Tensor, W_up: torch.Tensor, W_down: torch.Tensor) -> torch.Tensor:
    if not _fused(x, W_gate, W_up, W_down):
        return F.linear(F.silu(F.linear(x, W_gate)) * F.linear(x, W_up), W_down)
    lead = x.shape[:-1]
    y = _SwiGLUMLP.apply(x.reshape(-1, x.shape[-1]), W_gate, W_up, W_down)
    return y.view(*lead, W_down.shape[0])


class _RMSNormRows(torch.autograd.Function):
    """x = ZeroCenteredRMSNorm(hidden)[rows] (zRMSNorm.py:10-17, then moe_layer.py:39-42)."""

    @staticmethod
    def forward(ctx, hidden2, weight, eps: float, rows):
        y, rstd = zl.rmsnorm_rows(hidden2, weight, eps, rows)
        ctx.save_for_backward(hidden2, weight, rstd, rows if rows is not None else torch.empty(0))
        ctx.has_rows = rows is not None
        return y

    @staticmethod
    def backward(ctx, dy):
        hidden2, weight, rstd, rows = ctx.saved_tensors
        dx, dw = zl.rmsnorm_rows_backward(dy.contiguous(), hidden2, rows if ctx.has_rows else None, rstd, weight)
        return dx, dw, None, None


def rmsnorm_rows(hidden: torch.Tensor, weight: torch.Tensor, eps: float,
                 rows: Optional[torch.Tensor] = None) -> torch.Tensor:
    """ZeroCenteredRMSNorm of ``hidden`` [..., d], gathered at flat rows ``rows`` (None: all
    rows, keeping hidden's shape; else [len(rows), d]). One HIP pass each way."""
    d = hidden.shape[-1]
    flat = hidden.reshape(-1, d)
    y = _RMSNormRows.apply(flat, weight, float(eps), rows)
    return y.view(hidden.shape) if rows is None else y
