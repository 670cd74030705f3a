"""ScatterMoE kernel ops on MI355X — same names and signatures as the reference's
scattermoe/kernels/ops.py, backed by libzmoe_hip (hand-written gfx950 HIP).

Each op is also registered as a mutating ``torch.library`` custom op with a fake
implementation (reference ops.py:21, :212, :274, :461), in the ``zmoe``
namespace, so ``torch.compile`` treats it as opaque.
"""

from __future__ import annotations

from typing import Optional

import torch

from zmoe import ops as _z

BLOCK_M = 128  # kept for API compatibility (reference ops.py:6); tiles are chosen per launch


def rowwise_sum_product(A, B, dtype=None):
    """Reference ops.py:9-18: out[t, j] = sum_h A[t, j, h] * B[t, h] (fp32 accumulation)."""
    assert A.dim() == 3
    assert B.dim() == 2
    assert A.size(0) == B.size(0)
    assert A.size(2) == B.size(1)
    T, F, H = A.shape
    output = torch.empty((T, F), device=A.device, dtype=dtype or A.dtype)
    rowwise_sum_product_compileable(output, A, B)
    return output


@torch.library.custom_op("zmoe::rowwise_sum_product", mutates_args={"output"})
def rowwise_sum_product_compileable(output: torch.Tensor, A: torch.Tensor, B: torch.Tensor) -> None:
    _z.rowwise_sum_product(A, B, out=output)


@rowwise_sum_product_compileable.register_fake
def _(output: torch.Tensor, A: torch.Tensor, B: torch.Tensor) -> None:
    return None


def scatter2scatter(X, W, sorted_expert_idxs, sorted_scattered_idxs, k, b=None, x_grouped=False, y_grouped=False,
                    out=None, expert_offsets=None):
    """Reference ops.py:192-209 (grouped GEMM). ``expert_offsets`` is optional:
    when absent it is derived from ``sorted_expert_idxs`` on the device."""
    assert sorted_scattered_idxs.size(0) == sorted_expert_idxs.size(0)
    assert sorted_scattered_idxs.size(0) == X.size(0) * k
    y_dim = W.size(-1)
    L_scattered = sorted_expert_idxs.size(0)
    if out is None:
        output = torch.empty((L_scattered, y_dim), device=X.device, dtype=X.dtype)
    else:
        assert out.size(0) == L_scattered and out.size(1) == y_dim
        output = out
    scatter2scatter_compileable(output, W, X, k, sorted_expert_idxs, sorted_scattered_idxs, b, x_grouped, y_grouped,
                                expert_offsets)
    return output


@torch.library.custom_op("zmoe::scatter2scatter", mutates_args={"output"})
def scatter2scatter_compileable(output: torch.Tensor, W: torch.Tensor, X: torch.Tensor, k: int,
                                sorted_expert_idxs: torch.Tensor, sorted_scattered_idxs: torch.Tensor,
                                b: Optional[torch.Tensor], x_grouped: bool, y_grouped: bool,
                                expert_offsets: Optional[torch.Tensor]) -> None:
    _z.scatter2scatter(X, W, sorted_expert_idxs, sorted_scattered_idxs, k, b=b, x_grouped=x_grouped,
                       y_grouped=y_grouped, out=output, expert_offsets=expert_offsets)


@scatter2scatter_compileable.register_fake
def _(output, W, X, k, sorted_expert_idxs, sorted_scattered_idxs, b, x_grouped, y_grouped, expert_offsets) -> None:
    return None


def group_bwd_W(DY, X, expert_offsets, E, has_bias=False):
    """Reference ops.py:263-271: returns (DW [E, K, N] as a view of a contiguous
    [E, N, K] buffer, Db [E, N] or None). Experts with no rows get zeros."""
    DWt = torch.empty((E, DY.size(-1), X.size(-1)), device=DY.device, dtype=DY.dtype)
    DW = DWt.permute(0, 2, 1)
    Db = torch.empty((E, DY.size(-1)), device=DY.device, dtype=DY.dtype) if has_bias else None
    groupXtY_compileable(E, DW, Db, DY, X, expert_offsets)
    return DW, Db


@torch.library.custom_op("zmoe::groupXtY", mutates_args={"DW", "Db"})
def groupXtY_compileable(E: int, DW: torch.Tensor, Db: Optional[torch.Tensor], DY: torch.Tensor, X: torch.Tensor,
                         expert_offsets: torch.Tensor) -> None:
    DWt = DW.permute(0, 2, 1)
    if not DWt.is_contiguous():
        raise ValueError("groupXtY: DW must be the permuted view of a contiguous [E, N, K] tensor")
    _z.group_bwd_w(DY, X, expert_offsets, E, has_bias=Db is not None, out=DWt, out_bias=Db)


@groupXtY_compileable.register_fake
def _(E, DW, Db, DY, X, expert_offsets) -> None:
    return None


def group(A, sorted_expert_idxs, coeff=None, fan_out=1, out=None):
    """Reference ops.py:449-458: Y[n] = A[idx[n] // fan_out] * coeff[idx[n]]."""
    N = sorted_expert_idxs.size(0)
    K = A.size(1)
    assert A.size(0) * fan_out == N
    Y = out if out is not None else torch.empty((N, K), dtype=A.dtype, device=A.device)
    group_compileable(A, K, N, Y, coeff, coeff is not None, fan_out, sorted_expert_idxs)
    return Y


@torch.library.custom_op("zmoe::group", mutates_args={"Y"})
def group_compileable(A: torch.Tensor, K: int, N: int, Y: torch.Tensor, coeff: Optional[torch.Tensor],
                      has_coeff: bool, fan_out: int, sorted_expert_idxs: torch.Tensor) -> None:
    _z.group(A, sorted_expert_idxs, coeff=coeff if has_coeff else None, fan_out=fan_out, out=Y)


@group_compileable.register_fake
def _(A, K, N, Y, coeff, has_coeff, fan_out, sorted_expert_idxs) -> None:
    return None
