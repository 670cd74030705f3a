"""The layer's HIP entry points as ``torch.library`` custom ops (namespace ``zmoe``).

The reference keeps its layer compile-friendly by registering its kernels as custom
ops with fake implementations (scattermoe/kernels/ops.py:21, :212, :274, :461;
scattermoe/parallel_experts.py:6, :17) and compiles the whole forward
(main.py:929). These are the functional (non-mutating) ops that the autograd
functions of ``modeling.moe_layer``, ``scattermoe.mlp`` and ``zmoe.functional``
call: ``torch.compile`` sees each launch as one opaque node whose output shapes come
from the fake implementation, so tracing the layer needs no graph break and no host
sync. Each op runs the ``zmoe.ops`` wrapper of the same name (the C ABI through
ctypes) on the current stream.
"""

from __future__ import annotations

from typing import List, Optional

import torch

from . import ops as _z

_I64 = torch.int64
_F32 = torch.float32


def _empty(shape, like: torch.Tensor, dtype=None):
    return torch.empty(shape, dtype=dtype or like.dtype, device=like.device)


# ------------------------------------------------------------------ routing
@torch.library.custom_op("zmoe::route_topk", mutates_args=())
def route_topk(logits: torch.Tensor, expert_biases: torch.Tensor, k: int,
               round_probs_bf16: bool) -> List[torch.Tensor]:
    """moe_gate.py:27-34 from the logits: [idx int64, weight f32, prob f32], each [T, k]."""
    return list(_z.route_topk(logits, expert_biases, k, round_probs_bf16=round_probs_bf16))


@route_topk.register_fake
def _(logits, expert_biases, k, round_probs_bf16):
    T = logits.shape[0]
    return [_empty((T, k), logits, _I64), _empty((T, k), logits, _F32), _empty((T, k), logits, _F32)]


@torch.library.custom_op("zmoe::swiglu_route_backward", mutates_args=())
def swiglu_route_backward(dAs: torch.Tensor, Hs: torch.Tensor, d_gates: torch.Tensor, topk_prob: torch.Tensor,
                          topk_idx: torch.Tensor, num_experts: int) -> torch.Tensor:
    """[swiglu_backward(dAs, Hs) | d_logits] side by side in one [T, 2f + E] buffer: the
    shared expert's dH and the routing backward (autograd of moe_gate.py:27-34)."""
    T, two_f = Hs.shape
    G = torch.empty((T, two_f + num_experts), dtype=Hs.dtype, device=Hs.device)
    _z.swiglu_backward(dAs, Hs, out=G[:, :two_f])
    _z.route_topk_backward(d_gates, topk_prob, topk_idx, num_experts, Hs.dtype, out=G[:, two_f:])
    return G


@swiglu_route_backward.register_fake
def _(dAs, Hs, d_gates, topk_prob, topk_idx, num_experts):
    return _empty((Hs.shape[0], Hs.shape[1] + num_experts), Hs)


@torch.library.custom_op("zmoe::route_topk_backward", mutates_args=())
def route_topk_backward(d_weight: torch.Tensor, topk_prob: torch.Tensor, topk_idx: torch.Tensor, num_experts: int,
                        like: torch.Tensor) -> torch.Tensor:
    """d_logits [T, E] in ``like``'s dtype."""
    return _z.route_topk_backward(d_weight, topk_prob, topk_idx, num_experts, like.dtype)


@route_topk_backward.register_fake
def _(d_weight, topk_prob, topk_idx, num_experts, like):
    return _empty((topk_idx.shape[0], num_experts), like)


# ------------------------------------------------------------------ sort
@torch.library.custom_op("zmoe::flatten_sort_count", mutates_args=())
def flatten_sort_count(expert_idxs: torch.Tensor, num_experts: int) -> List[torch.Tensor]:
    """parallel_experts.py:21-28: [sorted_expert_idxs, sorted_scattered_idxs, expert_offsets,
    inverse int32]."""
    return list(_z.flatten_sort_count(expert_idxs, num_experts))


@flatten_sort_count.register_fake
def _(expert_idxs, num_experts):
    R = expert_idxs.numel()
    return [_empty((R,), expert_idxs, _I64), _empty((R,), expert_idxs, _I64),
            _empty((num_experts,), expert_idxs, _I64), _empty((R,), expert_idxs, torch.int32)]


# ------------------------------------------------------------------ grouped GEMMs
@torch.library.custom_op("zmoe::glu_w1_forward", mutates_args=())
def glu_w1_forward(x: torch.Tensor, W1: torch.Tensor, sorted_expert_idxs: torch.Tensor,
                   sorted_scattered_idxs: torch.Tensor, expert_offsets: torch.Tensor, k: int,
                   row_scale: Optional[torch.Tensor]) -> List[torch.Tensor]:
    """W1 grouped GEMM with the SwiGLU epilogue: [H [T*k, 2f], A [T*k, f]] (A scaled by
    ``row_scale`` when given)."""
    return list(_z.glu_w1_forward(x, W1, sorted_expert_idxs, sorted_scattered_idxs, expert_offsets, k,
                                  row_scale=row_scale))


@glu_w1_forward.register_fake
def _(x, W1, sorted_expert_idxs, sorted_scattered_idxs, expert_offsets, k, row_scale):
    R = x.shape[0] * k
    two_f = W1.shape[1]
    return [_empty((R, two_f), x), _empty((R, two_f // 2), x)]


@torch.library.custom_op("zmoe::grouped_mm", mutates_args=())
def grouped_mm(X: torch.Tensor, W: torch.Tensor, sorted_expert_idxs: torch.Tensor,
               sorted_scattered_idxs: torch.Tensor, k: int, x_grouped: bool, y_grouped: bool,
               expert_offsets: torch.Tensor, region: str) -> torch.Tensor:
    """scatter2scatter (ops.py:192-209) into a new [T*k, N] tensor; W the logical [E, K, N]."""
    return _z.scatter2scatter(X, W, sorted_expert_idxs, sorted_scattered_idxs, k, x_grouped=x_grouped,
                              y_grouped=y_grouped, expert_offsets=expert_offsets, region=region)


@grouped_mm.register_fake
def _(X, W, sorted_expert_idxs, sorted_scattered_idxs, k, x_grouped, y_grouped, expert_offsets, region):
    return _empty((sorted_expert_idxs.shape[0], W.shape[2]), X)


@torch.library.custom_op("zmoe::glu_w2_backward_dh", mutates_args=())
def glu_w2_backward_dh(dYg: torch.Tensor, W2: torch.Tensor, H: torch.Tensor, sorted_expert_idxs: torch.Tensor,
                       expert_offsets: torch.Tensor) -> torch.Tensor:
    """dH [T*k, 2f]: the W2 input-grad GEMM with the SwiGLU backward epilogue."""
    return _z.glu_w2_backward_dh(dYg, W2, H, sorted_expert_idxs, expert_offsets)


@glu_w2_backward_dh.register_fake
def _(dYg, W2, H, sorted_expert_idxs, expert_offsets):
    return _empty(H.shape, dYg)


def _wdt(DY: torch.Tensor, out_f32: bool) -> torch.dtype:
    return torch.float32 if out_f32 else DY.dtype


@torch.library.custom_op("zmoe::group_bwd_w", mutates_args=())
def group_bwd_w(DY: torch.Tensor, X: torch.Tensor, expert_offsets: torch.Tensor, num_experts: int,
                x_gather: Optional[torch.Tensor], x_div: int, out_f32: bool = False) -> torch.Tensor:
    """group_bwd_W (ops.py:263-271): DWt [E, N, K] (the parameter layout); ``out_f32``: fp32
    from the accumulators (bf16 operands, fp32 master weights)."""
    return _z.group_bwd_w(DY, X, expert_offsets, num_experts, x_gather=x_gather, x_div=x_div,
                          out_dtype=_wdt(DY, out_f32))[0]


@group_bwd_w.register_fake
def _(DY, X, expert_offsets, num_experts, x_gather, x_div, out_f32=False):
    return _empty((num_experts, DY.shape[1], X.shape[1]), DY, _wdt(DY, out_f32))


@torch.library.custom_op("zmoe::group_bwd_w_bias", mutates_args=())
def group_bwd_w_bias(DY: torch.Tensor, X: torch.Tensor, expert_offsets: torch.Tensor, num_experts: int,
                     x_gather: Optional[torch.Tensor], x_div: int) -> List[torch.Tensor]:
    """group_bwd_W with has_bias (ops.py:263-271, :430-438): [DWt [E, N, K], Db [E, N]]."""
    return list(_z.group_bwd_w(DY, X, expert_offsets, num_experts, has_bias=True, x_gather=x_gather, x_div=x_div))


@group_bwd_w_bias.register_fake
def _(DY, X, expert_offsets, num_experts, x_gather, x_div):
    return [_empty((num_experts, DY.shape[1], X.shape[1]), DY), _empty((num_experts, DY.shape[1]), DY)]


@torch.library.custom_op("zmoe::group_bwd_w_gather_dy", mutates_args=())
def group_bwd_w_gather_dy(DY: torch.Tensor, dy_gather: torch.Tensor, dy_div: int, X: torch.Tensor,
                          expert_offsets: torch.Tensor, num_experts: int, out_f32: bool = False) -> torch.Tensor:
    """Weight grads with DY's rows gathered in the kernel: DWt [E, N, K]."""
    return _z.group_bwd_w_gather_dy(DY, dy_gather, dy_div, X, expert_offsets, num_experts,
                                    out_dtype=_wdt(DY, out_f32))


@group_bwd_w_gather_dy.register_fake
def _(DY, dy_gather, dy_div, X, expert_offsets, num_experts, out_f32=False):
    return _empty((num_experts, DY.shape[1], X.shape[1]), DY, _wdt(DY, out_f32))


@torch.library.custom_op("zmoe::dense_wgrad", mutates_args=())
def dense_wgrad(DY: torch.Tensor, X: torch.Tensor, out_f32: bool = False) -> torch.Tensor:
    """DW [N, K] = DY^T X (the F.linear weight grad, split-K)."""
    return _z.dense_wgrad(DY, X, out_dtype=_wdt(DY, out_f32))


@dense_wgrad.register_fake
def _(DY, X, out_f32=False):
    return _empty((DY.shape[1], X.shape[1]), DY, _wdt(DY, out_f32))


# ------------------------------------------------------------------ row passes
@torch.library.custom_op("zmoe::combine", mutates_args=())
def combine(Y: torch.Tensor, gates: Optional[torch.Tensor], k: int, addend: Optional[torch.Tensor],
            out_rows: Optional[torch.Tensor], out_total: int) -> torch.Tensor:
    """out[t] = addend[t] + sum_j gates[t, j] Y[t*k + j] ([T, d], or the padded [out_total, d]
    when ``out_rows`` is given)."""
    return _z.combine(Y, gates, k, addend=addend, out_rows=out_rows, out_total=out_total if out_rows is not None
                      else None)


@combine.register_fake
def _(Y, gates, k, addend, out_rows, out_total):
    rows = out_total if out_rows is not None else Y.shape[0] // k
    return _empty((rows, Y.shape[1]), Y)


@torch.library.custom_op("zmoe::combine_backward", mutates_args=())
def combine_backward(Y: torch.Tensor, grad_out: torch.Tensor, gates: torch.Tensor, inverse: torch.Tensor,
                     grad_rows: Optional[torch.Tensor]) -> List[torch.Tensor]:
    """[d_gates [T, k] f32, gate-scaled grad rows [T*k, d] in sorted order]."""
    return list(_z.combine_backward(Y, grad_out, gates, inverse, grad_rows=grad_rows))


@combine_backward.register_fake
def _(Y, grad_out, gates, inverse, grad_rows):
    T, k = gates.shape
    return [_empty((T, k), gates, _F32), _empty((T * k, Y.shape[-1]), Y)]


@torch.library.custom_op("zmoe::sum_k", mutates_args=())
def sum_k(Xe: torch.Tensor, k: int, add0: Optional[torch.Tensor], out_f32: bool = False) -> torch.Tensor:
    """out[t] = sum_j Xe[t*k + j] (+ add0[t]) (parallel_experts.py:125); ``out_f32``: the fp32
    sum unrounded."""
    return _z.sum_k(Xe, k, add0=add0, out_dtype=torch.float32 if out_f32 else None)


@sum_k.register_fake
def _(Xe, k, add0, out_f32=False):
    return _empty((Xe.shape[0] // k, Xe.shape[1]), Xe, torch.float32 if out_f32 else None)


@torch.library.custom_op("zmoe::cast_bf16", mutates_args=())
def cast_bf16(src: torch.Tensor) -> torch.Tensor:
    """The bf16 compute copy of an fp32 tensor (fp32 master weights under bf16 autocast)."""
    return _z.cast_bf16(src).clone() if src.dtype == torch.bfloat16 else _z.cast_bf16(src)


@cast_bf16.register_fake
def _(src):
    return _empty(src.shape, src, torch.bfloat16)


@torch.library.custom_op("zmoe::swiglu", mutates_args=())
def swiglu(H: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up for H = [up | gate] (mlp.py:86, expert_layer.py:23-24)."""
    return _z.swiglu(H)


@swiglu.register_fake
def _(H):
    return _empty((H.shape[0], H.shape[1] // 2), H)


@torch.library.custom_op("zmoe::swiglu_backward", mutates_args=())
def swiglu_backward(dA: torch.Tensor, H: torch.Tensor) -> torch.Tensor:
    return _z.swiglu_backward(dA, H)


@swiglu_backward.register_fake
def _(dA, H):
    return _empty(H.shape, H)


@torch.library.custom_op("zmoe::swiglu_backward_gates", mutates_args=())
def swiglu_backward_gates(dA: torch.Tensor, H: torch.Tensor, row_scale: torch.Tensor,
                          slot_of_row: torch.Tensor) -> List[torch.Tensor]:
    """[dH [R, 2f], d_gates [R] f32 in slot order] of gate-scaled rows."""
    return list(_z.swiglu_backward_gates(dA, H, row_scale, slot_of_row))


@swiglu_backward_gates.register_fake
def _(dA, H, row_scale, slot_of_row):
    return [_empty(H.shape, H), _empty((H.shape[0],), H, _F32)]


@torch.library.custom_op("zmoe::rmsnorm_rows", mutates_args=())
def rmsnorm_rows(X: torch.Tensor, weight: torch.Tensor, eps: float, rows: Optional[torch.Tensor]) -> List[torch.Tensor]:
    """[Y [n, d], rstd [n] f32]: zRMSNorm.py:10-17 on rows ``rows`` of X."""
    return list(_z.rmsnorm_rows(X, weight, eps, rows))


@rmsnorm_rows.register_fake
def _(X, weight, eps, rows):
    n = X.shape[0] if rows is None else rows.numel()
    return [_empty((n, X.shape[1]), X), _empty((n,), X, _F32)]


@torch.library.custom_op("zmoe::rmsnorm_rows_backward", mutates_args=())
def rmsnorm_rows_backward(dY: torch.Tensor, X: torch.Tensor, rows: Optional[torch.Tensor], rstd: torch.Tensor,
                          weight: torch.Tensor) -> List[torch.Tensor]:
    """[dX [N, d] (zeros outside ``rows``), dweight]."""
    return list(_z.rmsnorm_rows_backward(dY, X, rows, rstd, weight))


@rmsnorm_rows_backward.register_fake
def _(dY, X, rows, rstd, weight):
    return [_empty(X.shape, X), _empty(weight.shape, weight)]
