"""torch-facing wrappers of the libzmoe_hip C ABI.

Every function checks devices, dtypes and shapes, allocates its outputs with
torch on the input's device (torch owns all memory), and enqueues the HIP work on
torch's current stream. Nothing here synchronises or falls back to another
implementation: unsupported inputs raise.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib as L
from . import profiling

_DT = {torch.float32: L.DTYPE_F32, torch.bfloat16: L.DTYPE_BF16}


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}; expected float32 or bfloat16") from None


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _require_cuda(*ts: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("zmoe ops need tensors on a HIP device")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("zmoe ops need all tensors on one device")
    return dev


def _rows(t: torch.Tensor) -> torch.Tensor:
    """2-D tensor with unit column stride (row stride may be anything)."""
    if t.dim() != 2:
        raise ValueError(f"expected a 2-D tensor, got shape {tuple(t.shape)}")
    return t if t.stride(1) == 1 else t.contiguous()


def _idx64(t: torch.Tensor) -> torch.Tensor:
    t = t.reshape(-1)
    if t.dtype != torch.int64:
        t = t.to(torch.int64)
    return t.contiguous()


# Feature widths the kernels cannot take directly. Their rows move as 16-byte chunks, so a
# width must be a multiple of 8 bf16 or 4 fp32 elements. The reference's kernels mask any
# width (scattermoe/kernels/ops.py:159-179, :404-435, :504-519); here the wrappers of the ops
# its module composition uses (group, scatter2scatter, group_bwd_w, combine, sum_k) copy an
# unaligned operand into a zero-padded one of the next aligned width, run the kernels, and
# return the unpadded columns. Zero columns add exact zeros to every sum, so the results are
# those of the unpadded arithmetic; the price is the copies (a slower path for such widths).
def _vec(dtype: torch.dtype) -> int:
    return 8 if dtype == torch.bfloat16 else 4


def _aligned(n: int, dtype: torch.dtype) -> bool:
    return n % _vec(dtype) == 0


def _up(n: int, dtype: torch.dtype) -> int:
    v = _vec(dtype)
    return -(-n // v) * v


def _pad_cols(t: Optional[torch.Tensor], n: int) -> Optional[torch.Tensor]:
    """``t`` [..., m] zero-padded to [..., n] (a new contiguous tensor), or ``t`` when m == n."""
    if t is None or t.shape[-1] == n:
        return t
    out = t.new_zeros(*t.shape[:-1], n)
    out[..., :t.shape[-1]] = t
    return out


def _unpad_into(full: torch.Tensor, n: int, out: Optional[torch.Tensor]) -> torch.Tensor:
    """The first n columns of ``full``, copied into ``out`` when given."""
    part = full[..., :n]
    if out is None:
        return part.contiguous()
    out.copy_(part)
    return out


# --------------------------------------------------------------------- routing
def route_topk(logits: torch.Tensor, expert_biases: torch.Tensor, k: int, round_probs_bf16: bool = False):
    """modeling/moe_gate.py:27-34 on given logits [T, E] -> (idx, weight, prob) [T, k]."""
    dev = _require_cuda(logits, expert_biases)
    logits = logits.contiguous()
    T, E = logits.shape
    bias = expert_biases.to(torch.float32).contiguous()
    if bias.numel() != E:
        raise ValueError("expert_biases must have E entries")
    idx = torch.empty((T, k), dtype=torch.int64, device=dev)
    w = torch.empty((T, k), dtype=torch.float32, device=dev)
    p = torch.empty((T, k), dtype=torch.float32, device=dev)
    with profiling.region("route_topk", dev):
        L.call("zmoe_route_topk", _ptr(logits), _dtype_code(logits), T, E, k, _ptr(bias), int(round_probs_bf16),
               _ptr(idx), _ptr(w), _ptr(p), _stream(dev))
    return idx, w, p


def route_topk_backward(d_weight: torch.Tensor, topk_prob: torch.Tensor, topk_idx: torch.Tensor, E: int,
                        dtype: torch.dtype, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """d_logits [T, E]; ``out`` may be a column slice of a wider row-major buffer."""
    dev = _require_cuda(d_weight, topk_prob, topk_idx, out)
    T, k = topk_idx.shape
    dw = d_weight.to(torch.float32).contiguous()
    if out is None:
        out = torch.empty((T, E), dtype=dtype, device=dev)
    elif out.shape != (T, E) or out.dtype != dtype or (T > 1 and out.stride(1) != 1):
        raise ValueError("route_topk_backward: out must be [T, E] of the logits dtype with unit column stride")
    L.call("zmoe_route_topk_backward", _ptr(dw), _ptr(topk_prob.contiguous()), _ptr(topk_idx.contiguous()), T, E,
           k, _ptr(out), out.stride(0), _DT[dtype], _stream(dev))
    return out


# --------------------------------------------------------------------- sort
def bincount(expert_idxs: torch.Tensor, num_experts: int) -> torch.Tensor:
    dev = _require_cuda(expert_idxs)
    flat = _idx64(expert_idxs)
    counts = torch.empty(num_experts, dtype=torch.int64, device=dev)
    L.call("zmoe_bincount", _ptr(flat), flat.numel(), num_experts, _ptr(counts), _stream(dev))
    return counts


def flatten_sort_count(expert_idxs: torch.Tensor, num_experts: int, return_workspace: bool = False):
    """scattermoe/parallel_experts.py:21-28 plus the inverse permutation.

    Returns (sorted_expert_idxs, sorted_scattered_idxs, expert_offsets, inverse)
    [+ workspace, whose first int32 is 1 when an index was outside [0, E)].
    """
    dev = _require_cuda(expert_idxs)
    flat = _idx64(expert_idxs)
    R = flat.numel()
    se = torch.empty(R, dtype=torch.int64, device=dev)
    ss = torch.empty(R, dtype=torch.int64, device=dev)
    off = torch.empty(num_experts, dtype=torch.int64, device=dev)
    inv = torch.empty(R, dtype=torch.int32, device=dev)
    nbytes = L.load().zmoe_sort_workspace_bytes(R, num_experts)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    with profiling.region("flatten_sort_count", dev):
        L.call("zmoe_flatten_sort_count", _ptr(flat), R, num_experts, _ptr(se), _ptr(ss), _ptr(off), _ptr(inv),
               _ptr(ws), nbytes, _stream(dev))
    if return_workspace:
        return se, ss, off, inv, ws
    return se, ss, off, inv


def sort_out_of_range(workspace: torch.Tensor) -> bool:
    """Host check (synchronises) of the sort's out-of-range flag."""
    return bool(workspace[:4].view(torch.int32)[0].item())


def offsets_from_sorted(sorted_expert_idxs: torch.Tensor, num_experts: int) -> torch.Tensor:
    dev = _require_cuda(sorted_expert_idxs)
    se = _idx64(sorted_expert_idxs)
    off = torch.empty(num_experts, dtype=torch.int64, device=dev)
    L.call("zmoe_offsets_from_sorted", _ptr(se), se.numel(), num_experts, _ptr(off), _stream(dev))
    return off


# --------------------------------------------------------------------- group
def group(A: torch.Tensor, sorted_idxs: torch.Tensor, coeff: Optional[torch.Tensor] = None, fan_out: int = 1,
          out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """scattermoe/kernels/ops.py:449-458: Y[n] = A[idx[n] // fan_out] * coeff[idx[n]]."""
    dev = _require_cuda(A, sorted_idxs, coeff, out)
    A = _rows(A)
    if not _aligned(A.shape[1], A.dtype):  # unaligned width: through a padded copy
        Kp = _up(A.shape[1], A.dtype)
        return _unpad_into(group(_pad_cols(A, Kp), sorted_idxs, coeff, fan_out), A.shape[1], out)
    idx = _idx64(sorted_idxs)
    N, K = idx.numel(), A.shape[1]
    if A.shape[0] * fan_out != N:
        raise ValueError("group: A.size(0) * fan_out must equal len(sorted_idxs)")
    Y = torch.empty((N, K), dtype=A.dtype, device=dev) if out is None else out
    if Y.shape != (N, K) or Y.dtype != A.dtype or Y.stride(1) != 1:
        raise ValueError("group: bad out tensor")
    c = None
    if coeff is not None:
        c = coeff.reshape(-1)
        if c.dtype not in _DT:
            c = c.float()
        c = c.contiguous()
    with profiling.region("group", dev):
        L.call("zmoe_group", _ptr(A), A.stride(0), K, _dtype_code(A), _ptr(idx), N, fan_out, _ptr(c),
               _DT[c.dtype] if c is not None else L.DTYPE_F32, _ptr(Y), Y.stride(0), _stream(dev))
    return Y


# --------------------------------------------------------------------- grouped GEMMs
def scatter2scatter(X: torch.Tensor, W: torch.Tensor, sorted_expert_idxs: torch.Tensor,
                    sorted_scattered_idxs: torch.Tensor, k: int, b: Optional[torch.Tensor] = None,
                    x_grouped: bool = False, y_grouped: bool = False, out: Optional[torch.Tensor] = None,
                    expert_offsets: Optional[torch.Tensor] = None, region: str = "scatter2scatter") -> torch.Tensor:
    """scattermoe/kernels/ops.py:192-209. W is the logical [E, K, N] operand (``region``: the
    profiling name of the launch)."""
    dev = _require_cuda(X, W, sorted_expert_idxs, sorted_scattered_idxs, b, out, expert_offsets)
    X = _rows(X)
    if W.dim() != 3:
        raise ValueError("scatter2scatter: W must be [E, K, N]")
    E, K, N = W.shape
    if W.dtype != X.dtype:
        raise ValueError("scatter2scatter: X and W dtypes differ")
    if not (_aligned(K, X.dtype) and _aligned(N, X.dtype)):  # unaligned widths: padded copies
        if X.shape[1] != K:
            raise ValueError("scatter2scatter: X.size(1) != W.size(1)")
        Kp, Np = _up(K, X.dtype), _up(N, X.dtype)
        # the padded weight in the nn.Linear layout [E, N, K] (the TN form), viewed [E, K, N]
        Wt = W.new_zeros(E, Np, Kp)
        Wt[:, :N, :K] = W.permute(0, 2, 1)
        Yp = scatter2scatter(_pad_cols(X, Kp), Wt.permute(0, 2, 1), sorted_expert_idxs, sorted_scattered_idxs, k,
                             b=_pad_cols(b, Np), x_grouped=x_grouped, y_grouped=y_grouped,
                             expert_offsets=expert_offsets, region=region)
        return _unpad_into(Yp, N, out)
    if W.stride(1) != 1 and W.stride(2) != 1:
        W = W.contiguous()
    se = _idx64(sorted_expert_idxs)
    ss = _idx64(sorted_scattered_idxs)
    R = se.numel()
    if ss.numel() != R or R != X.shape[0] * k:
        raise ValueError("scatter2scatter: sorted index lengths must equal X.size(0) * k")
    if X.shape[1] != K:
        raise ValueError("scatter2scatter: X.size(1) != W.size(1)")
    if out is None:
        out = torch.empty((R, N), dtype=X.dtype, device=dev)
    elif out.shape != (R, N) or out.dtype != X.dtype or out.stride(1) != 1:
        raise ValueError("scatter2scatter: bad out tensor")
    off = offsets_from_sorted(se, E) if expert_offsets is None else _idx64(expert_offsets)
    if b is not None:
        b = b.to(X.dtype).contiguous()
    M = X.shape[0]
    with profiling.region(region, dev):
        L.call("zmoe_scatter2scatter", _ptr(X), X.stride(0), _ptr(W), W.stride(0), W.stride(1), W.stride(2),
               _ptr(b), b.stride(0) if b is not None else 0, _ptr(se), _ptr(ss), _ptr(off), M, K, N, E, k,
               int(x_grouped), int(y_grouped), _dtype_code(X), _ptr(out), out.stride(0), _stream(dev))
    return out


def _wgrad_out_dtype(DY: torch.Tensor, out_dtype: Optional[torch.dtype], what: str) -> torch.dtype:
    """The weight grad's dtype: DY's (the reference's, ops.py:264-265), or float32 for bf16
    operands (the fp32 accumulators written unrounded: grads of fp32 master weights)."""
    od = DY.dtype if out_dtype is None else out_dtype
    if od != DY.dtype and not (DY.dtype == torch.bfloat16 and od == torch.float32):
        raise ValueError(f"{what}: out_dtype {od} with {DY.dtype} operands")
    return od


def group_bwd_w(DY: torch.Tensor, X: torch.Tensor, expert_offsets: torch.Tensor, E: int, has_bias: bool = False,
                x_gather: Optional[torch.Tensor] = None, x_div: int = 1, out: Optional[torch.Tensor] = None,
                out_bias: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None):
    """scattermoe/kernels/ops.py:263-271 -> (DWt [E, N, K] contiguous, Db [E, N] or None).

    ``x_gather`` makes row i of X read X[x_gather[i] // x_div] (no grouped copy).
    ``out`` / ``out_bias`` may supply the contiguous result buffers. ``out_dtype``
    float32 with bf16 operands: DWt unrounded from the fp32 accumulators (no bias grad).
    """
    dev = _require_cuda(DY, X, expert_offsets, x_gather)
    DY = _rows(DY)
    X = _rows(X)
    if DY.dtype != X.dtype:
        raise ValueError("group_bwd_w: DY and X dtypes differ")
    M, N = DY.shape
    K = X.shape[1]
    if not (_aligned(N, DY.dtype) and _aligned(K, DY.dtype)):  # unaligned widths: padded copies
        Np, Kp = _up(N, DY.dtype), _up(K, DY.dtype)
        DWp, Dbp = group_bwd_w(_pad_cols(DY, Np), _pad_cols(X, Kp), expert_offsets, E, has_bias=has_bias,
                               x_gather=x_gather, x_div=x_div, out_dtype=out_dtype)
        DWt = DWp[:, :N, :K].contiguous() if out is None else out.copy_(DWp[:, :N, :K])
        Db = None if Dbp is None else _unpad_into(Dbp, N, out_bias)
        return DWt, Db
    g = None
    if x_gather is not None:
        g = _idx64(x_gather)
        if g.numel() != M:
            raise ValueError("group_bwd_w: x_gather must have DY.size(0) entries")
    elif X.shape[0] != M:
        raise ValueError("group_bwd_w: X and DY row counts differ")
    od = _wgrad_out_dtype(DY, out_dtype, "group_bwd_w")
    if has_bias and od != DY.dtype:
        raise ValueError("group_bwd_w: the bias grad comes in DY's dtype only")
    DWt = torch.empty((E, N, K), dtype=od, device=dev) if out is None else out
    if DWt.shape != (E, N, K) or DWt.dtype != od or not DWt.is_contiguous():
        raise ValueError("group_bwd_w: bad out tensor")
    Db = None
    if has_bias:
        Db = torch.empty((E, N), dtype=DY.dtype, device=dev) if out_bias is None else out_bias
        if Db.shape != (E, N) or Db.dtype != DY.dtype or not Db.is_contiguous():
            raise ValueError("group_bwd_w: bad out_bias tensor")
    off = _idx64(expert_offsets)
    with profiling.region("group_bwd_w", dev):
        L.call("zmoe_group_bwd_w", _ptr(DY), DY.stride(0), _ptr(X), X.stride(0), _ptr(g), x_div, _ptr(off), M, N, K,
               E, _dtype_code(DY), _DT[od], _ptr(DWt), _ptr(Db), _stream(dev))
    return DWt, Db


def group_bwd_w_gather_dy(DY: torch.Tensor, dy_gather: torch.Tensor, dy_div: int, X: torch.Tensor,
                          expert_offsets: torch.Tensor, E: int, out: Optional[torch.Tensor] = None,
                          out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """group_bwd_w with the gather on DY (bf16): sorted row i of DY is DY[dy_gather[i] // dy_div],
    X [R, K] in sorted order. Returns DWt [E, N, K] (bf16, or float32 with ``out_dtype``)."""
    dev = _require_cuda(DY, dy_gather, X, expert_offsets)
    DY = _rows(DY)
    X = _rows(X)
    if DY.dtype != torch.bfloat16 or X.dtype != torch.bfloat16:
        raise ValueError("group_bwd_w_gather_dy: bf16 operands only")
    g = _idx64(dy_gather)
    M, K = X.shape
    N = DY.shape[1]
    if g.numel() != M or DY.shape[0] * dy_div < M:
        raise ValueError("group_bwd_w_gather_dy: dy_gather must have X.size(0) entries, into DY's rows")
    od = _wgrad_out_dtype(DY, out_dtype, "group_bwd_w_gather_dy")
    DWt = torch.empty((E, N, K), dtype=od, device=dev) if out is None else out
    if DWt.shape != (E, N, K) or DWt.dtype != od or not DWt.is_contiguous():
        raise ValueError("group_bwd_w_gather_dy: bad out tensor")
    off = _idx64(expert_offsets)
    with profiling.region("group_bwd_w", dev):
        L.call("zmoe_group_bwd_w_gather_dy", _ptr(DY), DY.stride(0), _ptr(g), int(dy_div), _ptr(X), X.stride(0),
               _ptr(off), M, N, K, E, _dtype_code(DY), _DT[od], _ptr(DWt), _stream(dev))
    return DWt


def dense_wgrad_splits(M: int, N: int, K: int, cus: int = 256) -> int:
    """Row splits for the dense weight-grad GEMM: the split count minimising
    (waves of tiles over the CUs) x (rows per split), plus the fp32 partials' extra
    HBM traffic, with at least 16 K-loop stages (1024 rows) per split."""
    tile = 256 if (M >= 256 and N >= 256 and K >= 256) else 128
    tiles = -(-N // tile) * -(-K // tile)
    stage_us, tile_fixed_us = 1.6, 11.0         # per 64-row stage and per tile, measured on MI355X
    bytes_per_us = 5.0e6                        # partial write + read at ~5 TB/s

    def cost(s: int) -> float:
        waves = -(-tiles * s // cus)
        stages = -(-M // (64 * s))
        extra = 0.0 if s == 1 else 2.0 * s * N * K * 4 / bytes_per_us
        return waves * (stages * stage_us + tile_fixed_us) + extra

    cands = [s for s in range(1, 65) if s == 1 or M // s >= 1024]
    return min(cands, key=cost)


def dense_wgrad(DY: torch.Tensor, X: torch.Tensor, splits: Optional[int] = None,
                out: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """DW [N, K] = DY[M, N]^T X[M, K]: the weight grad of an nn.Linear (F.linear backward);
    ``out_dtype`` float32 with bf16 operands writes the fp32 sum unrounded."""
    dev = _require_cuda(DY, X)
    DY = _rows(DY)
    X = _rows(X)
    if DY.dtype != X.dtype or DY.shape[0] != X.shape[0]:
        raise ValueError("dense_wgrad: DY and X must share dtype and row count")
    M, N = DY.shape
    K = X.shape[1]
    if splits is None:
        splits = dense_wgrad_splits(M, N, K)
    od = _wgrad_out_dtype(DY, out_dtype, "dense_wgrad")
    DW = torch.empty((N, K), dtype=od, device=dev) if out is None else out
    if DW.shape != (N, K) or DW.dtype != od or not DW.is_contiguous():
        raise ValueError("dense_wgrad: bad out tensor")
    nbytes = L.load().zmoe_dense_wgrad_workspace_bytes(N, K, splits if DY.dtype == torch.bfloat16 else 0)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    with profiling.region("dense_wgrad", dev):
        L.call("zmoe_dense_wgrad", _ptr(DY), DY.stride(0), _ptr(X), X.stride(0), M, N, K, _dtype_code(DY), _DT[od],
               splits, _ptr(DW), _ptr(ws), nbytes, _stream(dev))
    return DW


def glu_w1_forward(x: torch.Tensor, W1: torch.Tensor, sorted_expert_idxs, sorted_scattered_idxs, expert_offsets,
                   k: int, row_scale: Optional[torch.Tensor] = None):
    """W1 grouped GEMM with fused SwiGLU: returns H [R, 2f] and A [R, f] in sorted order.

    ``row_scale`` (f32 [R], sorted order; bf16 only): A[i] = row_scale[i] * silu(gate) * h."""
    dev = _require_cuda(x, W1, row_scale)
    x = _rows(x)
    W1 = W1.contiguous()
    E, two_f, d = W1.shape
    f = two_f // 2
    T = x.shape[0]
    R = T * k
    H = torch.empty((R, two_f), dtype=x.dtype, device=dev)
    A = torch.empty((R, f), dtype=x.dtype, device=dev)
    with profiling.region("glu_w1_forward", dev):
        if row_scale is None:
            L.call("zmoe_glu_w1_forward", _ptr(x), x.stride(0), _ptr(W1), _ptr(sorted_expert_idxs),
                   _ptr(sorted_scattered_idxs), _ptr(expert_offsets), T, d, f, E, k, _dtype_code(x), _ptr(H), _ptr(A),
                   _stream(dev))
        else:
            rs = row_scale.reshape(-1)
            if rs.dtype != torch.float32 or rs.numel() != R:
                raise ValueError("glu_w1_forward: row_scale must be float32 with T*k entries")
            L.call("zmoe_glu_w1_forward_scaled", _ptr(x), x.stride(0), _ptr(W1), _ptr(sorted_expert_idxs),
                   _ptr(sorted_scattered_idxs), _ptr(expert_offsets), T, d, f, E, k, _dtype_code(x),
                   _ptr(rs.contiguous()), _ptr(H), _ptr(A), _stream(dev))
    return H, A


def glu_w2_backward_dh(dYg: torch.Tensor, W2: torch.Tensor, H: torch.Tensor, sorted_expert_idxs, expert_offsets):
    """dA = dYg @ W2[e] fused with the SwiGLU backward: returns dH [R, 2f]."""
    dev = _require_cuda(dYg, W2, H)
    dYg = dYg.contiguous()
    W2 = W2.contiguous()
    E, d, f = W2.shape
    R = dYg.shape[0]
    dH = torch.empty((R, 2 * f), dtype=dYg.dtype, device=dev)
    with profiling.region("glu_w2_backward_dh", dev):
        L.call("zmoe_glu_w2_backward_dh", _ptr(dYg), _ptr(W2), _ptr(H), _ptr(sorted_expert_idxs),
               _ptr(expert_offsets), R, d, f, E, _dtype_code(dYg), _ptr(dH), _stream(dev))
    return dH


def glu_w2_backward_dh_gates(dout: torch.Tensor, W2: torch.Tensor, H: torch.Tensor, sorted_expert_idxs,
                             sorted_scattered_idxs, expert_offsets, k: int, gates: torch.Tensor):
    """glu_w2_backward_dh with the weighted combine's backward folded in (bf16): the A rows
    are dout's rows read in place (sorted row i reads token s_i // k), scaled by gates[s_i]
    after the GEMM, and the gates' grad <dout[t], Y[s]> is formed from the same products.
    Returns (dH [T*k, 2f], d_gates [T, k] f32)."""
    dev = _require_cuda(dout, W2, H, gates)
    dout = _rows(dout).contiguous()
    W2 = W2.contiguous()
    E, d, f = W2.shape
    T = dout.shape[0]
    R = T * k
    g = gates.reshape(-1).to(torch.float32).contiguous()
    if g.numel() != R or H.shape != (R, 2 * f):
        raise ValueError("glu_w2_backward_dh_gates: gates must hold T*k entries and H [T*k, 2f]")
    dH = torch.empty((R, 2 * f), dtype=dout.dtype, device=dev)
    d_gates = torch.empty((T, k), dtype=torch.float32, device=dev)
    nbytes = L.load().zmoe_glu_w2_backward_dh_gates_workspace_bytes(R, f)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    with profiling.region("glu_w2_backward_dh", dev):
        L.call("zmoe_glu_w2_backward_dh_gates", _ptr(dout), T, k, _ptr(W2), _ptr(H.contiguous()),
               _ptr(sorted_expert_idxs), _ptr(_idx64(sorted_scattered_idxs)), _ptr(expert_offsets), _ptr(g), d, f,
               E, _dtype_code(dout), _ptr(dH), _ptr(d_gates), _ptr(ws), nbytes, _stream(dev))
    return dH, d_gates


# --------------------------------------------------------------------- combine / reductions
def combine(Y: torch.Tensor, gates: Optional[torch.Tensor], k: int, addend: Optional[torch.Tensor] = None,
            out_rows: Optional[torch.Tensor] = None, out_total: Optional[int] = None) -> torch.Tensor:
    """out[t] = addend[t] + sum_j gates[t, j] * Y[t*k + j] (``gates = None``: all 1).

    With ``out_rows`` (int64 [T]) the result is the padded [out_total, d] tensor whose row
    out_rows[t] is token t's output and whose other rows are zero (moe_layer.py:55-56).
    """
    dev = _require_cuda(Y, gates, addend, out_rows)
    Y = Y.contiguous()
    d = Y.shape[-1]
    T = Y.numel() // (d * k)
    if not _aligned(d, Y.dtype):  # unaligned width: padded copies
        dp = _up(d, Y.dtype)
        a = None if addend is None else addend.reshape(T, d)
        full = combine(_pad_cols(Y.reshape(-1, d), dp), gates, k, _pad_cols(a, dp), out_rows, out_total)
        return full[:, :d].contiguous()
    g = None if gates is None else gates.reshape(T, k).to(torch.float32).contiguous()
    if addend is not None:
        addend = addend.reshape(T, d).to(Y.dtype).contiguous()
    with profiling.region("combine", dev):
        if out_rows is None:
            out = torch.empty((T, d), dtype=Y.dtype, device=dev)
            L.call("zmoe_combine", _ptr(Y), _ptr(g), _ptr(addend), T, k, d, _dtype_code(Y), _ptr(out), _stream(dev))
        else:
            rows = _idx64(out_rows)
            if rows.numel() != T:
                raise ValueError("combine: out_rows must hold one row per token")
            out = torch.zeros((out_total, d), dtype=Y.dtype, device=dev)
            L.call("zmoe_combine_rows", _ptr(Y), _ptr(g), _ptr(addend), T, k, d, _dtype_code(Y), _ptr(rows),
                   int(out_total), _ptr(out), _stream(dev))
    return out


def combine_backward(Y: Optional[torch.Tensor], grad_out: torch.Tensor, gates: torch.Tensor, inverse: torch.Tensor,
                     grad_rows: Optional[torch.Tensor] = None):
    """(d_gates [T, k] f32, grouped_grad_out [T*k, d] in sorted order).

    With ``grad_rows`` (int64 [T]) token t's gradient is row grad_rows[t] of the padded
    ``grad_out`` [rows, d], read in place. ``Y = None``: only the grouped rows (d_gates None).
    """
    dev = _require_cuda(Y, grad_out, gates, inverse, grad_rows)
    Y = None if Y is None else Y.contiguous()
    d = grad_out.shape[-1]
    dt = grad_out.dtype if Y is None else Y.dtype
    T, k = gates.shape
    g = gates.to(torch.float32).contiguous()
    d_gates = None if Y is None else torch.empty((T, k), dtype=torch.float32, device=dev)
    grouped = torch.empty((T * k, d), dtype=dt, device=dev)
    with profiling.region("combine_backward" if Y is not None else "combine_backward_scale", dev):
        if grad_rows is None:
            go = grad_out.reshape(T, d).to(dt).contiguous()
            L.call("zmoe_combine_backward", _ptr(Y), _ptr(go), _ptr(g), _ptr(inverse), T, k, d, _dtype_code(grouped),
                   _ptr(d_gates), _ptr(grouped), _stream(dev))
        else:
            go = grad_out.reshape(-1, d).to(dt).contiguous()
            rows = _idx64(grad_rows)
            if rows.numel() != T:
                raise ValueError("combine_backward: grad_rows must hold one row per token")
            L.call("zmoe_combine_backward_rows", _ptr(Y), _ptr(go), _ptr(rows), go.shape[0], _ptr(g), _ptr(inverse),
                   T, k, d, _dtype_code(grouped), _ptr(d_gates), _ptr(grouped), _stream(dev))
    return d_gates, grouped


def sum_k(Xe: torch.Tensor, k: int, add0: Optional[torch.Tensor] = None,
          add1: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """out[t] = sum_j Xe[t*k + j] (+ add0[t] + add1[t]), summed in fp32; ``out_dtype`` float32
    with bf16 rows writes the sum unrounded."""
    dev = _require_cuda(Xe, add0, add1)
    Xe = Xe.contiguous()
    d = Xe.shape[-1]
    T = Xe.numel() // (d * k)
    if not _aligned(d, Xe.dtype):  # unaligned width: padded copies
        dp = _up(d, Xe.dtype)
        pad = lambda a: None if a is None else _pad_cols(a.reshape(T, d), dp)  # noqa: E731
        return sum_k(_pad_cols(Xe.reshape(-1, d), dp), k, pad(add0), pad(add1), out_dtype)[:, :d].contiguous()
    od = Xe.dtype if out_dtype is None else out_dtype
    if od != Xe.dtype and not (Xe.dtype == torch.bfloat16 and od == torch.float32):
        raise ValueError(f"sum_k: out_dtype {od} with {Xe.dtype} rows")
    a0 = None if add0 is None else add0.reshape(T, d).to(Xe.dtype).contiguous()
    a1 = None if add1 is None else add1.reshape(T, d).to(Xe.dtype).contiguous()
    out = torch.empty((T, d), dtype=od, device=dev)
    with profiling.region("sum_k", dev):
        L.call("zmoe_sum_k", _ptr(Xe), T, k, d, _dtype_code(Xe), _ptr(a0), _ptr(a1), _DT[od], _ptr(out),
               _stream(dev))
    return out


def cast_bf16(src: torch.Tensor) -> torch.Tensor:
    """The bf16 copy of an fp32 tensor (round to nearest even), as ``src.to(torch.bfloat16)``,
    in one HIP pass; a bf16 tensor is returned as it is."""
    if src.dtype == torch.bfloat16:
        return src
    dev = _require_cuda(src)
    if src.dtype != torch.float32:
        raise ValueError(f"cast_bf16: float32 input expected, got {src.dtype}")
    src = src.contiguous()
    out = torch.empty(src.shape, dtype=torch.bfloat16, device=dev)
    with profiling.region("cast_bf16", dev):
        L.call("zmoe_cast_f32_bf16", _ptr(src), src.numel(), _ptr(out), _stream(dev))
    return out


def rowwise_sum_product(A: torch.Tensor, B: torch.Tensor, dtype: Optional[torch.dtype] = None,
                        out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """scattermoe/kernels/ops.py:9-18: out[t, j] = sum_h A[t, j, h] * B[t, h]."""
    dev = _require_cuda(A, B, out)
    if A.dim() != 3 or B.dim() != 2 or A.shape[0] != B.shape[0] or A.shape[2] != B.shape[1]:
        raise ValueError("rowwise_sum_product: expected A [T, F, H] and B [T, H]")
    A = A.contiguous()
    B = B.contiguous()
    T, F, H = A.shape
    if out is None:
        out = torch.empty((T, F), dtype=dtype or A.dtype, device=dev)
    with profiling.region("rowwise_sum_product", dev):
        L.call("zmoe_rowwise_sum_product", _ptr(A), _dtype_code(A), _ptr(B), _dtype_code(B), T, F, H, _ptr(out),
               _dtype_code(out), _stream(dev))
    return out


def swiglu(H: torch.Tensor) -> torch.Tensor:
    dev = _require_cuda(H)
    H = H.contiguous()
    R, two_f = H.shape
    A = torch.empty((R, two_f // 2), dtype=H.dtype, device=dev)
    L.call("zmoe_swiglu", _ptr(H), R, two_f // 2, _dtype_code(H), _ptr(A), _stream(dev))
    return A


def swiglu_backward_gates(dA: torch.Tensor, H: torch.Tensor, row_scale: torch.Tensor, slot_of_row: torch.Tensor):
    """SwiGLU backward of gate-scaled rows with the gates' grad, per sorted row r:
    dH[r] = swiglu_backward(row_scale[r] * dA[r], H[r]) and
    d_gates[slot_of_row[r]] = sum_c dA[r, c] * silu(H[r, f + c]) * H[r, c].
    Returns (dH [R, 2f], d_gates [R] f32 in slot order)."""
    dev = _require_cuda(dA, H, row_scale, slot_of_row)
    H = H.contiguous()
    dA = dA.to(H.dtype).contiguous()
    R, two_f = H.shape
    rs = row_scale.reshape(-1).to(torch.float32).contiguous()
    slots = _idx64(slot_of_row)
    if dA.shape != (R, two_f // 2) or rs.numel() != R or slots.numel() != R:
        raise ValueError("swiglu_backward_gates: dA [R, f], H [R, 2f], row_scale and slot_of_row [R]")
    dH = torch.empty_like(H)
    d_gates = torch.empty(R, dtype=torch.float32, device=dev)
    with profiling.region("swiglu_backward_gates", dev):
        L.call("zmoe_swiglu_backward_gates", _ptr(dA), _ptr(H), R, two_f // 2, _ptr(rs), _ptr(slots), _dtype_code(H),
               _ptr(dH), _ptr(d_gates), _stream(dev))
    return dH, d_gates


def swiglu_backward(dA: torch.Tensor, H: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """dH [R, 2f] from (dA [R, f], H [R, 2f]); ``out`` may be a column slice of a wider buffer."""
    dev = _require_cuda(dA, H, out)
    H = H.contiguous()
    dA = dA.to(H.dtype).contiguous()
    R, two_f = H.shape
    if out is None:
        out = torch.empty_like(H)
    elif out.shape != H.shape or out.dtype != H.dtype or (R > 1 and out.stride(1) != 1):
        raise ValueError("swiglu_backward: out must be [R, 2f] of H's dtype with unit column stride")
    L.call("zmoe_swiglu_backward", _ptr(dA), _ptr(H), R, two_f // 2, _dtype_code(H), _ptr(out), out.stride(0),
           _stream(dev))
    return out


def bias_update_(expert_biases: torch.Tensor, expert_offsets: torch.Tensor, update_rate: float) -> torch.Tensor:
    """main.py:161-175 in place on expert_biases (f32 [E]) from the sort's offsets."""
    dev = _require_cuda(expert_biases, expert_offsets)
    if expert_biases.dtype != torch.float32 or not expert_biases.is_contiguous():
        raise ValueError("bias_update_: expert_biases must be a contiguous float32 tensor")
    off = _idx64(expert_offsets)
    L.call("zmoe_bias_update", _ptr(off), off.numel(), float(update_rate), _ptr(expert_biases), _stream(dev))
    return expert_biases


def rmsnorm_rows(X: torch.Tensor, weight: torch.Tensor, eps: float, rows: Optional[torch.Tensor] = None):
    """modeling/zRMSNorm.py:10-17 on rows ``rows`` of X [N, d] (all rows when None):
    returns (Y [n, d] in X's dtype, rstd [n] f32)."""
    dev = _require_cuda(X, weight, rows)
    X = _rows(X)
    N, d = X.shape
    if weight.numel() != d:
        raise ValueError("rmsnorm_rows: weight must have d entries")
    w = weight.reshape(-1).contiguous()
    r = None if rows is None else _idx64(rows)
    n = N if r is None else r.numel()
    Y = torch.empty((n, d), dtype=X.dtype, device=dev)
    rstd = torch.empty(n, dtype=torch.float32, device=dev)
    with profiling.region("rmsnorm_rows", dev):
        L.call("zmoe_rmsnorm_rows", _ptr(X), X.stride(0), N, _ptr(r), n, d, _ptr(w), _dtype_code(w), float(eps),
               _dtype_code(X), _ptr(Y), _ptr(rstd), _stream(dev))
    return Y, rstd


def rmsnorm_rows_backward(dY: torch.Tensor, X: torch.Tensor, rows: Optional[torch.Tensor], rstd: torch.Tensor,
                          weight: torch.Tensor):
    """Backward of ``rmsnorm_rows``: (dX [N, d] with zeros outside ``rows``, dweight [d])."""
    dev = _require_cuda(dY, X, rows, rstd, weight)
    X = _rows(X)
    N, d = X.shape
    dY = dY.to(X.dtype).contiguous()
    r = None if rows is None else _idx64(rows)
    n = N if r is None else r.numel()
    if dY.shape != (n, d) or rstd.numel() != n:
        raise ValueError("rmsnorm_rows_backward: dY must be [n, d] and rstd [n]")
    w = weight.reshape(-1).contiguous()
    dX = torch.empty_like(X) if r is None else torch.zeros((N, d), dtype=X.dtype, device=dev)
    dw = torch.empty(d, dtype=w.dtype, device=dev)
    nbytes = L.load().zmoe_rmsnorm_rows_backward_workspace_bytes(n, d, _dtype_code(X))
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
    with profiling.region("rmsnorm_rows_backward", dev):
        L.call("zmoe_rmsnorm_rows_backward", _ptr(dY), _ptr(X), X.stride(0), N, _ptr(r), n, d,
               _ptr(rstd.contiguous()), _ptr(w), _dtype_code(w), _dtype_code(X), _ptr(dX), dX.stride(0), _ptr(dw),
               _ptr(ws), ws.numel(), _stream(dev))
    return dX, dw.view(weight.shape)


NS_COEFFS = (3.4445, -4.7750, 2.0315)  # optimizer/muon.py:16


def newton_schulz5(G: torch.Tensor, steps: int, coeffs=NS_COEFFS) -> torch.Tensor:
    """optimizer/muon.py:6-32 on G [..., m, n] (any float dtype): bf16 result of G's shape.

    Leading dims form the stack (one matrix each, as the reference's batched matmuls
    treat them); a tall stack (m > n) is transposed before and after, as muon.py:18-19
    and :29-30 do. m and n must be multiples of 8.
    """
    dev = _require_cuda(G)
    if G.ndim < 2:
        raise ValueError("newton_schulz5: G needs at least 2 dims")
    m, n = G.shape[-2], G.shape[-1]
    X = G.to(torch.bfloat16).reshape(-1, m, n)
    tall = m > n
    if tall:
        X = X.transpose(1, 2)
    if X.data_ptr() == G.data_ptr() or not X.is_contiguous():
        X = X.contiguous() if not X.is_contiguous() else X.clone()
    E, mm, nn = X.shape
    if E == 0:
        return X.reshape(G.shape)
    nbytes = int(L.load().zmoe_newton_schulz5_workspace_bytes(E, mm, nn))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    a, b, c = coeffs
    L.call("zmoe_newton_schulz5", _ptr(X), E, mm, nn, int(steps), float(a), float(b), float(c), _ptr(ws), nbytes,
           _stream(dev))
    if tall:
        X = X.transpose(1, 2)
    return X.reshape(G.shape)
