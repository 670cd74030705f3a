"""CPU restatement (numpy, float64 by default) of the reference MoE-layer hot path.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py``; never by the product package.

Every function cites the reference file:line it restates (paths relative to the
reference repository root). Where the reference leaves an order unspecified this
module fixes the contract the HIP path must meet bit-exactly:

* top-k slots are ordered by (biased score descending, expert index ascending);
  NaN ranks above every number (as ``torch.topk`` does), NaNs tie by index;
* the expert sort is stable by flat slot id ``t*k + j``.

Pinning (what checks each function, all in ``tests/test_oracle.py``):

* ``sigmoid_f32``          closed form at 0, symmetry p(x)+p(-x)=1, saturation.
* ``route_topk``           brute force (pure-Python full sort) on tiny E; equal
                           scores select 0..k-1; a huge bias forces selection while
                           the weight keeps the unbiased p; b=0 gives top-k of p;
                           weights sum to 1; NaN policy.
* ``flatten_sort_count``   brute force ``sorted(range(R), key=(e, i))``;
                           permutation; counts = histogram; inclusive offsets.
* ``group``                direct indexing identity on random data.
* ``scatter2scatter``      per-row dense loop (textbook matmul per row).
* ``group_bwd_w``          per-row outer-product accumulation; empty expert = 0.
* ``rowwise_sum_product``  einsum.
* ``parallel_linear_forward`` / ``parallel_linear_backward``: torch float64
                           autograd of a slot-by-slot formulation in every caller
                           mode (gathered or grouped input, slot or grouped
                           output, gates, bias), and float64 central differences
                           of every input element on tiny shapes; the bf16
                           storage mode against torch's own bf16 autograd of the
                           reference's composition (bit-equal but for rare
                           accumulation-order flips, far closer than exact mode).
* ``route_topk_backward``  torch autograd through sigmoid, gather and L1 normalise.
* ``glu_mlp_*`` / ``MoELayerOracle``: torch autograd of an independent per-token
                           dense formulation of the layer; float64 central
                           differences of the GLU experts on tiny shapes.
* ``bias_update``          closed form on a hand-built histogram.
* ``zc_rmsnorm_rows``      closed forms: a constant row c gives sign(c)(1 + w)/sqrt(1 +
                           eps/c^2); scale invariance at eps = 0; w = 0 gives rows of
                           unit RMS; the gather equals normalising every row then
                           indexing; backward against torch autograd of the reference
                           expression and central finite differences.
* ``newton_schulz5``       exact mode: the SVD closed form U phi^steps(S/||G||) V^T
                           with phi(s) = a s + b s^3 + c s^5; transpose symmetry;
                           bf16 mode: rounding points checked against torch's bf16
                           tensor ops on tiny matrices.
"""

from __future__ import annotations

import numpy as np

_PREC = {"float": np.float64}


def set_precision(dtype) -> None:
    """Float type of the GEMM/elementwise restatements (float64 for parity
    checks, float32 for the timed CPU baseline). Routing math stays float64."""
    _PREC["float"] = np.dtype(dtype).type


def _f():
    return _PREC["float"]


__all__ = [
    "set_precision",
    "bf16_round",
    "SIGMOID_ZERO_BELOW",
    "SIGMOID_SERIES_BELOW",
    "sigmoid_f32",
    "route_topk",
    "route_topk_backward",
    "expert_counts",
    "flatten_sort_count",
    "inverse_permutation",
    "group",
    "scatter2scatter",
    "group_bwd_w",
    "rowwise_sum_product",
    "parallel_linear_forward",
    "parallel_linear_backward",
    "glu_mlp_forward",
    "glu_mlp_backward",
    "swiglu",
    "swiglu_backward",
    "storage_rounder",
    "summand_rss",
    "shared_expert_forward",
    "shared_expert_backward",
    "MoELayerOracle",
    "zc_rmsnorm_rows",
    "zc_rmsnorm_rows_backward",
    "bias_update",
    "moe_load_metrics",
    "NS_COEFFS",
    "newton_schulz5",
]


# --------------------------------------------------------------------------- #
# numeric helpers
# --------------------------------------------------------------------------- #
def bf16_round(x):
    """Round float32 values to the nearest bfloat16 (ties to even); returns float32.

    This is the rounding ``tensor.to(torch.bfloat16)`` performs. NaN stays NaN.
    """
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    r = ((u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)) << np.uint64(16)
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out).astype(np.float32)


SIGMOID_ZERO_BELOW = -88.72283935546875
SIGMOID_SERIES_BELOW = 2.0 ** -12


def sigmoid_f32(logits):
    """sigmoid of float32 logits, correctly rounded to float32; 0 for logits at or below
    ``SIGMOID_ZERO_BELOW``.

    Restates ``torch.sigmoid(gate_output)`` (modeling/moe_gate.py:27). torch forms
    1 / (1 + exp(-z)) in float32, whose exp(-z) overflows to inf from z <= -88.7228...
    on, so its probability there is 0 (not the subnormal float64 value); this function
    follows it. Elsewhere torch's float32 evaluation can differ from the correctly
    rounded value by an ulp; the contract is the correctly rounded one:

    * |z| < 2^-12: p = 0.5 + z/4 - z^3/48 + ...; 0.5 + z/4 is exact in float64 and the
      cubic term cannot move it across an fp32 rounding midpoint unless it lies exactly on
      one (its distance from a midpoint is a multiple of z's last bit / 4, which exceeds
      |z|^3/48 here), so p is 0.5 + z/4 rounded to nearest, an exact tie going to the
      side the cubic term puts the true value on (down for z > 0, up for z < 0). Many
      small bf16 logits land on such ties, where a float64 evaluation's rounding depends
      on the last bit of its exp.
    * otherwise 1 / (1 + exp(-z)) in float64, rounded once.

    The HIP kernel evaluates the same two forms, so p agrees bit-for-bit.
    """
    with np.errstate(over="ignore", invalid="ignore"):  # NaN and infinite logits are part of the contract
        z = np.asarray(logits, dtype=np.float32).astype(np.float64)
        p = 1.0 / (1.0 + np.exp(-z))
    p = np.where(z <= SIGMOID_ZERO_BELOW, 0.0, p).astype(np.float32)
    small = np.abs(z) < SIGMOID_SERIES_BELOW
    if small.any():
        zs = z[small]
        s = 0.5 + 0.25 * zs                                   # exact
        f = s.astype(np.float32)
        fd = f.astype(np.float64)
        other = np.where(fd < s, np.nextafter(f, np.float32(1)), np.nextafter(f, np.float32(0)))
        tie = (fd != s) & (np.abs(s - fd) == np.abs(other.astype(np.float64) - s))
        side = np.where(zs > 0, np.minimum(f, other), np.maximum(f, other))
        p[small] = np.where(tie, side, f)
    return p


# --------------------------------------------------------------------------- #
# a1: routing (modeling/moe_gate.py:19-36)
# --------------------------------------------------------------------------- #
def route_topk(logits, expert_biases, k, round_probs_bf16=False):
    """Aux-loss-free sigmoid routing after the gate projection.

    Restates modeling/moe_gate.py:26-34:
      p = sigmoid(logits)                 (:27)
      s = p + expert_biases               (:29, bias after the sigmoid, fp32)
      idx = topk(s, k)                    (:30, selection only)
      w = gather(p, idx)                  (:33, unbiased p)
      w = w / max(sum(|w|), 1e-12)        (:34, F.normalize(p=1))

    ``round_probs_bf16`` reproduces the reference under bf16 autocast, where the
    sigmoid output is a bf16 tensor before the fp32 bias add.

    Returns (idx int64 [T,k], weights float32 [T,k], p_selected float32 [T,k]).
    """
    logits = np.asarray(logits, dtype=np.float32)
    T, E = logits.shape
    if not (0 < k <= E):
        raise ValueError("k must be in [1, E]")
    p = sigmoid_f32(logits)
    if round_probs_bf16:
        p = bf16_round(p)
    s = (p + np.asarray(expert_biases, dtype=np.float32)[None, :]).astype(np.float32)
    nan = np.isnan(s)
    neg = np.where(nan, np.float32(0.0), -s)
    e_idx = np.broadcast_to(np.arange(E), (T, E))
    # np.lexsort: last key is primary. NaN first, then score desc, then index asc.
    order = np.lexsort((e_idx, neg, ~nan), axis=-1)
    idx = order[:, :k].astype(np.int64)
    p_sel = np.take_along_axis(p, idx, axis=1).astype(np.float32)
    denom = np.maximum(np.abs(p_sel.astype(np.float64)).sum(axis=1, keepdims=True), 1e-12)
    w = (p_sel.astype(np.float64) / denom).astype(np.float32)
    return idx, w, p_sel


def route_topk_backward(d_weight, p_selected, idx, E):
    """Gradient of the routing weights w.r.t. the gate logits (float64).

    Autograd of modeling/moe_gate.py:27,33-34: through F.normalize(p=1)
    (w_j = p_j / S, S = max(sum p, eps)), the gather, and the sigmoid
    (dp/dz = p (1 - p)). Returns a dense [T, E] gradient (zero off the top-k).
    """
    dw = np.asarray(d_weight, dtype=np.float64)
    p = np.asarray(p_selected, dtype=np.float64)
    S_raw = np.abs(p).sum(axis=1, keepdims=True)
    S = np.maximum(S_raw, 1e-12)
    w = p / S
    # d(p_j/S)/dp_i = delta_ij / S - p_j sign(p_i) / S^2  (only while S > eps)
    inner = (dw * w).sum(axis=1, keepdims=True)
    dp = np.where(S_raw > 1e-12, (dw - inner * np.sign(p)) / S, dw / S)
    dz_sel = dp * p * (1.0 - p)
    T = dw.shape[0]
    dz = np.zeros((T, E), dtype=np.float64)
    np.put_along_axis(dz, np.asarray(idx, dtype=np.int64), dz_sel, axis=1)
    return dz


# --------------------------------------------------------------------------- #
# a3/a4: counts and the expert sort (scattermoe/parallel_experts.py:6-28)
# --------------------------------------------------------------------------- #
def expert_counts(expert_idxs, E):
    """``compileable_bincount`` (scattermoe/parallel_experts.py:6-15): int64 [E]."""
    flat = np.asarray(expert_idxs, dtype=np.int64).reshape(-1)
    if flat.size and (flat.min() < 0 or flat.max() >= E):
        raise ValueError("expert index out of range")
    return np.bincount(flat, minlength=E).astype(np.int64)


def flatten_sort_count(expert_idxs, E):
    """scattermoe/parallel_experts.py:21-28.

    sorted_expert_idxs, sorted_scattered_idxs = sort(expert_idxs.flatten())  (:25)
    expert_offsets = cumsum(bincount)  inclusive ends, no leading zero      (:26-27)
    The sort is stable: equal experts keep flat-slot order.
    """
    flat = np.asarray(expert_idxs, dtype=np.int64).reshape(-1)
    counts = expert_counts(flat, E)
    order = np.argsort(flat, kind="stable").astype(np.int64)
    return flat[order], order, np.cumsum(counts).astype(np.int64)


def inverse_permutation(sorted_scattered_idxs):
    """inv[slot] = position of that slot in expert-sorted order."""
    s = np.asarray(sorted_scattered_idxs, dtype=np.int64)
    inv = np.empty_like(s)
    inv[s] = np.arange(s.size, dtype=np.int64)
    return inv


# --------------------------------------------------------------------------- #
# a5: group (scattermoe/kernels/ops.py:449-529)
# --------------------------------------------------------------------------- #
def group(A, sorted_idxs, coeff=None, fan_out=1):
    """Y[n] = A[idx[n] // fan_out] * coeff[idx[n]]  (ops.py:504-519)."""
    A = np.asarray(A, dtype=_f())
    idx = np.asarray(sorted_idxs, dtype=np.int64)
    Y = A[idx // fan_out]
    if coeff is not None:
        c = np.asarray(coeff, dtype=_f()).reshape(-1)
        Y = Y * c[idx][:, None]
    return Y


# --------------------------------------------------------------------------- #
# a6: scatter2scatter (scattermoe/kernels/ops.py:122-255)
# --------------------------------------------------------------------------- #
def _expert_ranges(sorted_expert_idxs, E):
    se = np.asarray(sorted_expert_idxs, dtype=np.int64)
    ends = np.searchsorted(se, np.arange(E), side="right")
    starts = np.concatenate([[0], ends[:-1]])
    return starts, ends


def scatter2scatter(X, W, sorted_expert_idxs, sorted_scattered_idxs, k, b=None,
                    x_grouped=False, y_grouped=False):
    """Grouped linear over expert-sorted rows (ops.py:144-190).

    Sorted row i uses expert e = sorted_expert_idxs[i]; its input row is X[i] if
    ``x_grouped`` else X[sorted_scattered_idxs[i] // k] (:165-168); its output row
    is Y[i] if ``y_grouped`` else Y[sorted_scattered_idxs[i]] (:185-189).
    ``W`` is the logical [E, K, N] operand (the reference passes
    ``weight.permute(0, 2, 1)``); optional bias ``b`` [E, N] (:181-183).
    """
    X = np.asarray(X, dtype=_f())
    W = np.asarray(W, dtype=_f())
    se = np.asarray(sorted_expert_idxs, dtype=np.int64)
    ss = np.asarray(sorted_scattered_idxs, dtype=np.int64)
    R = se.size
    E, _, N = W.shape
    rows_in = np.arange(R) if x_grouped else ss // k
    rows_out = np.arange(R) if y_grouped else ss
    Y = np.zeros((R, N), dtype=_f())
    starts, ends = _expert_ranges(se, E)
    for e in range(E):
        s, t = starts[e], ends[e]
        if t <= s:
            continue
        blk = X[rows_in[s:t]] @ W[e]
        if b is not None:
            blk = blk + np.asarray(b, dtype=_f())[e][None, :]
        Y[rows_out[s:t]] = blk
    return Y


# --------------------------------------------------------------------------- #
# a7: group_bwd_W (scattermoe/kernels/ops.py:263-438)
# --------------------------------------------------------------------------- #
def group_bwd_w(DY, X, expert_offsets, E, has_bias=False):
    """DW[e] = X[s_e:t_e]^T @ DY[s_e:t_e] over each expert's sorted row range.

    ops.py:344-348 (range from inclusive offsets), :412-435 (accumulate), :264
    (pre-zeroed, so an empty expert gets exactly 0). Returns DW [E, K, N] (the
    logical view the reference returns) and Db [E, N] or None (:430-438).
    """
    DY = np.asarray(DY, dtype=_f())
    X = np.asarray(X, dtype=_f())
    off = np.asarray(expert_offsets, dtype=np.int64)
    K, N = X.shape[1], DY.shape[1]
    DW = np.zeros((E, K, N), dtype=_f())
    Db = np.zeros((E, N), dtype=_f()) if has_bias else None
    start = 0
    for e in range(E):
        end = int(off[e])
        if end > start:
            DW[e] = X[start:end].T @ DY[start:end]
            if has_bias:
                Db[e] = DY[start:end].sum(axis=0)
        start = end
    return DW, Db


# --------------------------------------------------------------------------- #
# a8: rowwise_sum_product (scattermoe/kernels/ops.py:9-80)
# --------------------------------------------------------------------------- #
def rowwise_sum_product(A, B):
    """out[t, j] = sum_h A[t, j, h] * B[t, h]  (ops.py:79)."""
    return np.einsum("tjh,th->tj", np.asarray(A, dtype=_f()), np.asarray(B, dtype=_f()))


# --------------------------------------------------------------------------- #
# a9/a10: ParallelLinear (scattermoe/parallel_experts.py:32-135)
# --------------------------------------------------------------------------- #
def parallel_linear_forward(x, W, k, sorted_expert_idxs, sorted_scattered_idxs,
                            expert_offsets, b=None, gates=None,
                            grouped_in=False, grouped_out=False, store=None):
    """ParallelLinear.forward (parallel_experts.py:34-68). W is logical [E, K, N].

    Returns (output, output_expanded) where output_expanded is the [T, k, N]
    per-slot output saved for backward when ``gates`` is given (:50-55).
    ``store`` rounds where a bf16 path stores (see ``storage_rounder``): the expert
    outputs (:41-47) and the gate-weighted combine (:50-52).
    """
    r = storage_rounder(store)
    out = r(scatter2scatter(x, W, sorted_expert_idxs, sorted_scattered_idxs, k, b=b,
                            x_grouped=grouped_in, y_grouped=grouped_out))
    if gates is None:
        return out, None
    g = np.asarray(gates, dtype=_f())
    T, kk = g.shape
    expanded = out.reshape(T, kk, out.shape[-1])
    return r(np.einsum("tj,tjn->tn", g, expanded)), expanded


def parallel_linear_backward(grad_out, x, W, k, sorted_expert_idxs, sorted_scattered_idxs,
                             expert_offsets, b=None, gates=None, output_expanded=None,
                             grouped_in=False, grouped_out=False, store=None):
    """ParallelLinear.backward (parallel_experts.py:70-135).

    Returns (d_input, d_weights [E, K, N], d_biases or None, d_gates or None).
    ``store`` rounds where a bf16 path stores: d_gates (in the gates' dtype, :82), the
    gate-scaled grouped grad rows (:95-97), the weight and bias grads (:105-110), the
    per-slot input grads (:112-120) and their k-sum (:125).
    """
    r = storage_rounder(store)
    grad_out = np.asarray(grad_out, dtype=_f())
    E = np.asarray(W).shape[0]
    if gates is not None:
        d_gates = r(rowwise_sum_product(output_expanded, grad_out))          # :82
        gates_flat = np.asarray(gates, dtype=_f()).reshape(-1)
        gate_fan = np.asarray(gates).shape[1]
    else:
        d_gates, gates_flat, gate_fan = None, None, 1
    if grouped_out:
        grouped_grad_out = grad_out                                            # :93
    else:
        grouped_grad_out = r(group(grad_out, sorted_scattered_idxs,            # :95-97
                                   coeff=gates_flat, fan_out=gate_fan))
    grouped_x = x if grouped_in else group(x, sorted_scattered_idxs, fan_out=k)  # :98-103
    d_w, d_b = group_bwd_w(grouped_grad_out, grouped_x, expert_offsets, E,       # :105-110
                           has_bias=b is not None)
    d_w = r(d_w)
    d_b = None if d_b is None else r(d_b)
    Wt = np.transpose(np.asarray(W, dtype=_f()), (0, 2, 1))
    d_exp = r(scatter2scatter(grouped_grad_out, Wt, sorted_expert_idxs,          # :112-120
                              sorted_scattered_idxs, 1, x_grouped=True, y_grouped=grouped_in))
    if k == 1:
        d_input = d_exp
    else:
        d_input = r(d_exp.reshape(np.asarray(x).shape[0], k, -1).sum(axis=1))  # :125
    return d_input, d_w, d_b, d_gates


# --------------------------------------------------------------------------- #
# a12: GLUMLP (scattermoe/mlp.py:51-95)
# --------------------------------------------------------------------------- #
def _silu(z):
    return z / (1.0 + np.exp(-z))


def swiglu(H):
    """chunk(2) then silu(second half) * first half (mlp.py:81-87)."""
    f = H.shape[-1] // 2
    h, g = H[..., :f], H[..., f:]
    return _silu(g) * h


def swiglu_backward(dA, H):
    """Gradient of swiglu w.r.t. H = [h | g]."""
    f = H.shape[-1] // 2
    h, g = H[..., :f], H[..., f:]
    s = 1.0 / (1.0 + np.exp(-g))
    dh = dA * g * s
    dg = dA * h * s * (1.0 + g * (1.0 - s))
    return np.concatenate([dh, dg], axis=-1)


def storage_rounder(store):
    """The rounding applied where the path stores a tensor.

    ``None``: exact (no rounding; the float64 restatement). ``"bf16"``: a value is
    formed in this module's float type, rounded to float32 (the fp32 accumulator or
    elementwise result) and then to bfloat16 (the stored activation), as every bf16
    tensor the path writes is produced: GEMM outputs (scattermoe/kernels/ops.py:202,
    :434 store in the operand dtype), elementwise results and the combine/k-sum rows.
    """
    if store is None:
        return lambda a: a
    if store == "bf16":
        return lambda a: bf16_round(np.asarray(a, dtype=np.float32)).astype(_f())
    raise ValueError(f"unknown store {store!r}")


def glu_mlp_forward(x, expert_p, expert_idxs, W1, W2, store=None, gate_scale_on="Y", residual=None):
    """GLUMLP.forward (mlp.py:74-95).

    x [T, d]; expert_p, expert_idxs [T, k]; W1 [E, 2f, d] and W2 [E, d, f] in
    ``nn.Parameter`` storage (the reference permutes them to [E, in, out]).

    ``store`` rounds at the stored tensors (see ``storage_rounder``): H (:80-85), the
    activation A (:86), the per-slot W2 outputs Y (:87-93) and the combined output.
    ``gate_scale_on`` says where the routing weights multiply: ``"Y"`` on the W2 outputs
    as the reference does (parallel_experts.py:50-52), ``"A"`` on the activations before
    the W2 product (w (A W2) = (w A) W2, equal in exact arithmetic; the rounding points
    differ). ``residual`` [T, d] (the shared expert's output, moe_layer.py:53) is added
    before the output is rounded, as one pass forms both sums.
    Returns (y [T, d], cache) with the tensors the backward needs.
    """
    r = storage_rounder(store)
    x = np.asarray(x, dtype=_f())
    T, k = np.asarray(expert_idxs).shape
    E = np.asarray(W1).shape[0]
    se, ss, off = flatten_sort_count(expert_idxs, E)                          # :76-77
    W1l = np.transpose(np.asarray(W1, dtype=_f()), (0, 2, 1))
    W2l = np.transpose(np.asarray(W2, dtype=_f()), (0, 2, 1))
    gates = np.asarray(expert_p, dtype=_f())
    w_sorted = gates.reshape(-1)[ss]
    H = r(scatter2scatter(x, W1l, se, ss, k, y_grouped=True))                 # :80-85
    if gate_scale_on == "Y":
        A = r(swiglu(H))                                                      # :86
    elif gate_scale_on == "A":
        A = r(w_sorted[:, None] * swiglu(H))
    else:
        raise ValueError("gate_scale_on must be 'Y' or 'A'")
    Y = r(scatter2scatter(A, W2l, se, ss, 1, x_grouped=True, y_grouped=False))  # :87-93, slot order
    Y3 = Y.reshape(T, k, -1)
    y = np.einsum("tj,tjn->tn", gates, Y3) if gate_scale_on == "Y" else Y3.sum(axis=1)  # parallel_experts.py:50-52
    if residual is not None:
        y = np.asarray(residual, dtype=_f()) + y
    y = r(y)
    cache = dict(x=x, se=se, ss=ss, off=off, H=H, A=A, y_exp=Y3, gates=gates, w_sorted=w_sorted, k=k,
                 W1l=W1l, W2l=W2l, store=store, gate_scale_on=gate_scale_on)
    return y, cache


def summand_rss(sum_of_products, a, b):
    """Root-sum-square of the summands of every element of a product-sum: the same
    reduction ``sum_of_products(a, b)`` applied to a**2 and b**2, square-rooted.

    It bounds the largest summand (max |a_r b_r| <= rss), so one bf16 ulp of any single
    stored summand moves the sum by at most 2**-8 * rss: the scale of the rounding flips
    that accumulation order alone causes in bf16 reductions (see tests/helpers.py)."""
    return np.sqrt(sum_of_products(np.asarray(a, dtype=_f()) ** 2, np.asarray(b, dtype=_f()) ** 2))


def glu_mlp_backward(dy, cache, rss=False, round_wgrads=True):
    """Autograd of GLUMLP (mlp.py:74-95 through parallel_experts.py:70-135), at the
    rounding points of ``glu_mlp_forward``'s ``store``.

    Returns (dx [T, d], dW1 [E, 2f, d], dW2 [E, d, f], d_gates [T, k]). dx (the k-sum of
    the per-slot input grads, parallel_experts.py:125) and d_gates (fp32 in the path) are
    not rounded: the caller adds its other input-grad terms before the one rounding.
    With ``rss=True`` a fifth item maps "W1", "W2", "d_gates" to the root-sum-square of
    each element's summands (``summand_rss``). ``round_wgrads=False`` leaves dW1 and dW2
    unrounded (fp32 grads of fp32 master weights, summed over the stored summands).
    """
    c = cache
    r = storage_rounder(c["store"])
    rw = r if round_wgrads else storage_rounder(None)
    dy = np.asarray(dy, dtype=_f())
    se, ss, off, k = c["se"], c["ss"], c["off"], c["k"]
    E = c["W1l"].shape[0]
    T = dy.shape[0]
    W2t = np.transpose(c["W2l"], (0, 2, 1))
    if c["gate_scale_on"] == "Y":
        d_gates = rowwise_sum_product(c["y_exp"], dy)                         # :82
        G = r(group(dy, ss, coeff=c["gates"].reshape(-1), fan_out=k))          # :95-97
        dA = r(scatter2scatter(G, W2t, se, ss, 1, x_grouped=True, y_grouped=True))  # :112-120
        dH = r(swiglu_backward(dA, c["H"]))
    else:
        # dout[t]'s rows unscaled; the gates' grad <dout[t], Y> = <dout[t] W2_e, A / w>
        G = group(dy, ss, fan_out=k)
        dA = r(scatter2scatter(G, W2t, se, ss, 1, x_grouped=True, y_grouped=True))
        d_sorted = (dA * swiglu(c["H"])).sum(axis=1)
        d_gates = np.empty(T * k, dtype=_f())
        d_gates[ss] = d_sorted
        d_gates = d_gates.reshape(T, k)
        dH = r(swiglu_backward(c["w_sorted"][:, None] * dA, c["H"]))
    dW2l, _ = group_bwd_w(G, c["A"], off, E)                                    # :105-110
    grouped_x = group(c["x"], ss, fan_out=k)                                   # :98-103
    dW1l, _ = group_bwd_w(dH, grouped_x, off, E)
    W1t = np.transpose(c["W1l"], (0, 2, 1))
    dXe = r(scatter2scatter(dH, W1t, se, ss, 1, x_grouped=True, y_grouped=False))
    dx = dXe.reshape(T, k, -1).sum(axis=1)                                     # :125
    out = (dx, rw(np.transpose(dW1l, (0, 2, 1))), rw(np.transpose(dW2l, (0, 2, 1))), d_gates)
    if not rss:
        return out
    wsum = lambda a, b: group_bwd_w(a, b, off, E)[0]  # noqa: E731
    if c["gate_scale_on"] == "Y":
        g_rss = summand_rss(rowwise_sum_product, c["y_exp"], dy)
    else:
        g_rss = np.empty(T * k, dtype=_f())
        g_rss[ss] = np.sqrt(((dA * swiglu(c["H"])) ** 2).sum(axis=1))
        g_rss = g_rss.reshape(T, k)
    return out + ({"W1": np.transpose(summand_rss(wsum, dH, grouped_x), (0, 2, 1)),
                   "W2": np.transpose(summand_rss(wsum, G, c["A"]), (0, 2, 1)), "d_gates": g_rss},)


# --------------------------------------------------------------------------- #
# a14: shared expert (modeling/expert_layer.py:23-24)
# --------------------------------------------------------------------------- #
def shared_expert_forward(x, Wg, Wu, Wd, store=None):
    """down(silu(gate(x)) * up(x)) with nn.Linear weights [out, in]; ``store`` rounds
    the two projections, the activation and the output."""
    r = storage_rounder(store)
    x = np.asarray(x, dtype=_f())
    g = r(x @ np.asarray(Wg, dtype=_f()).T)
    u = r(x @ np.asarray(Wu, dtype=_f()).T)
    a = r(_silu(g) * u)
    return r(a @ np.asarray(Wd, dtype=_f()).T), (x, g, u, a)


def shared_expert_backward(dy, cache, Wg, Wu, Wd, store=None, rss=False, round_wgrads=True):
    """Returns (dx, dWg, dWu, dWd); dx is not rounded (the caller adds its other terms).
    With ``rss=True`` a fifth item maps "gate", "up", "down" to the weight grads'
    summand root-sum-squares. ``round_wgrads=False`` leaves the weight grads unrounded."""
    r = storage_rounder(store)
    rw = r if round_wgrads else storage_rounder(None)
    x, g, u, a = cache
    dy = np.asarray(dy, dtype=_f())
    Wg = np.asarray(Wg, dtype=_f())
    Wu = np.asarray(Wu, dtype=_f())
    Wd = np.asarray(Wd, dtype=_f())
    dWd = rw(dy.T @ a)
    da = r(dy @ Wd)
    s = 1.0 / (1.0 + np.exp(-g))
    du = r(da * g * s)
    dg = r(da * u * s * (1.0 + g * (1.0 - s)))
    dx = dg @ Wg + du @ Wu
    out = (dx, rw(dg.T @ x), rw(du.T @ x), dWd)
    if not rss:
        return out
    tsum = lambda a, b: a.T @ b  # noqa: E731
    return out + ({"gate": summand_rss(tsum, dg, x), "up": summand_rss(tsum, du, x),
                   "down": summand_rss(tsum, dy, a)},)


# --------------------------------------------------------------------------- #
# a13: MoELayer (modeling/moe_layer.py:38-59)
# --------------------------------------------------------------------------- #
class MoELayerOracle:
    """Forward and backward of ``MoELayer`` on the valid tokens.

    Parameters follow the reference state dict: gate ``weight [E, d]`` and
    ``expert_biases [E]`` (moe_gate.py:12-13); ``W1 [E, 2f, d]``, ``W2 [E, d, f]``
    (mlp.py:58-59); shared ``gate/up/down_proj`` (expert_layer.py:12-14), or
    ``None`` for no shared expert.

    ``logits`` may be supplied to forward() so the routing starts from exactly the
    gate projection the device computed (the projection itself is checked with a
    tolerance; routing from given logits is checked bit-exactly).

    ``store`` / ``gate_scale_on``: as in ``glu_mlp_forward``. With ``store="bf16"`` the
    gate's logits grad is rounded (it is stored in the logits dtype), and so is the
    hidden states' grad: with ``gate_scale_on="A"`` (the layer as one function) the gate
    and shared-expert input grads are formed by one product and rounded, then added to
    the routed k-sum and rounded once more; with ``"Y"`` (the module composition) the
    three terms are summed and rounded once (autograd's accumulation order is not
    modelled; it moves the result by at most an ulp or two). ``f32_weight_grads``: the
    weight grads (gate, routed, shared) are left unrounded, as the path writes them for
    fp32 master weights under bf16 autocast; everything else rounds as ``store`` says.
    """

    def __init__(self, Wgate, expert_biases, W1, W2, k, shared=None, round_probs_bf16=False, store=None,
                 gate_scale_on="Y", expert_ids=None, f32_weight_grads=False):
        """``expert_ids`` (sorted, optional): W1 and W2 hold only these experts' weights
        (a compact stack for checks on a few tokens of a wide layer); the routing still
        runs over all gate rows, and tokens must select only these experts. dW1 / dW2
        then cover the same experts."""
        self.expert_ids = None if expert_ids is None else np.asarray(expert_ids, dtype=np.int64)
        self.Wgate = np.asarray(Wgate, dtype=_f())
        self.bias = np.asarray(expert_biases, dtype=np.float32)
        self.W1 = np.asarray(W1, dtype=_f())
        self.W2 = np.asarray(W2, dtype=_f())
        self.k = int(k)
        self.shared = None if shared is None else tuple(np.asarray(w, dtype=_f()) for w in shared)
        self.round_probs_bf16 = round_probs_bf16
        self.store = store
        self.gate_scale_on = gate_scale_on
        self.round_wgrads = not f32_weight_grads

    def forward(self, x, logits=None):
        x = np.asarray(x, dtype=_f())
        if logits is None:
            logits = (x @ self.Wgate.T).astype(np.float32)                    # moe_gate.py:26
        idx, w, p_sel = route_topk(logits, self.bias, self.k, self.round_probs_bf16)
        scache, ys = None, None
        if self.shared is not None:
            ys, scache = shared_expert_forward(x, *self.shared, store=self.store)   # moe_layer.py:47
        local = idx
        if self.expert_ids is not None:
            local = np.searchsorted(self.expert_ids, idx)
            if np.any(local >= self.expert_ids.size) or np.any(self.expert_ids[np.minimum(
                    local, self.expert_ids.size - 1)] != idx):
                raise ValueError("a token selected an expert outside expert_ids")
        out, mcache = glu_mlp_forward(x, w, local, self.W1, self.W2, store=self.store,  # moe_layer.py:51-53
                                      gate_scale_on=self.gate_scale_on, residual=ys)
        self._cache = dict(x=x, idx=idx, w=w, p_sel=p_sel, mcache=mcache, scache=scache)
        return out, idx, w

    def backward(self, dout, rss=False):
        """Returns dict of grads: x, gate_weight, W1, W2 (+ shared_*), d_gates, d_logits.
        With ``rss=True`` also "rss": the summand root-sum-square of every weight grad and
        of d_gates, keyed like the grads."""
        r = storage_rounder(self.store)
        c = self._cache
        dout = np.asarray(dout, dtype=_f())
        res = glu_mlp_backward(dout, c["mcache"], rss=rss, round_wgrads=self.round_wgrads)
        dx_routed, dW1, dW2, d_gates = res[:4]
        E = self.Wgate.shape[0]
        dz = r(route_topk_backward(d_gates, c["p_sel"], c["idx"], E))
        rw = r if self.round_wgrads else storage_rounder(None)
        grads = {"gate_weight": rw(dz.T @ c["x"])}
        if rss:
            grads["rss"] = dict(res[4], gate_weight=summand_rss(lambda a, b: a.T @ b, dz, c["x"]))
        dx_dense = dz @ self.Wgate
        if self.shared is not None:
            sres = shared_expert_backward(dout, c["scache"], *self.shared, store=self.store, rss=rss,
                                          round_wgrads=self.round_wgrads)
            dxs, dWg, dWu, dWd = sres[:4]
            dx_dense = dx_dense + dxs
            grads.update(shared_gate=dWg, shared_up=dWu, shared_down=dWd)
            if rss:
                grads["rss"].update({"shared_" + n: v for n, v in sres[4].items()})
        if self.gate_scale_on == "A":
            dx_dense = r(dx_dense)
        grads.update(x=r(dx_routed + dx_dense), W1=dW1, W2=dW2, d_gates=d_gates, d_logits=dz)
        return grads


# --------------------------------------------------------------------------- #
# (f)-2: the RMSNorm producer and the unpad gather in front of the layer
# --------------------------------------------------------------------------- #
def zc_rmsnorm_rows(hidden, weight, eps=1e-6, rows=None):
    """ZeroCenteredRMSNorm (modeling/zRMSNorm.py:10-17) then index_first_axis
    (modeling/moe_layer.py:39-42): y[i] = h * rsqrt(mean(h^2) + eps) * (1 + w) with
    h = hidden[rows[i]] (all rows when ``rows`` is None). Float arithmetic throughout
    (the reference's fp32, here this module's float type); the caller rounds to the
    input dtype. Returns (y [n, d], rstd [n])."""
    H = np.asarray(hidden, dtype=_f())
    H = H if rows is None else H[np.asarray(rows, dtype=np.int64)]
    r = 1.0 / np.sqrt((H * H).mean(axis=-1, keepdims=True) + eps)
    return H * r * (1.0 + np.asarray(weight, dtype=_f())), r[:, 0]


def zc_rmsnorm_rows_backward(dy, hidden, weight, rstd, rows=None):
    """Autograd of ``zc_rmsnorm_rows``: (dhidden [N, d], zero outside ``rows``; dweight [d]).

    With g = dy (1 + w): dh = r g - h r^3 / d * sum_j g_j h_j; dw = sum_i dy_i h_i r_i."""
    H_all = np.asarray(hidden, dtype=_f())
    idx = np.arange(H_all.shape[0]) if rows is None else np.asarray(rows, dtype=np.int64)
    H = H_all[idx]
    dy = np.asarray(dy, dtype=_f())
    r = np.asarray(rstd, dtype=_f())[:, None]
    g = dy * (1.0 + np.asarray(weight, dtype=_f()))
    dh = r * g - H * r ** 3 * (g * H).sum(axis=-1, keepdims=True) / H.shape[-1]
    dH = np.zeros_like(H_all)
    dH[idx] = dh
    return dH, (dy * H * r).sum(axis=0)


# --------------------------------------------------------------------------- #
# (f)-1: aux-loss-free bias update and load metrics
# --------------------------------------------------------------------------- #
def bias_update(expert_biases, topk_idx, E, update_rate):
    """main.py:161-175: b += gamma * sign(mean(counts) - counts), in float32."""
    counts = expert_counts(topk_idx, E).astype(np.float32)
    if np.asarray(topk_idx).size == 0:
        return np.asarray(expert_biases, dtype=np.float32).copy()
    err = np.float32(counts.mean(dtype=np.float32)) - counts
    return (np.asarray(expert_biases, dtype=np.float32)
            + np.float32(update_rate) * np.sign(err).astype(np.float32)).astype(np.float32)


def moe_load_metrics(topk_idx, E):
    """utils/trainutils.py:124-135 per-layer metrics from the expert histogram."""
    counts = expert_counts(topk_idx, E)
    total = np.asarray(topk_idx).size
    expected = total / E
    return dict(
        pct_experts_used=100.0 * float((counts > 0).sum()) / E,
        load_imbalance=float(np.abs(counts / expected - 1.0).mean()),
        max_expert_pct=float(counts.max()) * 100.0 / total,
        min_expert_pct=float(counts.min()) * 100.0 / total,
    )


# --------------------------------------------------------------------------- #
# (f)-3: Newton-Schulz orthogonalisation inside the MuonMD step
# --------------------------------------------------------------------------- #
NS_COEFFS = (3.4445, -4.7750, 2.0315)  # optimizer/muon.py:16


def newton_schulz5(G, steps, coeffs=NS_COEFFS, bf16=True):
    """optimizer/muon.py:6-32 on G [..., m, n] (float64 arithmetic).

    bf16=True models the reference's bf16 tensor arithmetic: the input is rounded to
    bf16; every GEMM result (float64 here, fp32-accumulated there) is rounded to
    float32 and then to bf16; every elementwise product or sum is formed in float32
    and rounded to bf16. ``c * A @ A`` parses as ``(c * A) @ A`` (muon.py:26).
    bf16=False is exact arithmetic (no rounding), which the SVD closed form pins.
    Returns float32 values (bf16-representable in bf16 mode).
    """
    a, b, c = (np.float32(v) for v in coeffs)
    G = np.asarray(G)
    tall = G.shape[-2] > G.shape[-1]

    def rnd(x):
        return bf16_round(np.asarray(x, dtype=np.float32)).astype(np.float64) if bf16 else np.asarray(x, np.float64)

    def mul(s, x):  # python-float scalar times a bf16 tensor: float32 opmath, one rounding
        return rnd(np.float32(s) * np.asarray(x, np.float32)) if bf16 else float(s) * x

    def add(x, y):
        return rnd(np.asarray(x, np.float32) + np.asarray(y, np.float32)) if bf16 else x + y

    X = rnd(G.astype(np.float32) if bf16 else G.astype(np.float64))
    if tall:
        X = np.swapaxes(X, -1, -2)
    nrm = np.sqrt((X * X).sum(axis=(-2, -1), keepdims=True))
    if bf16:
        nrm = rnd(nrm)
        den = rnd(np.float32(nrm) + np.float32(1e-7))
        X = rnd(np.asarray(X, np.float32) / np.asarray(den, np.float32))
    else:
        X = X / (nrm + 1e-7)
    for _ in range(steps):
        A = rnd(X @ np.swapaxes(X, -1, -2))
        B = add(mul(b, A), rnd(mul(c, A) @ A))
        X = add(mul(a, X), rnd(B @ X))
    if tall:
        X = np.swapaxes(X, -1, -2)
    return np.asarray(X, dtype=np.float32)
