"""Pins the CPU oracle against brute force, closed forms, invariants, an
independent torch-autograd formulation and float64 finite differences.

The reference ships no tests or golden vectors for the MoE path, so each oracle
function is pinned here by mathematics chosen so that a plausible mistake (a
dropped term, a wrong sign or index, a transposed operand) fails a check.
"""

import math
import types

import numpy as np
import pytest
import torch

import oracle as O


def rng(seed=0):
    return np.random.default_rng(seed)


# ----------------------------------------------------------------- numerics
def test_bf16_round_matches_torch():
    x = rng(1).standard_normal(4096).astype(np.float32) * 10
    x[:4] = [0.0, -0.0, np.inf, -np.inf]
    ref = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(O.bf16_round(x), ref)
    assert np.isnan(O.bf16_round(np.array([np.nan], np.float32)))[0]


def test_sigmoid_closed_forms():
    assert O.sigmoid_f32(np.array([0.0]))[0] == np.float32(0.5)
    x = rng(2).standard_normal(1000) * 8
    p, q = O.sigmoid_f32(x).astype(np.float64), O.sigmoid_f32(-x).astype(np.float64)
    np.testing.assert_allclose(p + q, 1.0, atol=2e-7)
    assert O.sigmoid_f32(np.array([-1000.0]))[0] == 0.0
    assert O.sigmoid_f32(np.array([1000.0]))[0] == 1.0
    # correctly rounded: agrees with float64 math.exp for a few values
    for v in (0.25, -3.5, 7.0):
        assert O.sigmoid_f32(np.array([v]))[0] == np.float32(1.0 / (1.0 + math.exp(-v)))


def _sigmoid_correctly_rounded_f32(z: float) -> np.float32:
    """sigmoid(z) to 50 digits (decimal), then the nearest float32 (ties impossible but
    at z = 0), by comparing the candidate and its neighbours exactly."""
    import decimal

    ctx = decimal.Context(prec=50)
    d = ctx.divide(1, ctx.add(1, ctx.exp(decimal.Decimal(-z))))
    f = np.float32(float(d))
    cands = [np.nextafter(f, np.float32(-1)), f, np.nextafter(f, np.float32(2))]
    return min(cands, key=lambda c: abs(decimal.Decimal(float(c)) - d))


def test_sigmoid_is_correctly_rounded():
    """Against a 50-digit evaluation rounded to the nearest float32: every bf16 logit (the
    small ones land on fp32 rounding ties of 0.5 + z/4 that a float64 evaluation cannot
    resolve) and a sample of float32 logits, outside the saturated range."""
    z16 = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    r = rng(21)
    zf = np.concatenate([(r.standard_normal(3000) * 6).astype(np.float32),
                         (r.standard_normal(3000) * 1e-4).astype(np.float32),
                         np.float32(2.0 ** -12) * np.array([0.999999, 1.0, -0.999999, -1.0], np.float32)])
    for z in (z16, zf):
        z = z[np.isfinite(z) & (z > O.SIGMOID_ZERO_BELOW)]
        got = O.sigmoid_f32(z)
        ref = np.array([_sigmoid_correctly_rounded_f32(float(v)) for v in z], np.float32)
        bad = got.view(np.uint32) != ref.view(np.uint32)
        assert not bad.any(), (z[bad][:5], got[bad][:5], ref[bad][:5])


def test_sigmoid_saturates_where_torch_does():
    """Every float32 logit in [-100, -85]: the oracle's p is 0 exactly where torch's float32
    sigmoid is 0 (its exp(-z) overflows), and subnormal-or-larger elsewhere."""
    lo, hi = np.float32(-85.0).view(np.uint32), np.float32(-100.0).view(np.uint32)
    z = np.arange(lo, hi, dtype=np.uint32).view(np.float32)
    t = torch.sigmoid(torch.from_numpy(z)).numpy()
    p = O.sigmoid_f32(z)
    np.testing.assert_array_equal(p == 0, t == 0)
    assert (z[p == 0] <= O.SIGMOID_ZERO_BELOW).all() and (p[z > O.SIGMOID_ZERO_BELOW] > 0).all()
    # away from saturation the two differ by at most an ulp of float32
    np.testing.assert_allclose(p[p > 0], t[p > 0], rtol=2.4e-7, atol=0)


# ----------------------------------------------------------------- routing
def _brute_route(logits, bias, k, round_bf16=False):
    T, E = logits.shape
    p = O.sigmoid_f32(logits)
    if round_bf16:
        p = O.bf16_round(p)
    s = (p + bias[None, :]).astype(np.float32)
    idx = np.zeros((T, k), np.int64)
    for t in range(T):
        def key(e):
            v = float(s[t, e])
            return (0 if math.isnan(v) else 1, 0.0 if math.isnan(v) else -v, e)
        order = sorted(range(E), key=key)
        idx[t] = order[:k]
    return idx, p


@pytest.mark.parametrize("round_bf16", [False, True])
def test_route_topk_brute_force(round_bf16):
    r = rng(3)
    T, E, k = 64, 7, 3
    logits = r.standard_normal((T, E)).astype(np.float32)
    logits[:8] = np.round(logits[:8])  # exact ties inside rows
    bias = (r.standard_normal(E) * 0.1).astype(np.float32)
    bias[:3] = 0.0
    idx, w, p_sel = O.route_topk(logits, bias, k, round_probs_bf16=round_bf16)
    bidx, p = _brute_route(logits, bias, k, round_bf16)
    np.testing.assert_array_equal(idx, bidx)
    np.testing.assert_array_equal(p_sel, np.take_along_axis(p, bidx, 1))
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=0, atol=k * 2e-7)
    assert (w > 0).all()


def test_route_equal_scores_pick_lowest_indices():
    idx, w, _ = O.route_topk(np.zeros((5, 16), np.float32), np.zeros(16, np.float32), 4)
    np.testing.assert_array_equal(idx, np.tile(np.arange(4), (5, 1)))
    np.testing.assert_allclose(w, 0.25)


def test_route_bias_selects_but_weight_uses_unbiased_p():
    r = rng(4)
    logits = r.standard_normal((10, 8)).astype(np.float32)
    bias = np.zeros(8, np.float32)
    bias[5] = 100.0
    idx, w, p_sel = O.route_topk(logits, bias, 2)
    assert (idx[:, 0] == 5).all()
    p = O.sigmoid_f32(logits)
    np.testing.assert_array_equal(p_sel[:, 0], p[:, 5])
    # with b = 0 selection is the top-k of p
    idx0, _, _ = O.route_topk(logits, np.zeros(8, np.float32), 2)
    np.testing.assert_array_equal(np.sort(idx0, 1), np.sort(np.argsort(-p, 1, kind="stable")[:, :2], 1))


def test_route_nan_ranks_first():
    logits = np.zeros((1, 6), np.float32)
    logits[0, 4] = np.nan
    logits[0, 2] = 3.0
    idx, _, _ = O.route_topk(logits, np.zeros(6, np.float32), 3)
    np.testing.assert_array_equal(idx[0], [4, 2, 0])


def test_route_backward_matches_autograd():
    r = rng(5)
    T, E, k = 12, 9, 3
    logits = r.standard_normal((T, E))
    idx, w, p_sel = O.route_topk(logits.astype(np.float32), np.zeros(E, np.float32), k)
    dw = r.standard_normal((T, k))
    z = torch.tensor(logits.astype(np.float32).astype(np.float64), requires_grad=True)
    p = torch.sigmoid(z)
    wt = torch.nn.functional.normalize(p.gather(1, torch.from_numpy(idx)), p=1, dim=-1)
    (wt * torch.from_numpy(dw)).sum().backward()
    # the oracle starts from float32 p; compare at float32 resolution
    dz = O.route_topk_backward(dw, p_sel, idx, E)
    np.testing.assert_allclose(dz, z.grad.numpy(), rtol=1e-5, atol=1e-6)


# ----------------------------------------------------------------- sort / count
def test_flatten_sort_count_brute_force():
    r = rng(6)
    T, k, E = 50, 4, 9
    idx = np.stack([r.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
    se, ss, off = O.flatten_sort_count(idx, E)
    flat = idx.reshape(-1)
    order = sorted(range(flat.size), key=lambda i: (flat[i], i))
    np.testing.assert_array_equal(ss, order)
    np.testing.assert_array_equal(se, flat[order])
    counts = [int((flat == e).sum()) for e in range(E)]
    np.testing.assert_array_equal(off, np.cumsum(counts))
    assert off[-1] == T * k
    np.testing.assert_array_equal(np.sort(ss), np.arange(T * k))
    inv = O.inverse_permutation(ss)
    np.testing.assert_array_equal(ss[inv], np.arange(T * k))


def test_counts_reject_out_of_range():
    with pytest.raises(ValueError):
        O.expert_counts(np.array([0, 5]), 5)


# ----------------------------------------------------------------- group / gemm
def test_group_identity():
    r = rng(7)
    A = r.standard_normal((6, 5))
    idx = r.permutation(12)
    c = r.standard_normal(12)
    Y = O.group(A, idx, coeff=c, fan_out=2)
    for n in range(12):
        np.testing.assert_allclose(Y[n], A[idx[n] // 2] * c[idx[n]])


@pytest.mark.parametrize("xg,yg", [(False, True), (True, False), (True, True), (False, False)])
def test_scatter2scatter_rowwise_loop(xg, yg):
    r = rng(8)
    T, k, E, K, N = 11, 2, 4, 6, 5
    idx = np.stack([r.choice(E, k, replace=False) for _ in range(T)])
    se, ss, _ = O.flatten_sort_count(idx, E)
    X = r.standard_normal((T * k if xg else T, K))
    W = r.standard_normal((E, K, N))
    b = r.standard_normal((E, N))
    Y = O.scatter2scatter(X, W, se, ss, k, b=b, x_grouped=xg, y_grouped=yg)
    for i in range(T * k):
        xin = X[i] if xg else X[ss[i] // k]
        row = i if yg else ss[i]
        ref = np.array([sum(xin[q] * W[se[i], q, n] for q in range(K)) + b[se[i], n] for n in range(N)])
        np.testing.assert_allclose(Y[row], ref, rtol=1e-12, atol=1e-12)


def test_group_bwd_w_outer_products_and_empty_expert():
    r = rng(9)
    E, K, N = 5, 3, 4
    counts = np.array([3, 0, 2, 4, 0])
    off = np.cumsum(counts)
    M = off[-1]
    X, DY = r.standard_normal((M, K)), r.standard_normal((M, N))
    DW, Db = O.group_bwd_w(DY, X, off, E, has_bias=True)
    start = 0
    for e in range(E):
        ref = np.zeros((K, N))
        for i in range(start, off[e]):
            ref += np.outer(X[i], DY[i])
        np.testing.assert_allclose(DW[e], ref, atol=1e-12)
        start = off[e]
    assert not DW[1].any() and not DW[4].any() and not Db[1].any()


# ----------------------------------------------------------------- ParallelLinear
# The modes a caller of ParallelLinear can use (reference parallel_experts.py:34-135).
# A gathered input fans each token out to its ``fan`` slots (k = fan). A grouped input
# is already one row per slot, so it is called with k = 1, as GLUMLP's W2 is (mlp.py:89);
# the reference's k-sum at :124-125 would not fit any other k. Gates [T, fan] combine
# the slot rows of a token, so they go with slot-order output (:50-52).
_PL_MODES = [
    # (fan, grouped_in, grouped_out, gates, bias)
    (3, False, False, False, False),
    (1, False, False, False, True),
    (3, False, True, False, True),
    (3, False, False, True, False),
    (3, False, False, True, True),
    (3, True, False, False, True),
    (3, True, True, False, False),
    (3, True, False, True, True),
]


def _pl_case(seed, fan, grouped_in, gates, bias, T=5, E=4, K=6, N=5):
    r = rng(seed)
    idx = np.stack([r.choice(E, fan, replace=False) for _ in range(T)])
    se, ss, off = O.flatten_sort_count(idx, E)
    R = T * fan
    C = dict(
        x=r.standard_normal((R if grouped_in else T, K)),
        W=r.standard_normal((E, K, N)),
        b=r.standard_normal((E, N)) if bias else None,
        gates=(r.random((T, fan)) + 0.2) if gates else None,
    )
    return C, se, ss, off, (1 if grouped_in else fan)


def _pl_torch(C, se, ss, k, grouped_in, grouped_out):
    """ParallelLinear written slot by slot in torch float64 (autograd supplies the
    backward): sorted position i applies expert se[i] to row i of a grouped input, or
    to token ss[i] // k of a gathered one, and writes the slot's row ss[i], or row i
    when the output is grouped; gates then weight the fan rows of each token."""
    t = lambda a: None if a is None else torch.tensor(a, dtype=torch.float64, requires_grad=True)
    x, W, b, g = t(C["x"]), t(C["W"]), t(C["b"]), t(C["gates"])
    R = se.size
    rows = [None] * R
    for i in range(R):
        slot = int(ss[i])
        xin = x[i] if grouped_in else x[slot // k]
        y = xin @ W[int(se[i])]
        if b is not None:
            y = y + b[int(se[i])]
        rows[i if grouped_out else slot] = y
    Y = torch.stack(rows)
    if g is not None:
        fan = g.shape[1]
        out = torch.stack([sum(g[tt, j] * Y[tt * fan + j] for j in range(fan)) for tt in range(g.shape[0])])
    else:
        out = Y
    return out, (x, W, b, g)


@pytest.mark.parametrize("fan,grouped_in,grouped_out,gates,bias", _PL_MODES)
def test_parallel_linear_vs_torch_autograd(fan, grouped_in, grouped_out, gates, bias):
    C, se, ss, off, k = _pl_case(30 + fan, fan, grouped_in, gates, bias)
    out, expanded = O.parallel_linear_forward(C["x"], C["W"], k, se, ss, off, b=C["b"], gates=C["gates"],
                                              grouped_in=grouped_in, grouped_out=grouped_out)
    tout, (x, W, b, g) = _pl_torch(C, se, ss, k, grouped_in, grouped_out)
    np.testing.assert_allclose(out, tout.detach().numpy(), rtol=1e-12, atol=1e-12)
    assert (expanded is None) == (not gates)
    dy = rng(40).standard_normal(out.shape)
    dx, dW, db, dg = O.parallel_linear_backward(dy, C["x"], C["W"], k, se, ss, off, b=C["b"], gates=C["gates"],
                                                output_expanded=expanded, grouped_in=grouped_in,
                                                grouped_out=grouped_out)
    (tout * torch.from_numpy(dy)).sum().backward()
    np.testing.assert_allclose(dx, x.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dW, W.grad.numpy(), rtol=1e-12, atol=1e-12)
    if bias:
        np.testing.assert_allclose(db, b.grad.numpy(), rtol=1e-12, atol=1e-12)
    else:
        assert db is None
    if gates:
        np.testing.assert_allclose(dg, g.grad.numpy(), rtol=1e-12, atol=1e-12)
    else:
        assert dg is None


@pytest.mark.parametrize("fan,grouped_in,grouped_out,gates,bias", [_PL_MODES[2], _PL_MODES[4], _PL_MODES[7]])
def test_parallel_linear_finite_differences(fan, grouped_in, grouped_out, gates, bias):
    """Central differences in float64 of <out, dy> against the oracle's backward."""
    C, se, ss, off, k = _pl_case(50 + fan, fan, grouped_in, gates, bias, T=4, E=3, K=4, N=3)
    kw = dict(grouped_in=grouped_in, grouped_out=grouped_out)
    out, expanded = O.parallel_linear_forward(C["x"], C["W"], k, se, ss, off, b=C["b"], gates=C["gates"], **kw)
    dy = rng(51).standard_normal(out.shape)
    grads = O.parallel_linear_backward(dy, C["x"], C["W"], k, se, ss, off, b=C["b"], gates=C["gates"],
                                       output_expanded=expanded, **kw)
    named = dict(zip(("x", "W", "b", "gates"), grads))

    def loss():
        y, _ = O.parallel_linear_forward(C["x"], C["W"], k, se, ss, off, b=C["b"], gates=C["gates"], **kw)
        return float((y * dy).sum())

    eps = 1e-6
    for name in ("x", "W", "b", "gates"):
        if C[name] is None:
            continue
        flat = C[name].reshape(-1)
        for q in range(flat.size):
            old = flat[q]
            flat[q] = old + eps
            lp = loss()
            flat[q] = old - eps
            lm = loss()
            flat[q] = old
            num = (lp - lm) / (2 * eps)
            assert abs(num - named[name].reshape(-1)[q]) < 1e-7 * max(1.0, abs(num)), (name, q)


def _torch_bf16_parallel_linear(C, se, ss, k, grouped_in, grouped_out, dy):
    """The reference's ParallelLinear composition in torch's own bf16 tensor arithmetic
    (CPU autograd): per-expert bf16 matmuls (fp32 accumulation, one rounding; addmm adds
    the bias before it, as the reference's kernel does, ops.py:181-183), the slot rows assembled in a bf16 buffer and combined by a
    bf16 bmm with bf16 gates (parallel_experts.py:50-52). A gathered x comes from a float32
    leaf cast after the gather, so its k slots' grads are summed in fp32 and rounded once
    (as the path's k-sum does)."""
    bf = torch.bfloat16
    x = torch.tensor(C["x"], dtype=torch.float32).requires_grad_(True)
    W = torch.tensor(C["W"]).to(bf).requires_grad_(True)
    b = None if C["b"] is None else torch.tensor(C["b"]).to(bf).requires_grad_(True)
    g = None if C["gates"] is None else torch.tensor(C["gates"]).to(bf).requires_grad_(True)
    R, N = se.size, C["W"].shape[2]
    Y = torch.zeros(R, N, dtype=bf)
    for e in range(C["W"].shape[0]):
        pos = np.nonzero(se == e)[0]
        if pos.size == 0:
            continue
        rows_in = torch.from_numpy(pos if grouped_in else ss[pos] // k)
        ye = x[rows_in].to(bf) @ W[e] if b is None else torch.addmm(b[e], x[rows_in].to(bf), W[e])
        Y = Y.index_copy(0, torch.from_numpy(pos if grouped_out else ss[pos]), ye)
    out = Y if g is None else (g.unsqueeze(1) @ Y.view(g.shape[0], g.shape[1], N)).squeeze(1)
    (out.float() * torch.from_numpy(dy).float()).sum().backward()
    return out, x.grad.to(bf), W.grad, None if b is None else b.grad, None if g is None else g.grad


@pytest.mark.parametrize("fan,grouped_in,grouped_out,gates,bias", _PL_MODES)
def test_parallel_linear_bf16_store_matches_torch_bf16_arithmetic(fan, grouped_in, grouped_out, gates, bias):
    """store="bf16" rounds where the reference's composition in bf16 tensor arithmetic
    stores: bit for bit but for rare accumulation-order flips (torch sums in float32, the
    oracle in float64), and far closer to torch's results than the exact mode, so a rounding
    point left out, added or misplaced fails."""
    T, E, K, N = 48, 4, 64, 40
    C, se, ss, off, k = _pl_case(70 + fan, fan, grouped_in, gates, bias, T=T, E=E, K=K, N=N)
    b16 = lambda a: None if a is None else O.bf16_round(np.asarray(a, np.float32)).astype(np.float64)  # noqa: E731
    C = {key: b16(v) for key, v in C.items()}
    dy = b16(rng(71).standard_normal((T, N) if gates else (T * fan, N)))
    tres = [None if t is None else t.detach().double().numpy()
            for t in _torch_bf16_parallel_linear(C, se, ss, k, grouped_in, grouped_out, dy)]
    got = {}
    for store in (None, "bf16"):
        out, exp = O.parallel_linear_forward(C["x"], C["W"], k, se, ss, off, b=C["b"], gates=C["gates"],
                                             grouped_in=grouped_in, grouped_out=grouped_out, store=store)
        dx, dW, db, dg = O.parallel_linear_backward(dy, C["x"], C["W"], k, se, ss, off, b=C["b"],
                                                    gates=C["gates"], output_expanded=exp, grouped_in=grouped_in,
                                                    grouped_out=grouped_out, store=store)
        got[store] = (out, O.bf16_round(dx) if store is None else dx, dW, db, dg)
    for i, name in enumerate(("out", "dx", "dW", "db", "d_gates")):
        ref = tres[i]
        if ref is None:
            assert got["bf16"][i] is None
            continue
        same = np.mean(got["bf16"][i] == ref)
        assert same >= 0.99, (name, same)
        assert np.all(np.abs(got["bf16"][i] - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-30), name
        eb, ee = _rel_fro(got["bf16"][i], ref), _rel_fro(got[None][i], ref)
        assert eb <= 0.25 * ee or eb == 0.0, (name, eb, ee)


def test_rowwise_sum_product():
    r = rng(10)
    A, B = r.standard_normal((4, 3, 7)), r.standard_normal((4, 7))
    out = O.rowwise_sum_product(A, B)
    for t in range(4):
        for j in range(3):
            assert abs(out[t, j] - sum(A[t, j, h] * B[t, h] for h in range(7))) < 1e-12


# ----------------------------------------------------------------- layer backward
def _tiny_layer(seed, shared=True, T=6, d=8, E=4, k=2, f=4, fs=4):
    r = rng(seed)
    P = dict(
        x=r.standard_normal((T, d)),
        Wg=r.standard_normal((E, d)) * 0.5,
        bias=(r.standard_normal(E) * 0.1).astype(np.float32),
        W1=r.standard_normal((E, 2 * f, d)) / math.sqrt(d),
        W2=r.standard_normal((E, d, f)) / math.sqrt(f),
        shared=(r.standard_normal((fs, d)) / math.sqrt(d), r.standard_normal((fs, d)) / math.sqrt(d),
                r.standard_normal((d, fs)) / math.sqrt(fs)) if shared else None,
        k=k,
    )
    return P


def _torch_dense_layer(P, idx):
    """Independent dense formulation (per-token loop) for torch autograd."""
    t = lambda a: torch.tensor(a, dtype=torch.float64, requires_grad=True)
    x, Wg, W1, W2 = t(P["x"]), t(P["Wg"]), t(P["W1"]), t(P["W2"])
    shared = [t(w) for w in P["shared"]] if P["shared"] is not None else None
    p = torch.sigmoid((x @ Wg.T).float().double())
    sel = torch.from_numpy(idx)
    w = torch.nn.functional.normalize(p.gather(1, sel), p=1, dim=-1)
    f = W1.shape[1] // 2
    rows = []
    for ti in range(x.shape[0]):
        acc = 0
        for j in range(idx.shape[1]):
            e = int(idx[ti, j])
            hg = W1[e] @ x[ti]
            a = torch.nn.functional.silu(hg[f:]) * hg[:f]
            acc = acc + w[ti, j] * (W2[e] @ a)
        rows.append(acc)
    out = torch.stack(rows)
    if shared is not None:
        g, u, dn = shared
        out = out + (torch.nn.functional.silu(x @ g.T) * (x @ u.T)) @ dn.T
    return out, (x, Wg, W1, W2, shared)


@pytest.mark.parametrize("shared", [True, False])
def test_layer_forward_backward_vs_torch_autograd(shared):
    P = _tiny_layer(11, shared=shared)
    orc = O.MoELayerOracle(P["Wg"], P["bias"], P["W1"], P["W2"], P["k"], shared=P["shared"])
    # route from float32 logits computed identically on both sides
    logits = (P["x"] @ P["Wg"].T).astype(np.float32)
    out, idx, _ = orc.forward(P["x"], logits=logits)
    dout = rng(12).standard_normal(out.shape)
    g = orc.backward(dout)
    tout, (x, Wg, W1, W2, sh) = _torch_dense_layer(P, idx)
    np.testing.assert_allclose(out, tout.detach().numpy(), rtol=1e-6, atol=1e-6)
    (tout * torch.from_numpy(dout)).sum().backward()
    # The oracle's p is float32-rounded; the torch path rounds logits to float32 too.
    tol = dict(rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(g["W1"], W1.grad.numpy(), **tol)
    np.testing.assert_allclose(g["W2"], W2.grad.numpy(), **tol)
    np.testing.assert_allclose(g["x"], x.grad.numpy(), **tol)
    np.testing.assert_allclose(g["gate_weight"], Wg.grad.numpy(), **tol)
    if shared:
        np.testing.assert_allclose(g["shared_gate"], sh[0].grad.numpy(), **tol)
        np.testing.assert_allclose(g["shared_up"], sh[1].grad.numpy(), **tol)
        np.testing.assert_allclose(g["shared_down"], sh[2].grad.numpy(), **tol)


def test_glu_mlp_finite_differences():
    """Central differences of the routed experts in float64 (routing held fixed)."""
    P = _tiny_layer(13, shared=False, T=4, d=5, E=3, k=2, f=3)
    r = rng(14)
    idx = np.stack([r.choice(3, 2, replace=False) for _ in range(4)])
    gates = r.random((4, 2)) + 0.1
    dy = r.standard_normal((4, 5))

    def loss(x, W1, W2, gates):
        y, _ = O.glu_mlp_forward(x, gates, idx, W1, W2)
        return float((y * dy).sum())

    y, cache = O.glu_mlp_forward(P["x"], gates, idx, P["W1"], P["W2"])
    dx, dW1, dW2, dg = O.glu_mlp_backward(dy, cache)
    eps = 1e-6
    args = dict(x=P["x"].copy(), W1=P["W1"].copy(), W2=P["W2"].copy(), gates=gates.copy())
    for name, analytic in (("x", dx), ("W1", dW1), ("W2", dW2), ("gates", dg)):
        a = args[name]
        flat = a.reshape(-1)
        for q in r.choice(flat.size, min(12, flat.size), replace=False):
            old = flat[q]
            flat[q] = old + eps
            lp = loss(**args)
            flat[q] = old - eps
            lm = loss(**args)
            flat[q] = old
            num = (lp - lm) / (2 * eps)
            assert abs(num - analytic.reshape(-1)[q]) < 1e-6 * max(1.0, abs(num)), (name, q)


# ----------------------------------------------------------------- bias update
def test_bias_update_closed_form():
    idx = np.array([[0, 1], [0, 2], [0, 1]])  # counts [3, 2, 1, 0], mean 1.5
    b = O.bias_update(np.zeros(4, np.float32), idx, 4, 1e-3)
    np.testing.assert_array_equal(b, np.array([-1e-3, -1e-3, 1e-3, 1e-3], np.float32))
    m = O.moe_load_metrics(idx, 4)
    assert m["pct_experts_used"] == 75.0 and m["max_expert_pct"] == 50.0 and m["min_expert_pct"] == 0.0
    assert abs(m["load_imbalance"] - np.mean(np.abs(np.array([3, 2, 1, 0]) / 1.5 - 1))) < 1e-12


# ----------------------------------------------------------------- Newton-Schulz (MuonMD)
def _phi_power(s, steps):
    a, b, c = O.NS_COEFFS
    for _ in range(steps):
        s = a * s + b * s**3 + c * s**5
    return s


@pytest.mark.parametrize("shape", [(3, 6, 10), (2, 12, 5), (1, 9, 9)])
@pytest.mark.parametrize("steps", [0, 1, 5])
def test_newton_schulz_exact_is_svd_closed_form(shape, steps):
    """Exact arithmetic: NS(G) = U phi^steps(S / (||G||_F + 1e-7)) V^T (muon.py:21-27)."""
    G = np.random.default_rng(7).standard_normal(shape)
    got = O.newton_schulz5(G, steps, bf16=False).astype(np.float64)
    for e in range(shape[0]):
        U, S, Vt = np.linalg.svd(G[e], full_matrices=False)
        s = S / (np.linalg.norm(G[e]) + 1e-7)
        ref = (U * _phi_power(s, steps)) @ Vt
        np.testing.assert_allclose(got[e], ref, rtol=0, atol=1e-6 * max(1.0, np.abs(ref).max()))


def test_newton_schulz_transpose_symmetry():
    G = np.random.default_rng(8).standard_normal((2, 8, 24)).astype(np.float32)
    for bf16 in (False, True):
        a = O.newton_schulz5(G, 5, bf16=bf16)
        b = O.newton_schulz5(np.swapaxes(G, -1, -2), 5, bf16=bf16)
        np.testing.assert_array_equal(a, np.swapaxes(b, -1, -2))


def _torch_ns_steps(G, steps):
    """The reference expression in torch bf16 tensor ops (CPU), X after each step."""
    a, b, c = O.NS_COEFFS
    X = torch.from_numpy(G).bfloat16()
    tall = X.size(-2) > X.size(-1)
    if tall:
        X = X.mT
    X = X / (X.norm(dim=(-2, -1), keepdim=True) + 1e-7)
    out = []
    for _ in range(steps):
        A = X @ X.mT
        B = b * A + c * A @ A
        X = a * X + B @ X
        out.append((X.mT if tall else X).float().numpy())
    return out


@pytest.mark.parametrize("shape", [(3, 8, 16), (2, 16, 8), (4, 32, 48)])
@pytest.mark.parametrize("seed", [9, 10, 11])
def test_newton_schulz_bf16_rounding_points_match_torch(shape, seed):
    """bf16 mode rounds where torch's bf16 tensor ops round (CPU torch, tiny sizes).

    One step is compared bit for bit. Over five steps a single accumulation-order
    flip in one GEMM output (torch sums in float32, the oracle in float64) is
    amplified by the iteration (slope a = 3.44 at 0), so five steps are compared by
    relative Frobenius error against the bf16 tolerance 2e-2.
    """
    G = np.random.default_rng(seed).standard_normal(shape).astype(np.float32)
    ref = _torch_ns_steps(G, 5)
    np.testing.assert_array_equal(O.newton_schulz5(G, 1), ref[0])
    got5 = O.newton_schulz5(G, 5)
    assert np.linalg.norm(got5 - ref[4]) <= 2e-2 * np.linalg.norm(ref[4])


def test_newton_schulz_singular_values_land_in_band():
    """The quintic drives every singular value of a well-conditioned input to ~[0.5, 1.5]."""
    G = np.random.default_rng(10).standard_normal((2, 32, 64))
    X = O.newton_schulz5(G, 5)
    for e in range(2):
        s = np.linalg.svd(X[e].astype(np.float64), compute_uv=False)
        assert s.min() > 0.5 and s.max() < 1.5, (s.min(), s.max())


# ----------------------------------------------------------------- bf16 storage model
def _bf16_inputs(seed, T=96, d=64, E=6, k=3, f=48, fs=32):
    """Tiny layer inputs, every value bf16-representable; gates from the routing."""
    r = rng(seed)
    b = lambda a: O.bf16_round(np.asarray(a, np.float32)).astype(np.float64)  # noqa: E731
    P = dict(
        x=b(r.standard_normal((T, d))),
        Wg=b(r.standard_normal((E, d)) / math.sqrt(d)),
        bias=(r.standard_normal(E) * 0.1).astype(np.float32),
        W1=b(r.standard_normal((E, 2 * f, d)) / math.sqrt(d)),
        W2=b(r.standard_normal((E, d, f)) / math.sqrt(d)),
        shared=tuple(b(r.standard_normal(s) / math.sqrt(d)) for s in ((fs, d), (fs, d), (d, fs))),
        dy=b(r.standard_normal((T, d))),
        k=k,
    )
    logits = O.bf16_round((P["x"] @ P["Wg"].T).astype(np.float32))
    P["idx"], P["w"], P["p"] = O.route_topk(logits, P["bias"], k, round_probs_bf16=True)
    P["logits"] = logits
    return P


def _torch_bf16_glu(P, gate_scale_on, residual):
    """The routed experts in torch's own bf16 tensor arithmetic (CPU), through autograd:
    bf16 matmuls (fp32 accumulation, one rounding), elementwise work in fp32 cast to
    bf16 where the path stores it, the combine summed in fp32 with the residual."""
    bf = torch.bfloat16
    # x is gathered from a float32 leaf, so the k slots' input grads are summed in fp32
    # (as the path's k-sum does) rather than in a bf16 buffer
    x = torch.tensor(P["x"], dtype=torch.float32).requires_grad_(True)
    W1 = torch.tensor(P["W1"]).to(bf).requires_grad_(True)
    W2 = torch.tensor(P["W2"]).to(bf).requires_grad_(True)
    gates = torch.tensor(P["w"]).requires_grad_(True)
    idx = torch.tensor(P["idx"])
    T, k = idx.shape
    f = W1.shape[1] // 2
    acc = torch.tensor(residual, dtype=torch.float32)
    saved = {}
    for e in range(W1.shape[0]):
        tok, slot = torch.nonzero(idx == e, as_tuple=True)
        if tok.numel() == 0:
            continue
        H = x[tok].to(bf) @ W1[e].T
        a = torch.nn.functional.silu(H[:, f:].float()) * H[:, :f].float()
        we = gates[tok, slot][:, None]
        A = (a if gate_scale_on == "Y" else we * a).to(bf)
        Y = A @ W2[e].T
        acc = acc.index_add(0, tok, Y.float() * we if gate_scale_on == "Y" else Y.float())
        saved[e] = (tok, H)
    y = acc.to(bf)
    (y.float() * torch.tensor(P["dy"], dtype=torch.float32)).sum().backward()
    return y, x.grad, W1.grad, W2.grad, gates.grad, saved


def _rel_fro(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def _f64(t):
    return t.detach().double().numpy()


@pytest.mark.parametrize("gate_scale_on", ["Y", "A"])
@pytest.mark.parametrize("seed", [31, 32])
def test_bf16_store_matches_torch_bf16_arithmetic(gate_scale_on, seed):
    """store="bf16" rounds where bf16 tensor arithmetic stores (torch CPU bf16 autograd).

    The stored tensors (H, the output, dW1, dW2) agree bit for bit except for rare
    accumulation-order flips (torch sums in float32, the oracle in float64), and every
    result is far closer to torch's than the exact mode is: a rounding point left out,
    added or misplaced shows up as the exact mode's ~2^-9 relative noise on many
    elements. dx differs more (torch accumulates the k slots' grads in bf16; the path
    sums them in fp32 and rounds once: dx is compared after that rounding)."""
    P = _bf16_inputs(seed)
    res = O.bf16_round(np.random.default_rng(seed + 100).standard_normal(P["x"].shape).astype(np.float32))
    ty, tdx, tdW1, tdW2, tdg, saved = _torch_bf16_glu(P, gate_scale_on, res)
    got = {}
    for store in (None, "bf16"):
        y, cache = O.glu_mlp_forward(P["x"], P["w"], P["idx"], P["W1"], P["W2"], store=store,
                                     gate_scale_on=gate_scale_on, residual=res.astype(np.float64))
        dx, dW1, dW2, dg = O.glu_mlp_backward(P["dy"], cache)
        got[store] = dict(y=y, dx=O.bf16_round(dx), W1=dW1, W2=dW2, g=dg, cache=cache)
    tdx = tdx.to(torch.bfloat16)
    b = got["bf16"]
    # H per expert (the first stored tensor): identical but for rare flips of one bf16 ulp
    for e, (tok, H) in saved.items():
        rows = np.nonzero(b["cache"]["se"] == e)[0]
        oh, th = b["cache"]["H"][rows], _f64(H)
        assert np.mean(oh == th) >= 0.995, e
        assert np.all(np.abs(oh - th) <= np.abs(th) * 2.0 ** -7), e
    for name, ref in (("y", _f64(ty)), ("dx", _f64(tdx)), ("W1", _f64(tdW1)), ("W2", _f64(tdW2))):
        same = np.mean(b[name] == ref)
        assert same >= 0.99, (name, same)
        assert np.mean(got[None][name] == ref) < 0.9 * same, name
    for name, ref in (("y", _f64(ty)), ("dx", _f64(tdx)), ("W1", _f64(tdW1)), ("W2", _f64(tdW2)),
                      ("g", _f64(tdg))):
        eb, ee = _rel_fro(b[name], ref), _rel_fro(got[None][name], ref)
        assert eb <= 0.25 * ee, (name, eb, ee)


@pytest.mark.parametrize("gate_scale_on", ["Y", "A"])
def test_f32_weight_grads_are_the_unrounded_bf16_store_grads(gate_scale_on):
    """f32_weight_grads leaves the weight grads unrounded and changes nothing else: rounding
    them to bf16 gives the bf16 storage model's grads bit for bit (that mode is pinned against
    torch's bf16 arithmetic above), the other grads and the output are identical, and the
    unrounded grads are not already bf16 values."""
    P = _bf16_inputs(41)
    kw = dict(shared=P["shared"], round_probs_bf16=True, store="bf16", gate_scale_on=gate_scale_on)
    got = {}
    for f32 in (False, True):
        orc = O.MoELayerOracle(P["Wg"], P["bias"], P["W1"], P["W2"], P["k"], f32_weight_grads=f32, **kw)
        out, idx, _ = orc.forward(P["x"], logits=P["logits"])
        got[f32] = (out, idx, orc.backward(P["dy"]))
    np.testing.assert_array_equal(got[True][0], got[False][0])
    np.testing.assert_array_equal(got[True][1], got[False][1])
    g32, g16 = got[True][2], got[False][2]
    for name in ("gate_weight", "W1", "W2", "shared_gate", "shared_up", "shared_down"):
        np.testing.assert_array_equal(O.bf16_round(g32[name].astype(np.float32)), g16[name], err_msg=name)
        assert np.mean(O.bf16_round(g32[name].astype(np.float32)) != g32[name]) > 0.5, name
    for name in ("x", "d_gates", "d_logits"):
        np.testing.assert_array_equal(g32[name], g16[name], err_msg=name)


def test_bf16_store_shared_expert_matches_torch():
    P = _bf16_inputs(33)
    bf = torch.bfloat16
    x = torch.tensor(P["x"]).to(bf).requires_grad_(True)
    fs = P["shared"][0].shape[0]
    # the up and gate projections as one product over [W_up; W_gate] (one input-grad product)
    Wcat = torch.tensor(np.concatenate([P["shared"][1], P["shared"][0]])).to(bf).requires_grad_(True)
    Wd = torch.tensor(P["shared"][2]).to(bf).requires_grad_(True)
    Hs = x @ Wcat.T
    u, g = Hs[:, :fs], Hs[:, fs:]
    a = (torch.nn.functional.silu(g.float()) * u.float()).to(bf)
    y = a @ Wd.T
    (y.float() * torch.tensor(P["dy"], dtype=torch.float32)).sum().backward()
    Wu, Wg = types.SimpleNamespace(grad=Wcat.grad[:fs]), types.SimpleNamespace(grad=Wcat.grad[fs:])
    for store in ("bf16", None):
        oy, cache = O.shared_expert_forward(P["x"], *P["shared"], store=store)
        odx, odWg, odWu, odWd = O.shared_expert_backward(P["dy"], cache, *P["shared"], store=store)
        if store == "bf16":
            fr = {n: np.mean(o == _f64(t)) for n, o, t in (("y", oy, y), ("Wg", odWg, Wg.grad),
                                                            ("Wu", odWu, Wu.grad), ("Wd", odWd, Wd.grad))}
            fr["x"] = np.mean(O.bf16_round(odx) == _f64(x.grad))
            assert min(fr.values()) >= 0.99, fr
            eb = _rel_fro(O.bf16_round(odx), _f64(x.grad))
        else:
            assert np.mean(oy == _f64(y)) < 0.5
            assert _rel_fro(O.bf16_round(odx), _f64(x.grad)) > 4 * eb


@pytest.mark.parametrize("store,gate_scale_on", [(None, "Y"), (None, "A"), ("bf16", "Y"), ("bf16", "A")])
def test_torch_layer_restatement_equals_numpy_oracle(store, gate_scale_on):
    """oracle/torch_layer.py (float64 torch ops, used on the device at full sizes) gives
    the numpy oracle's results: bit for bit under the bf16 storage model (both round
    float64 values at the same points), to float64 accuracy in exact mode."""
    from oracle.torch_layer import TorchLayerRef

    P = _bf16_inputs(34, T=80, E=7)
    orc = O.MoELayerOracle(P["Wg"], P["bias"], P["W1"], P["W2"], P["k"], shared=P["shared"],
                           round_probs_bf16=True, store=store, gate_scale_on=gate_scale_on)
    out, idx, w = orc.forward(P["x"], logits=P["logits"])
    g = orc.backward(P["dy"])
    t = lambda a: torch.tensor(a, dtype=torch.float64)  # noqa: E731
    ref = TorchLayerRef(t(P["Wg"]), t(P["W1"]), t(P["W2"]), P["k"], shared=tuple(t(s) for s in P["shared"]),
                        store=store, gate_scale_on=gate_scale_on)
    tout = ref.forward(t(P["x"]), torch.tensor(idx), torch.tensor(w), torch.tensor(P["p"]))
    tg = ref.backward(t(P["dy"]), rss=True)
    g_rss = orc.backward(P["dy"], rss=True)["rss"]
    names = ("W1", "W2", "gate_weight", "d_gates", "shared_gate", "shared_up", "shared_down")
    assert sorted(tg["rss"]) == sorted(g_rss) == sorted(names)
    for n in names:
        np.testing.assert_allclose(g_rss[n], _f64(tg["rss"][n]), rtol=1e-10, atol=1e-12, err_msg=n)
    pairs = [("out", out, tout)] + [(n, g[n], tg[n]) for n in ("x", "W1", "W2", "gate_weight", "d_gates",
                                                              "d_logits", "shared_gate", "shared_up",
                                                              "shared_down")]
    for name, a, b in pairs:
        if store == "bf16" and name not in ("d_gates",):
            np.testing.assert_array_equal(a, _f64(b), err_msg=name)
        else:
            np.testing.assert_allclose(a, _f64(b), rtol=1e-10, atol=1e-12, err_msg=name)


def test_bf16_store_is_exact_mode_when_off():
    """store=None reproduces the exact restatement that autograd and finite differences pin."""
    P = _bf16_inputs(35)
    for gso in ("Y", "A"):
        a = O.MoELayerOracle(P["Wg"], P["bias"], P["W1"], P["W2"], P["k"], shared=P["shared"],
                             round_probs_bf16=True, gate_scale_on=gso)
        oa, _, _ = a.forward(P["x"], logits=P["logits"])
        ga = a.backward(P["dy"])
        if gso == "Y":
            ref_out, ref_g = oa, ga
        else:
            np.testing.assert_allclose(oa, ref_out, rtol=1e-12, atol=1e-12)
            for n in ("x", "W1", "W2", "gate_weight", "d_gates"):
                np.testing.assert_allclose(ga[n], ref_g[n], rtol=1e-10, atol=1e-12, err_msg=n)


def test_layer_oracle_compact_expert_stack():
    """A compact stack of the touched experts gives the full stack's results for the
    same tokens (their dW rows included)."""
    P = _bf16_inputs(36, T=20, E=12)
    full = O.MoELayerOracle(P["Wg"], P["bias"], P["W1"], P["W2"], P["k"], shared=P["shared"],
                            round_probs_bf16=True, store="bf16", gate_scale_on="A")
    out, idx, _ = full.forward(P["x"], logits=P["logits"])
    g = full.backward(P["dy"])
    ids = np.unique(idx)
    comp = O.MoELayerOracle(P["Wg"], P["bias"], P["W1"][ids], P["W2"][ids], P["k"], shared=P["shared"],
                            round_probs_bf16=True, store="bf16", gate_scale_on="A", expert_ids=ids)
    out_c, idx_c, _ = comp.forward(P["x"], logits=P["logits"])
    gc = comp.backward(P["dy"])
    np.testing.assert_array_equal(idx_c, idx)
    np.testing.assert_array_equal(out_c, out)
    for n in ("x", "gate_weight", "d_logits", "shared_up"):
        np.testing.assert_array_equal(gc[n], g[n], err_msg=n)
    np.testing.assert_array_equal(gc["W1"], g["W1"][ids])
    np.testing.assert_array_equal(gc["W2"], g["W2"][ids])
    with pytest.raises(ValueError):
        O.MoELayerOracle(P["Wg"], P["bias"], P["W1"][ids[1:]], P["W2"][ids[1:]], P["k"], store="bf16",
                         expert_ids=ids[1:], round_probs_bf16=True).forward(P["x"], logits=P["logits"])


def test_summand_rss_brute_force():
    """rss of every weight grad and of the gates' grad equals the root-sum-square of the
    explicit per-row summands, and bounds the largest of them."""
    P = _bf16_inputs(37, T=12, d=8, E=3, k=2, f=4, fs=4)
    for gso in ("Y", "A"):
        orc = O.MoELayerOracle(P["Wg"], P["bias"], P["W1"], P["W2"], P["k"], shared=P["shared"],
                               round_probs_bf16=True, store="bf16", gate_scale_on=gso)
        orc.forward(P["x"], logits=P["logits"])
        g = orc.backward(P["dy"], rss=True)
        c = orc._cache["mcache"]
        # dW2[e] = sum over e's rows r of G[r]^T A[r] (G: the grad rows W2 sees)
        G = O.group(P["dy"], c["ss"], coeff=c["gates"].reshape(-1) if gso == "Y" else None, fan_out=2)
        if gso == "Y":
            G = O.bf16_round(G)
        for e in range(3):
            rows = np.nonzero(c["se"] == e)[0]
            terms = np.stack([np.outer(G[r], c["A"][r]) for r in rows]) if rows.size else np.zeros((1, 8, 4))
            np.testing.assert_allclose(g["rss"]["W2"][e], np.sqrt((terms ** 2).sum(0)), rtol=1e-12, atol=1e-15)
            assert np.all(np.abs(terms).max(0) <= g["rss"]["W2"][e] * (1 + 1e-12))
        # gate weight grad: sum over tokens of d_logits[t]^T x[t]
        terms = np.einsum("te,td->ted", g["d_logits"], P["x"])
        np.testing.assert_allclose(g["rss"]["gate_weight"], np.sqrt((terms ** 2).sum(0)), rtol=1e-12, atol=1e-15)


# ----------------------------------------------------------------- RMSNorm producer
def test_rmsnorm_closed_forms():
    r = rng(40)
    w = r.standard_normal(16) * 0.1
    # constant rows: y = sign(c) (1 + w) / sqrt(1 + eps / c^2)
    for c in (3.0, -0.25, 1e-3):
        y, rs = O.zc_rmsnorm_rows(np.full((1, 16), c), w, eps=1e-6)
        np.testing.assert_allclose(y[0], np.sign(c) * (1 + w) / np.sqrt(1 + 1e-6 / c ** 2), rtol=1e-13)
        np.testing.assert_allclose(rs[0], 1 / np.sqrt(c * c + 1e-6), rtol=1e-13)
    # scale invariance at eps = 0, and w = 0 gives unit-RMS rows
    X = r.standard_normal((5, 16))
    y1, _ = O.zc_rmsnorm_rows(X, w, eps=0.0)
    y2, _ = O.zc_rmsnorm_rows(X * 37.5, w, eps=0.0)
    np.testing.assert_allclose(y1, y2, rtol=1e-13)
    y0, _ = O.zc_rmsnorm_rows(X, np.zeros(16), eps=0.0)
    np.testing.assert_allclose(np.sqrt((y0 ** 2).mean(axis=1)), 1.0, rtol=1e-13)
    # the gather: normalise every row, then index
    rows = np.array([4, 0, 2])
    yg, rg = O.zc_rmsnorm_rows(X, w, rows=rows)
    ya, ra = O.zc_rmsnorm_rows(X, w)
    np.testing.assert_array_equal(yg, ya[rows])
    np.testing.assert_array_equal(rg, ra[rows])


def test_rmsnorm_backward_vs_torch_autograd_and_fd():
    r = rng(41)
    N, d = 7, 12
    X = r.standard_normal((N, d))
    w = r.standard_normal(d) * 0.2
    rows = np.array([6, 1, 3, 2])
    dy = r.standard_normal((rows.size, d))
    y, rstd = O.zc_rmsnorm_rows(X, w, eps=1e-6, rows=rows)
    dX, dw = O.zc_rmsnorm_rows_backward(dy, X, w, rstd, rows=rows)
    # torch autograd of the reference expression (zRMSNorm.py:10-17), float64
    tx = torch.tensor(X, requires_grad=True)
    tw = torch.tensor(w, requires_grad=True)
    h = tx[torch.tensor(rows)]
    ty = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6) * (1.0 + tw)
    np.testing.assert_allclose(y, ty.detach().numpy(), rtol=1e-13, atol=1e-14)
    (ty * torch.tensor(dy)).sum().backward()
    np.testing.assert_allclose(dX, tx.grad.numpy(), rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(dw, tw.grad.numpy(), rtol=1e-12, atol=1e-13)
    assert not dX[[0, 4, 5]].any()  # rows outside the gather get no gradient
    # central finite differences of sum(y * dy)
    eps = 1e-6
    for (a, q), an in (((X, (1, 5)), dX[1, 5]), ((w, (3,)), dw[3])):
        old = a[q]
        a[q] = old + eps
        lp = float((O.zc_rmsnorm_rows(X, w, rows=rows)[0] * dy).sum())
        a[q] = old - eps
        lm = float((O.zc_rmsnorm_rows(X, w, rows=rows)[0] * dy).sum())
        a[q] = old
        assert abs((lp - lm) / (2 * eps) - an) < 1e-7


@pytest.mark.parametrize("shared", [False, True])
def test_torch_eager_forward_equals_numpy_oracle(shared):
    """oracle/torch_eager.py (the C1 CPU baseline: the reference forward as eager torch)
    computes the numpy oracle's forward: the same routing, and on float64 inputs the
    same outputs up to the oracle's float32 routing probabilities (it rounds the
    logits and p to float32, as the layer stores them: relative 1e-6); on float32
    inputs, float32 accuracy norm-wise. Top-k slot order is unspecified in the
    reference (topk(sorted=False)), so slots are compared as per-token sets."""
    from oracle.torch_eager import c1_inputs, moe_forward

    x, Wg, bias, W1, W2 = c1_inputs(T=96, d=64, E=6, f=40, seed=3)
    bias = torch.randn(6, generator=torch.Generator().manual_seed(4)) * 0.1
    sh = tuple(torch.randn(s, generator=torch.Generator().manual_seed(5)) * 0.125
               for s in ((24, 64), (24, 64), (64, 24))) if shared else None
    orc = O.MoELayerOracle(_f64(Wg), bias.numpy().astype(np.float32), _f64(W1), _f64(W2), 3,
                           shared=tuple(_f64(s) for s in sh) if shared else None)
    rout, ridx, rw = orc.forward(_f64(x))
    d = lambda t: t.to(torch.float64)  # noqa: E731
    out, idx, w = moe_forward(d(x), d(Wg), d(bias), d(W1), d(W2), 3, shared=tuple(map(d, sh)) if shared else None)
    np.testing.assert_array_equal(np.sort(idx.numpy(), axis=1), np.sort(ridx, axis=1))
    order = np.argsort(idx.numpy(), axis=1)
    rorder = np.argsort(ridx, axis=1)
    np.testing.assert_allclose(np.take_along_axis(w.numpy(), order, 1), np.take_along_axis(rw, rorder, 1),
                               rtol=1e-6, atol=0)
    np.testing.assert_allclose(out.numpy(), rout, rtol=1e-6, atol=1e-7)
    out32, _, _ = moe_forward(x, Wg, bias, W1, W2, 3, shared=sh)
    assert np.linalg.norm(out32.double().numpy() - rout) <= 1e-5 * np.linalg.norm(rout)


@pytest.mark.parametrize("shared", [False, True])
def test_torch_eager_step_equals_numpy_oracle_backward(shared):
    """oracle/torch_eager.py's moe_step (the C3 CPU baseline: the reference layer as eager
    torch under autograd) gives the numpy oracle's backward: dx, the gate weight's grad
    (through the gathered, normalised probabilities), dW1, dW2 and the shared expert's
    grads, in float64 up to the oracle's float32 routing probabilities (relative 1e-6)."""
    from oracle.torch_eager import moe_step

    g = torch.Generator().manual_seed(11)
    T, d, E, k, f = 80, 48, 7, 3, 24
    x = torch.randn(T, d, generator=g, dtype=torch.float64)
    Wg = torch.randn(E, d, generator=g, dtype=torch.float64) * 0.1
    bias = (torch.randn(E, generator=g) * 0.1).to(torch.float32)
    W1 = torch.randn(E, 2 * f, d, generator=g, dtype=torch.float64) * d ** -0.5
    W2 = torch.randn(E, d, f, generator=g, dtype=torch.float64) * f ** -0.5
    sh = tuple(torch.randn(s, generator=g, dtype=torch.float64) * 0.15 for s in ((16, d), (16, d), (d, 16))) \
        if shared else None
    dout = torch.randn(T, d, generator=g, dtype=torch.float64)
    out, grads = moe_step(x, Wg, bias.double(), W1, W2, k, dout, shared=sh)
    orc = O.MoELayerOracle(Wg.numpy(), bias.numpy(), W1.numpy(), W2.numpy(), k,
                           shared=tuple(t.numpy() for t in sh) if shared else None)
    rout, _, _ = orc.forward(x.numpy())
    ref = orc.backward(dout.numpy())
    np.testing.assert_allclose(out.numpy(), rout, rtol=1e-6, atol=1e-7)
    keys = ["x", "gate_weight", "W1", "W2"] + (["shared_gate", "shared_up", "shared_down"] if shared else [])
    assert sorted(grads) == sorted(keys)
    for n in keys:
        a, b = grads[n].numpy(), ref[n]
        assert np.linalg.norm(a - b) <= 1e-6 * np.linalg.norm(b), n
