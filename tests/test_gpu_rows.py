"""GPU parity: dispatch gather (group), combine, combine backward, k-sum,
rowwise_sum_product and SwiGLU against the oracle."""

import numpy as np
import pytest
import torch

import oracle as O
from helpers import TOL, assert_close, gen, np64, random_topk

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("T,d,k,coeff", [(300, 256, 2, False), (300, 2048, 8, True), (77, 64, 1, True),
                                         (1024, 7168, 8, True)])
def test_group(hip_device, dtype, T, d, k, coeff):
    from zmoe import ops

    g = gen(T + d)
    A = torch.randn(T, d, generator=g).to(dtype)
    idx = torch.randperm(T * k, generator=g)
    c = torch.randn(T * k, generator=g) if coeff else None
    Y = ops.group(A.to(hip_device), idx.to(hip_device), coeff=None if c is None else c.to(hip_device), fan_out=k)
    ref = O.group(np64(A), idx.numpy(), coeff=None if c is None else c.numpy(), fan_out=k)
    if coeff:
        # one multiply, then rounding to the storage type
        assert_close(np64(Y), ref, rtol=2 ** -7 if dtype == torch.bfloat16 else 1e-6, atol=0, what="group")
    else:
        np.testing.assert_array_equal(np64(Y), ref)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("T,d,k", [(513, 256, 2), (300, 2048, 8), (64, 7168, 8), (5, 96, 3)])
def test_combine_and_backward(hip_device, dtype, T, d, k):
    from zmoe import ops

    g = gen(T * d + k)
    Y = torch.randn(T * k, d, generator=g).to(dtype)
    gates = torch.rand(T, k, generator=g)
    add = torch.randn(T, d, generator=g).to(dtype)
    dout = torch.randn(T, d, generator=g).to(dtype)
    idx = random_topk(T, 4 * k, k, seed=1)
    _, ss, _, inv = ops.flatten_sort_count(idx.to(hip_device), 4 * k)
    out = ops.combine(Y.to(hip_device), gates.to(hip_device), k, addend=add.to(hip_device))
    ref = np.einsum("tj,tjd->td", gates.double().numpy(), np64(Y).reshape(T, k, d)) + np64(add)
    tol = TOL[dtype]
    assert_close(np64(out), ref, **tol, what="combine")

    d_gates, grouped = ops.combine_backward(Y.to(hip_device), dout.to(hip_device), gates.to(hip_device), inv)
    ref_dg = O.rowwise_sum_product(np64(Y).reshape(T, k, d), np64(dout))
    assert_close(d_gates.cpu().numpy(), ref_dg, rtol=1e-5, atol=1e-4, what="d_gates")
    ref_grouped = O.group(np64(dout), ss.cpu().numpy(), coeff=gates.double().numpy().reshape(-1), fan_out=k)
    assert_close(np64(grouped), ref_grouped, **tol, what="grouped_grad_out")
    # unit gates (gates = None): the plain k-sum plus the addend
    out1 = ops.combine(Y.to(hip_device), None, k, addend=add.to(hip_device))
    ref1 = np64(Y).reshape(T, k, d).sum(1) + np64(add)
    assert_close(np64(out1), ref1, **tol, what="combine without gates")
    # without Y: the same grouped rows, no gate grads
    no_dg, grouped2 = ops.combine_backward(None, dout.to(hip_device), gates.to(hip_device), inv)
    assert no_dg is None and torch.equal(grouped2, grouped)


@pytest.mark.parametrize("dtype", DTYPES)
def test_sum_k_and_rowwise(hip_device, dtype):
    from zmoe import ops

    T, d, k = 257, 1024, 8
    g = gen(9)
    Xe = torch.randn(T * k, d, generator=g).to(dtype)
    a0 = torch.randn(T, d, generator=g).to(dtype)
    a1 = torch.randn(T, d, generator=g).to(dtype)
    out = ops.sum_k(Xe.to(hip_device), k, a0.to(hip_device), a1.to(hip_device))
    ref = np64(Xe).reshape(T, k, d).sum(1) + np64(a0) + np64(a1)
    assert_close(np64(out), ref, **TOL[dtype], what="sum_k")
    A = torch.randn(T, k, 100, generator=g).to(dtype)
    B = torch.randn(T, 100, generator=g)
    rs = ops.rowwise_sum_product(A.to(hip_device), B.to(hip_device), dtype=torch.float32)
    assert_close(rs.cpu().numpy(), O.rowwise_sum_product(np64(A), np64(B)), rtol=1e-5, atol=1e-5, what="rowwise")


@pytest.mark.parametrize("k", [8, 3])
def test_sum_k_fp32_out_of_bf16_rows(hip_device, k):
    """bf16 rows summed into fp32 output (the input grad of an fp32 residual stream): the fp32
    sum unrounded, within fp32 rounding of the float64 sum; its bf16 rounding is the bf16-output
    launch's result bit for bit."""
    from zmoe import ops

    T, d = 301, 768
    g = gen(19 + k)
    Xe = torch.randn(T * k, d, generator=g).to(torch.bfloat16).to(hip_device)
    a0 = torch.randn(T, d, generator=g).to(torch.bfloat16).to(hip_device)
    out = ops.sum_k(Xe, k, a0, out_dtype=torch.float32)
    assert out.dtype == torch.float32
    ref = np64(Xe).reshape(T, k, d).sum(1) + np64(a0)
    assert_close(np64(out), ref, rtol=1e-6, atol=1e-6, what="sum_k fp32 out")
    assert torch.equal(out.to(torch.bfloat16), ops.sum_k(Xe, k, a0))


@pytest.mark.parametrize("n", [0, 5, 8, 4099, 1 << 20])
def test_cast_bf16_matches_torch(hip_device, n):
    """The compute-copy cast equals torch's fp32 -> bf16 conversion bit for bit (round to
    nearest even, ties, subnormals, infinities; NaN stays NaN), tails of n % 8 included."""
    from zmoe import ops

    g = gen(n + 1)
    x = torch.randn(n, generator=g) * torch.exp2(torch.randint(-140, 120, (n,), generator=g).float())
    if n >= 8:
        # exact ties at bf16 rounding midpoints (both parities), the largest finite values, specials
        x[:8] = torch.tensor([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8), 3.3895e38, -3.3895e38,
                              float("inf"), float("-inf"), float("nan")])
    xd = x.to(hip_device)
    got = ops.cast_bf16(xd)
    ref = xd.to(torch.bfloat16)
    assert got.shape == ref.shape and got.dtype == torch.bfloat16
    gi, ri = got.view(torch.int16), ref.view(torch.int16)
    nan = torch.isnan(ref)
    assert torch.equal(torch.isnan(got), nan)
    assert torch.equal(gi[~nan], ri[~nan])


@pytest.mark.parametrize("dtype", DTYPES)
def test_swiglu(hip_device, dtype):
    from zmoe import ops

    g = gen(10)
    H = torch.randn(333, 2 * 768, generator=g).to(dtype)
    dA = torch.randn(333, 768, generator=g).to(dtype)
    A = ops.swiglu(H.to(hip_device))
    assert_close(np64(A), O.swiglu(np64(H)), **TOL[dtype], what="swiglu")
    dH = ops.swiglu_backward(dA.to(hip_device), H.to(hip_device))
    assert_close(np64(dH), O.swiglu_backward(np64(dA), np64(H)), **TOL[dtype], what="swiglu_backward")
    # into the leading columns of a wider buffer: the rest of each row is left alone
    buf = torch.full((333, 2 * 768 + 24), 7.0, dtype=dtype, device=hip_device)
    ops.swiglu_backward(dA.to(hip_device), H.to(hip_device), out=buf[:, :2 * 768])
    assert torch.equal(buf[:, :2 * 768], dH) and bool((buf[:, 2 * 768:] == 7.0).all())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("R,f", [(333, 768), (64, 136), (1, 8), (5, 264)])
def test_swiglu_backward_gates(hip_device, dtype, R, f):
    """dH = swiglu_backward(row_scale * dA, H) and d_gates[slot] = <dA, silu(g) * h> per row."""
    from zmoe import ops

    g = gen(R + f)
    H = torch.randn(R, 2 * f, generator=g).to(dtype)
    dA = torch.randn(R, f, generator=g).to(dtype)
    rs = torch.rand(R, generator=g) + 0.05
    slots = torch.from_numpy(np.random.default_rng(R).permutation(R))
    dH, dg = ops.swiglu_backward_gates(dA.to(hip_device), H.to(hip_device), rs.to(hip_device), slots.to(hip_device))
    ref_dH = O.swiglu_backward(rs.double().numpy()[:, None] * np64(dA), np64(H))
    assert_close(np64(dH), ref_dH, **TOL[dtype], what="dH")
    ref_dg = np.empty(R)
    ref_dg[slots.numpy()] = (np64(dA) * O.swiglu(np64(H))).sum(1)
    assert_close(dg.cpu().numpy().astype(np.float64), ref_dg, **TOL[dtype], what="d_gates")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_combine_rows_writes_padded_layout(hip_device, dtype):
    """zmoe_combine_rows / zmoe_combine_backward_rows (the re-pad of moe_layer.py:55-56 folded
    in) against the row-contiguous calls; row numbers outside [0, total) are skipped on write
    and read as zero."""
    from zmoe import ops

    T, k, d, total = 37, 4, 96, 60
    g = gen(12)
    Y = torch.randn(T * k, d, generator=g).to(dtype).to(hip_device)
    w = torch.rand(T, k, generator=g).to(hip_device)
    add = torch.randn(T, d, generator=g).to(dtype).to(hip_device)
    rows = torch.randperm(total, generator=g)[:T].to(hip_device)
    rows[5] = -1        # outside the padded output: not written
    rows[9] = total     # outside: not written
    ref = ops.combine(Y, w, k, addend=add)
    out = ops.combine(Y, w, k, addend=add, out_rows=rows, out_total=total)
    ok = (rows >= 0) & (rows < total)
    assert torch.equal(out[rows[ok]], ref[ok])
    written = torch.zeros(total, dtype=torch.bool, device=hip_device)
    written[rows[ok]] = True
    assert (out[~written] == 0).all()

    dout_pad = torch.randn(total, d, generator=g).to(dtype).to(hip_device)
    _, ss, _, inv = ops.flatten_sort_count(random_topk(T, 8, k, seed=12).to(hip_device), 8)
    dout = torch.zeros(T, d, dtype=dtype, device=hip_device)
    dout[ok] = dout_pad[rows[ok]]
    dg_ref, gr_ref = ops.combine_backward(Y, dout, w, inv)
    dg, gr = ops.combine_backward(Y, dout_pad, w, inv, grad_rows=rows)
    assert torch.equal(dg, dg_ref) and torch.equal(gr, gr_ref)
