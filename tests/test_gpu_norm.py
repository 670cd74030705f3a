"""GPU parity of the RMSNorm producer fused with the unpad gather (zmoe_rmsnorm_rows and
its backward; modeling/zRMSNorm.py:10-17 then modeling/moe_layer.py:39-42) against the
oracle, and of MoELayer.forward(..., norm=...) against normalising first and then
calling the layer, and against the oracle end to end."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from helpers import TOL, assert_close, assert_close_fro, gen, np64

pytestmark = pytest.mark.gpu

# (N rows of hidden, d, rows to gather: None = all, "perm" = a shuffled subset)
SHAPES = [(37, 256, None), (300, 1024, "perm"), (33, 2048, "perm"), (9, 7168, "perm"), (5, 64, None),
          (70, 200, "perm"), (2048, 512, "perm")]


def _inputs(N, d, rows, dtype, w_dtype, seed):
    g = gen(seed)
    X = (torch.randn(N, d, generator=g) * 1.7).to(dtype)
    w = (torch.randn(d, generator=g) * 0.3).to(w_dtype)
    r = None
    if rows == "perm":
        r = torch.randperm(N, generator=g)[: max(1, (3 * N) // 4)]
    return X, w, r


@pytest.mark.parametrize("dtype,w_dtype", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                           (torch.float32, torch.float32)])
@pytest.mark.parametrize("N,d,rows", SHAPES)
def test_rmsnorm_rows_forward_backward(hip_device, dtype, w_dtype, N, d, rows):
    from zmoe import ops

    X, w, r = _inputs(N, d, rows, dtype, w_dtype, seed=N + d)
    rd = None if r is None else r.to(hip_device)
    Y, rstd = ops.rmsnorm_rows(X.to(hip_device), w.to(hip_device), 1e-6, rd)
    ry, rr = O.zc_rmsnorm_rows(np64(X), np64(w), 1e-6, None if r is None else r.numpy())
    tol = TOL[dtype]
    assert Y.dtype == dtype
    assert_close(np64(Y), ry, **tol, what="y")
    assert_close(rstd.cpu().numpy(), rr, rtol=1e-6, atol=0, what="rstd")
    n = ry.shape[0]
    dY = torch.randn(n, d, generator=gen(N * 7 + d)).to(dtype)
    dX, dw = ops.rmsnorm_rows_backward(dY.to(hip_device), X.to(hip_device), rd, rstd, w.to(hip_device))
    rdX, rdw = O.zc_rmsnorm_rows_backward(np64(dY), np64(X), np64(w), rr, None if r is None else r.numpy())
    assert dX.shape == X.shape and dw.dtype == w_dtype
    assert_close(np64(dX), rdX, **tol, what="dX")
    if r is not None:
        outside = np.setdiff1d(np.arange(N), r.numpy())
        assert not dX[torch.from_numpy(outside).to(hip_device)].any(), "rows outside the gather get zero grad"
    if w_dtype == torch.float32 and n >= 256:  # fp32 sums over hundreds of rows: norm-wise (helpers.TOL)
        assert_close_fro(np64(dw), rdw, what="dw")
    else:
        assert_close(np64(dw), rdw, **TOL[w_dtype], what="dw")


def test_rmsnorm_rows_out_of_range_and_empty(hip_device):
    from zmoe import ops

    X = torch.randn(6, 128, device=hip_device).to(torch.bfloat16)
    w = torch.zeros(128, device=hip_device)
    Y, rstd = ops.rmsnorm_rows(X, w, 1e-6, torch.tensor([2, 9, 0], device=hip_device))
    assert not Y[1].any() and float(rstd[1]) == 0.0  # a row outside [0, 6): zero output
    ref, _ = O.zc_rmsnorm_rows(np64(X), np.zeros(128), 1e-6, np.array([2, 0]))
    assert_close(np64(Y[[0, 2]]), ref, **TOL[torch.bfloat16], what="valid rows")
    Y0, r0 = ops.rmsnorm_rows(X, w, 1e-6, torch.empty(0, dtype=torch.int64, device=hip_device))
    assert Y0.shape == (0, 128) and r0.shape == (0,)


def test_zero_centered_rmsnorm_module(hip_device):
    """The module keeps the reference's contract: parameter ``weight`` (zeros), eps 1e-6,
    input dtype in and out, gain 1 + weight."""
    from modeling.zRMSNorm import ZeroCenteredRMSNorm

    m = ZeroCenteredRMSNorm(256)
    assert list(m.state_dict()) == ["weight"] and m.eps == 1e-6 and not m.weight.any()
    m = m.to(hip_device)
    with torch.no_grad():
        m.weight.copy_(torch.randn(256) * 0.1)
    x = torch.randn(2, 5, 256, device=hip_device).to(torch.bfloat16).requires_grad_(True)
    y = m(x)
    assert y.shape == x.shape and y.dtype == torch.bfloat16
    ry, rr = O.zc_rmsnorm_rows(np64(x.view(10, 256)), np64(m.weight), 1e-6)
    assert_close(np64(y.view(10, 256)), ry, **TOL[torch.bfloat16], what="module y")
    dy = torch.randn(2, 5, 256, device=hip_device).to(torch.bfloat16)
    y.backward(dy)
    rdx, rdw = O.zc_rmsnorm_rows_backward(np64(dy.view(10, 256)), np64(x.view(10, 256)), np64(m.weight), rr)
    assert_close(np64(x.grad.view(10, 256)), rdx, **TOL[torch.bfloat16], what="module dx")
    assert_close(np64(m.weight.grad), rdw, **TOL[torch.float32], what="module dw (fp32 weight, 10 rows)")


def _layer(dev):
    from modeling.model_config import ModelConfig
    from modeling.moe_layer import MoELayer
    from modeling.zRMSNorm import ZeroCenteredRMSNorm

    torch.manual_seed(5)
    cfg = ModelConfig(hidden_size=256, intermediate_size=128, n_experts=18, n_shared_experts=2, n_experts_per_token=4)
    layer = MoELayer(cfg).to(dev).to(torch.bfloat16)
    layer.gate.expert_biases.data = (0.1 * torch.randn(16)).to(dev)
    norm = ZeroCenteredRMSNorm(256).to(dev)
    with torch.no_grad():
        norm.weight.copy_(torch.randn(256) * 0.2)
    return layer, norm


@pytest.mark.parametrize("unpad", [False, True])
def test_layer_with_norm_matches_norm_then_layer(hip_device, unpad):
    """MoELayer(h, unpad, norm=n) equals MoELayer(n(h), unpad): the same output and routing
    and the same hidden-state grad bit for bit (the same per-row arithmetic), the norm
    weight's grad up to fp32 summation order, the layer's grads bit for bit."""
    layer, norm = _layer(hip_device)
    B, S = 2, 300
    valid = torch.tensor([i for i in range(B * S) if (i % 9) != 4], device=hip_device) if unpad else None
    h = torch.randn(B, S, 256, device=hip_device).to(torch.bfloat16)
    dout = torch.randn(B, S, 256, device=hip_device).to(torch.bfloat16)
    runs = []
    for fused in (True, False):
        layer.zero_grad(set_to_none=True)
        norm.zero_grad(set_to_none=True)
        x = h.clone().requires_grad_(True)
        out, idx = layer(x, unpad_indices=valid, norm=norm) if fused else layer(norm(x), unpad_indices=valid)
        out.backward(dout)
        runs.append((out, idx, x.grad, norm.weight.grad, {n: p.grad for n, p in layer.named_parameters()}))
    (o1, i1, g1, w1, p1), (o0, i0, g0, w0, p0) = runs
    assert torch.equal(o1, o0) and torch.equal(i1, i0)
    assert torch.equal(g1, g0)
    for n in p0:
        assert torch.equal(p1[n], p0[n]), n
    assert_close(np64(w1), np64(w0), rtol=1e-5, atol=1e-5, what="norm weight grad")


def test_layer_with_norm_vs_oracle(hip_device):
    """End to end: hidden -> norm -> gather -> layer -> out, and the grads of hidden and of
    the norm weight, against the oracle (bf16 storage model of the whole-layer path)."""
    layer, norm = _layer(hip_device)
    B, S, d = 2, 200, 256
    valid = torch.tensor([i for i in range(B * S) if (i % 7) != 2], device=hip_device)
    h = (torch.randn(B, S, d, device=hip_device) * 2.0).to(torch.bfloat16).requires_grad_(True)
    dout = torch.randn(B, S, d, device=hip_device).to(torch.bfloat16)
    out, idx = layer(h, unpad_indices=valid, norm=norm)
    out.backward(dout)
    hf, vn = np64(h.view(B * S, d)), valid.cpu().numpy()
    x, rstd = O.zc_rmsnorm_rows(hf, np64(norm.weight), norm.eps, vn)
    x = O.bf16_round(x).astype(np.float64)  # the layer's input, stored in bf16
    with torch.no_grad():
        xd = torch.from_numpy(x).to(hip_device).to(torch.bfloat16)
        logits = F.linear(xd, layer.gate.weight).float().cpu().numpy()
    se = layer.shared_experts
    orc = O.MoELayerOracle(np64(layer.gate.weight), layer.gate.expert_biases.cpu().numpy(),
                           np64(layer.routed_experts.experts.weight), np64(layer.routed_experts.output_experts.weight),
                           4, shared=(np64(se.gate_proj.weight), np64(se.up_proj.weight), np64(se.down_proj.weight)),
                           round_probs_bf16=True, store="bf16", gate_scale_on="A")
    rout, ridx, _ = orc.forward(x, logits=logits)
    np.testing.assert_array_equal(idx.view(B * S, 4).cpu().numpy()[vn], ridx)
    tol = TOL[torch.bfloat16]
    assert_close(np64(out.view(B * S, d))[vn], rout, **tol, what="out")
    g = orc.backward(np64(dout.view(B * S, d))[vn])
    dx_layer = O.bf16_round(g["x"]).astype(np.float64)  # the layer's input grad, stored in bf16
    rdh, rdw = O.zc_rmsnorm_rows_backward(dx_layer, hf, np64(norm.weight), rstd, vn)
    assert_close(np64(h.grad.view(B * S, d)), rdh, **tol, what="d hidden")
    rss = np.sqrt(((dx_layer * hf[vn] * rstd[:, None]) ** 2).sum(axis=0))
    # fp32 norm weight, a sum over the stored bf16 layer input grads: + 2^-7 rss (helpers.TOL)
    assert_close(np64(norm.weight.grad), rdw, **TOL[torch.bfloat16], what="d norm.weight", rss=rss)
