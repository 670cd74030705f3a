"""Feature widths that are not whole 16-byte chunks (K, N or d not a multiple of 8 bf16 or 4
fp32 elements), which the reference's masked kernels accept (scattermoe/kernels/ops.py:159-179,
:404-435, :504-519): the op wrappers run them through zero-padded copies, and the modules fall
back from the fused paths to the module composition. Checked against the oracle at the
north-star tolerances."""

import numpy as np
import pytest
import torch

import oracle as O
from helpers import TOL, assert_close, assert_close_fro, gen, np64, random_topk

pytestmark = pytest.mark.gpu

# (K, N): every residue of 8 appears in K or N; fp32 rows need multiples of 4
WIDTHS = [(100, 37), (13, 200), (257, 259), (6, 3), (130, 66), (41, 255), (7, 128), (64, 17)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("K,N", WIDTHS)
@pytest.mark.parametrize("xg,yg", [(False, True), (True, False), (False, False)])
def test_scatter2scatter_any_width(hip_device, dtype, K, N, xg, yg):
    from zmoe import ops

    T, E, k = 300, 8, 2
    idx = random_topk(T, E, k, seed=K + N, skew=0.5)
    se, ss, off, _ = ops.flatten_sort_count(idx.to(hip_device), E)
    g = gen(K * 7 + N)
    X = torch.randn(T * k if xg else T, K, generator=g).to(dtype)
    Wp = (torch.randn(E, N, K, generator=g) / K ** 0.5).to(dtype)
    b = (torch.randn(E, N, generator=g) * 0.3).to(dtype)
    Y = ops.scatter2scatter(X.to(hip_device), Wp.to(hip_device).permute(0, 2, 1), se, ss, 1 if xg else k,
                            b=b.to(hip_device), x_grouped=xg, y_grouped=yg, expert_offsets=off)
    assert Y.shape == (T * k, N)
    ref = O.scatter2scatter(np64(X), np64(Wp).transpose(0, 2, 1), se.cpu().numpy(), ss.cpu().numpy(),
                            1 if xg else k, b=np64(b), x_grouped=xg, y_grouped=yg)
    assert_close(np64(Y), ref, **TOL[dtype], what=f"scatter2scatter K={K} N={N}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("K,N", WIDTHS)
def test_group_bwd_w_any_width(hip_device, dtype, K, N):
    from zmoe import ops

    T, E, k = 300, 8, 3
    idx = random_topk(T, E, k, seed=3 * K + N, skew=1.0)
    se, ss, off, _ = ops.flatten_sort_count(idx.to(hip_device), E)
    g = gen(K + 11 * N)
    DY = torch.randn(T * k, N, generator=g).to(dtype)
    X = torch.randn(T, K, generator=g).to(dtype)
    DWt, Db = ops.group_bwd_w(DY.to(hip_device), X.to(hip_device), off, E, has_bias=True, x_gather=ss, x_div=k)
    assert DWt.shape == (E, N, K) and DWt.is_contiguous() and Db.shape == (E, N)
    ref, rb = O.group_bwd_w(np64(DY), O.group(np64(X), ss.cpu().numpy(), fan_out=k), off.cpu().numpy(), E,
                            has_bias=True)
    if dtype == torch.float32:
        assert_close_fro(np64(DWt), ref.transpose(0, 2, 1), what="group_bwd_w f32")
    else:
        assert_close(np64(DWt), ref.transpose(0, 2, 1), **TOL[dtype], what=f"group_bwd_w K={K} N={N}")
    assert_close(np64(Db), rb, **TOL[dtype], what="bias grad")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("d", [3, 37, 100, 255])
def test_row_passes_any_width(hip_device, dtype, d):
    """group (with coefficients), combine (gates, addend, padded output rows) and the k-sum."""
    from zmoe import ops

    T, k = 211, 4
    g = gen(d)
    A = torch.randn(T, d, generator=g).to(dtype)
    perm = torch.randperm(T * k, generator=g)
    c = torch.rand(T * k, generator=g)
    Y = ops.group(A.to(hip_device), perm.to(hip_device), coeff=c.to(hip_device), fan_out=k)
    assert_close(np64(Y), O.group(np64(A), perm.numpy(), coeff=c.double().numpy(), fan_out=k), **TOL[dtype],
                 what="group")
    Ye = torch.randn(T * k, d, generator=g).to(dtype)
    gates = torch.rand(T, k, generator=g)
    add = torch.randn(T, d, generator=g).to(dtype)
    rows = torch.randperm(T + 50, generator=g)[:T]
    out = ops.combine(Ye.to(hip_device), gates.to(hip_device), k, add.to(hip_device), rows.to(hip_device), T + 50)
    ref = np.zeros((T + 50, d))
    ref[rows.numpy()] = np64(add) + np.einsum("tj,tjd->td", gates.double().numpy(), np64(Ye).reshape(T, k, d))
    assert_close(np64(out), ref, **TOL[dtype], what="combine")
    s = ops.sum_k(Ye.to(hip_device), k, add.to(hip_device))
    assert_close(np64(s), np64(Ye).reshape(T, k, d).sum(1) + np64(add), **TOL[dtype], what="sum_k")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_glumlp_odd_widths(hip_device, dtype):
    """GLUMLP(input_size=100, hidden_size=52): the fused path declines these widths and the
    module composition runs, forward and backward, against the oracle."""
    from scattermoe.mlp import GLUMLP

    torch.manual_seed(5)
    T, d, f, E, k = 400, 100, 52, 8, 2
    mlp = GLUMLP(d, f, E, k).to(hip_device).to(dtype)
    x = torch.randn(T, d, device=hip_device).to(dtype).requires_grad_(True)
    idx = random_topk(T, E, k, seed=9).to(hip_device)
    p = (torch.rand(T, k, generator=gen(4)) + 0.1).to(hip_device)
    y = mlp(x, p, idx)
    dy = torch.randn(T, d, generator=gen(6)).to(dtype).to(hip_device)
    y.backward(dy)
    bf16 = dtype == torch.bfloat16
    ry, cache = O.glu_mlp_forward(np64(x), p.double().cpu().numpy(), idx.cpu().numpy(), np64(mlp.experts.weight),
                                  np64(mlp.output_experts.weight), store="bf16" if bf16 else None)
    rdx, rdW1, rdW2, _, rss = O.glu_mlp_backward(np64(dy), cache, rss=True)
    tol = TOL[dtype]
    assert_close(np64(y), ry, **tol, what="y")
    assert_close(np64(x.grad), rdx, **tol, what="dx")
    if bf16:  # the composition rounds silu(gate) and the product as two bf16 ops: two rss allowances
        assert_close(np64(mlp.experts.weight.grad), rdW1, **tol, what="dW1", rss=2 * rss["W1"])
        assert_close(np64(mlp.output_experts.weight.grad), rdW2, **tol, what="dW2", rss=2 * rss["W2"])
    else:
        assert_close_fro(np64(mlp.experts.weight.grad), rdW1, what="dW1")
        assert_close_fro(np64(mlp.output_experts.weight.grad), rdW2, what="dW2")


def test_moe_layer_odd_hidden_size(hip_device):
    """MoELayer with hidden_size = 100 and intermediate_size = 36 (bf16), forward and backward:
    the whole-layer function declines these widths; the composition's routing is bit-exact
    and its output and grads are within the bf16 bound of the oracle."""
    from modeling.model_config import ModelConfig
    from modeling.moe_layer import MoELayer

    torch.manual_seed(8)
    d, f, E, k = 100, 36, 12, 3
    cfg = ModelConfig(hidden_size=d, intermediate_size=f, n_experts=E + 1, n_shared_experts=1,
                      n_experts_per_token=k)
    layer = MoELayer(cfg).to(hip_device).to(torch.bfloat16)
    layer.gate.expert_biases.data = (0.1 * torch.randn(E)).to(hip_device)
    T = 500
    x = torch.randn(1, T, d, device=hip_device).to(torch.bfloat16).requires_grad_(True)
    out, idx = layer(x)
    dout = torch.randn(1, T, d, device=hip_device).to(torch.bfloat16)
    out.backward(dout)
    se = layer.shared_experts
    with torch.no_grad():
        logits = torch.nn.functional.linear(x.detach().view(T, d), layer.gate.weight).float().cpu().numpy()
    orc = O.MoELayerOracle(np64(layer.gate.weight), layer.gate.expert_biases.cpu().numpy(),
                           np64(layer.routed_experts.experts.weight), np64(layer.routed_experts.output_experts.weight),
                           k, shared=(np64(se.gate_proj.weight), np64(se.up_proj.weight), np64(se.down_proj.weight)),
                           round_probs_bf16=True, store="bf16", gate_scale_on="Y")
    rout, ridx, _ = orc.forward(np64(x.view(T, d)), logits=logits)
    np.testing.assert_array_equal(idx.view(T, k).cpu().numpy(), ridx)
    tol = TOL[torch.bfloat16]
    assert_close(np64(out.view(T, d)), rout, **tol, what="out")
    g = orc.backward(np64(dout.view(T, d)), rss=True)
    assert_close(np64(x.grad.view(T, d)), g["x"], **tol, what="dx")
    keys = {"gate.weight": "gate_weight", "routed_experts.experts.weight": "W1",
            "routed_experts.output_experts.weight": "W2", "shared_experts.gate_proj.weight": "shared_gate",
            "shared_experts.up_proj.weight": "shared_up", "shared_experts.down_proj.weight": "shared_down"}
    for n, p in layer.named_parameters():
        # the composition rounds a few more intermediates than the oracle models (torch's silu
        # and product as separate bf16 ops): two rss allowances, as for the two-path comparison
        assert_close(np64(p.grad), g[keys[n]], **tol, what=n, rss=2 * g["rss"][keys[n]])
