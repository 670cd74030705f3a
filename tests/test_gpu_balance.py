"""GPU checks of the reference GLUMLP call (no residual) and of the trainer-side
load-balancing helpers: the aux-loss-free bias update (main.py:161-175) and the
MoE load metrics (utils/trainutils.py:110-142), against the oracle."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle as O
from helpers import TOL, assert_close, gen, np64, random_topk

pytestmark = pytest.mark.gpu


def test_glumlp_reference_call_forward_backward(hip_device):
    """GLUMLP.forward(x, expert_p, expert_idxs) exactly as the reference calls it (mlp.py:74),
    forward and backward, bf16, against the float64 oracle."""
    from scattermoe.mlp import GLUMLP

    T, d, E, k, f = 256, 128, 8, 2, 64
    g = gen(4)
    x = torch.randn(T, d, generator=g)
    W1 = torch.randn(E, 2 * f, d, generator=g) * d ** -0.5
    W2 = torch.randn(E, d, f, generator=g) * d ** -0.5
    idx = random_topk(T, E, k, seed=4)
    p = torch.rand(T, k, generator=g)
    p = p / p.sum(1, keepdim=True)
    dy = torch.randn(T, d, generator=g)

    mlp = GLUMLP(d, f, E, k).to(hip_device).to(torch.bfloat16)
    with torch.no_grad():
        mlp.experts.weight.copy_(W1)
        mlp.output_experts.weight.copy_(W2)
    xd = x.to(torch.bfloat16).to(hip_device).requires_grad_(True)
    pd = p.to(hip_device).requires_grad_(True)
    y = mlp(xd, pd, idx.to(hip_device))
    y.backward(dy.to(torch.bfloat16).to(hip_device))

    xr = np64(x.to(torch.bfloat16))
    W1r, W2r = np64(W1.to(torch.bfloat16)), np64(W2.to(torch.bfloat16))
    # bf16 storage model of this path (routing weights on the W2 outputs)
    ry, cache = O.glu_mlp_forward(xr, np64(p), idx.numpy(), W1r, W2r, store="bf16", gate_scale_on="Y")
    rdx, rdW1, rdW2, rdg, rss = O.glu_mlp_backward(np64(dy.to(torch.bfloat16)), cache, rss=True)
    tol = TOL[torch.bfloat16]
    assert_close(np64(y), ry, **tol, what="y")
    assert_close(np64(xd.grad), rdx, **tol, what="dx")
    assert_close(np64(pd.grad), rdg, **tol, what="d expert_p", rss=rss["d_gates"])
    assert_close(np64(mlp.experts.weight.grad), rdW1, **tol, what="dW1", rss=rss["W1"])
    assert_close(np64(mlp.output_experts.weight.grad), rdW2, **tol, what="dW2", rss=rss["W2"])
    # the sort's offsets of this forward are kept on the module
    counts = np.bincount(idx.numpy().reshape(-1), minlength=E)
    np.testing.assert_array_equal(mlp.last_expert_offsets.cpu().numpy(), np.cumsum(counts))


def _model_with_gates(E, n_layers, dev):
    layers = []
    for i in range(n_layers):
        gate = SimpleNamespace(n_routed_experts=E,
                               expert_biases=(torch.arange(E, dtype=torch.float32) * 1e-3 * (i + 1)).to(dev))
        layers.append(SimpleNamespace(mlp=SimpleNamespace(gate=gate)))
    return SimpleNamespace(layers=layers)


@pytest.mark.parametrize("masked", [False, True])
def test_aux_loss_free_update_matches_reference_rule(hip_device, masked):
    from zmoe.balance import auxillary_loss_free_update

    B, S, E, k = 4, 50, 16, 4
    model = _model_with_gates(E, 3, hip_device)
    b0 = [l.mlp.gate.expert_biases.cpu().numpy().copy() for l in model.layers]
    all_idx = [random_topk(B * S, E, k, seed=10 + i, skew=1.0 * i).view(B, S, k) for i in range(3)]
    mask = (torch.rand(B, S, generator=gen(3)) > 0.3).long() if masked else None
    auxillary_loss_free_update(model, [t.to(hip_device) for t in all_idx], 1e-3,
                               attention_mask=mask.to(hip_device) if masked else None)
    for i, layer in enumerate(model.layers):
        idx = all_idx[i][mask.bool()] if masked else all_idx[i]
        ref = O.bias_update(b0[i], idx.numpy(), E, 1e-3)
        np.testing.assert_array_equal(layer.mlp.gate.expert_biases.cpu().numpy(), ref)


def test_log_moe_metrics_matches_reference_formulas(hip_device):
    from zmoe.balance import log_moe_metrics

    B, S, E, k = 2, 64, 32, 4
    gates = [(1, SimpleNamespace(n_routed_experts=E)), (3, SimpleNamespace(n_routed_experts=E))]
    all_idx = [random_topk(B * S, E, k, seed=20 + i, skew=2.0).view(B, S, k) for i in range(2)]
    mask = (torch.rand(B, S, generator=gen(5)) > 0.2).long()
    m = log_moe_metrics(gates, [t.to(hip_device) for t in all_idx], step=7, attention_mask=mask.to(hip_device))
    for (layer_idx, _), t in zip(gates, all_idx):
        ref = O.moe_load_metrics(t[mask.bool()].numpy(), E)
        for name, v in ref.items():
            got = m[f"experts/layer_{layer_idx}_{name}"]
            assert abs(got - v) <= 1e-5 * max(1.0, abs(v)), (layer_idx, name, got, v)


def test_bias_update_from_layer_offsets_equals_masked_update(hip_device):
    """After an unpadded forward, the sort's offsets give the reference's masked update."""
    from modeling.model_config import ModelConfig
    from modeling.moe_layer import MoELayer
    from zmoe.balance import auxillary_loss_free_update, update_biases_from_layers

    torch.manual_seed(0)
    cfg = ModelConfig(hidden_size=128, intermediate_size=64, n_experts=18, n_shared_experts=2, n_experts_per_token=4)
    layer = MoELayer(cfg).to(hip_device)
    B, S = 3, 64
    mask = (torch.rand(B, S, generator=gen(6)) > 0.25).to(hip_device)
    valid = mask.view(-1).nonzero().view(-1)
    with torch.no_grad():
        _, topk_idx = layer(torch.randn(B, S, 128, device=hip_device), unpad_indices=valid)
    b0 = layer.gate.expert_biases.clone()
    update_biases_from_layers([layer], 1e-3)
    fast = layer.gate.expert_biases.clone()
    layer.gate.expert_biases.copy_(b0)
    auxillary_loss_free_update(SimpleNamespace(layers=[SimpleNamespace(mlp=layer)]), [topk_idx], 1e-3,
                               attention_mask=mask.long())
    assert torch.equal(fast, layer.gate.expert_biases)
    assert not torch.equal(fast, b0)
