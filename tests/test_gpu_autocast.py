"""The layer in the reference's own training mode: fp32 master weights (main.py:595), bf16
autocast (main.py:746), an fp32 residual stream into the layer and unpad_indices
(transformer_block.py:40-43, moe_layer.py:39-57).

The whole-layer function must run there (not the module composition), computing in bf16
on copies of the weights and writing fp32 weight grads straight from its fp32 accumulators.
Checked against the oracle on the same bf16-rounded operands (store="bf16", the routing
weights applied to A, weight grads left unrounded): routing bit-exact, out, the hidden
states' grad and every parameter grad at the bf16 bound (+ 2^-7 rss for the weight grads'
sums over stored bf16 summands, as in the bf16 tests).
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from helpers import TOL, assert_close, np64

pytestmark = pytest.mark.gpu


def _bf(t: torch.Tensor) -> np.ndarray:
    """The bf16 compute copy of a tensor, as float64."""
    return np64(t.detach().to(torch.bfloat16))


@pytest.mark.parametrize("param_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("with_norm", [False, True])
def test_layer_autocast_fp32_master_weights(hip_device, param_dtype, with_norm, monkeypatch):
    from modeling import moe_layer as ML
    from modeling.model_config import ModelConfig
    from modeling.zRMSNorm import ZeroCenteredRMSNorm

    calls = []
    real_apply = ML._FusedMoELayer.apply
    monkeypatch.setattr(ML._FusedMoELayer, "apply", lambda *a: calls.append(1) or real_apply(*a))

    torch.manual_seed(7)
    d, f, E, k, n_shared = 256, 128, 16, 4, 2
    cfg = ModelConfig(hidden_size=d, intermediate_size=f, n_experts=E + n_shared, n_shared_experts=n_shared,
                      n_experts_per_token=k)
    layer = ML.MoELayer(cfg).to(hip_device).to(param_dtype)
    layer.gate.expert_biases.data = (0.1 * torch.randn(E)).to(hip_device)  # the fp32 buffer
    norm = None
    if with_norm:
        norm = ZeroCenteredRMSNorm(d).to(hip_device)
        with torch.no_grad():
            norm.weight.copy_(0.1 * torch.randn(d))
        norm.weight.requires_grad_(False)
    B, S = 2, 300
    valid = torch.tensor([i for i in range(B * S) if (i % 7) != 2], device=hip_device)
    h = torch.randn(B, S, d, device=hip_device).requires_grad_(True)   # fp32 residual stream
    dout = torch.randn(B, S, d, device=hip_device).to(torch.bfloat16)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out, idx = layer(h, unpad_indices=valid, norm=norm)
    assert calls, "the whole-layer function did not run under autocast"
    assert out.dtype == torch.bfloat16
    out.backward(dout)
    for n, p in layer.named_parameters():
        assert p.grad is not None and p.grad.dtype == param_dtype, n
    assert h.grad.dtype == torch.float32

    # the layer's input rows as the function saw them (bf16) and the device's logits
    hv = h.detach().reshape(B * S, d)[valid]
    if with_norm:  # the same norm launch as inside the layer (the norm itself: test_gpu_norm.py)
        from zmoe import ops

        with torch.no_grad():
            xv = ops.rmsnorm_rows(h.detach().reshape(B * S, d), norm.weight, norm.eps, rows=valid)[0]
        xv = xv.to(torch.bfloat16)
    else:
        xv = hv.to(torch.bfloat16)
    se = layer.shared_experts
    with torch.no_grad():
        logits = F.linear(xv, layer.gate.weight.to(torch.bfloat16)).float().cpu().numpy()
    f32 = param_dtype == torch.float32
    orc = O.MoELayerOracle(_bf(layer.gate.weight), layer.gate.expert_biases.cpu().numpy(),
                           _bf(layer.routed_experts.experts.weight), _bf(layer.routed_experts.output_experts.weight),
                           k, shared=(_bf(se.gate_proj.weight), _bf(se.up_proj.weight), _bf(se.down_proj.weight)),
                           round_probs_bf16=True, store="bf16", gate_scale_on="A", f32_weight_grads=f32)
    rout, ridx, _ = orc.forward(np64(xv), logits=logits)
    flat_idx = idx.reshape(B * S, k)
    np.testing.assert_array_equal(flat_idx[valid].cpu().numpy(), ridx)
    pad = torch.ones(B * S, dtype=torch.bool, device=hip_device)
    pad[valid] = False
    assert bool((flat_idx[pad] == 0).all())
    tol = TOL[torch.bfloat16]
    flat_out = out.reshape(B * S, d)
    assert_close(np64(flat_out[valid]), rout, **tol, what="out")
    assert bool((flat_out[pad] == 0).all())
    g = orc.backward(np64(dout.reshape(B * S, d)[valid]), rss=True)
    gh = h.grad.reshape(B * S, d)
    assert bool((gh[pad] == 0).all())
    if not with_norm:  # the hidden states' grad is the layer input's grad on the valid rows
        assert_close(np64(gh[valid]), g["x"], **tol, what="d hidden")
    keys = {"gate.weight": "gate_weight", "routed_experts.experts.weight": "W1",
            "routed_experts.output_experts.weight": "W2", "shared_experts.gate_proj.weight": "shared_gate",
            "shared_experts.up_proj.weight": "shared_up", "shared_experts.down_proj.weight": "shared_down"}
    for n, p in layer.named_parameters():
        assert_close(np64(p.grad), g[keys[n]], **tol, what=n, rss=g["rss"][keys[n]])


def test_layer_autocast_matches_bf16_layer(hip_device):
    """Under autocast with fp32 weights the layer's forward equals the pure-bf16 layer built
    from the rounded weights bit for bit (same kernels on the same bf16 operands); its fp32
    input grad is the same fp32 k-sum unrounded, and its fp32 weight grads round to the bf16
    layer's grads but for rare accumulation flips."""
    from modeling.model_config import ModelConfig
    from modeling.moe_layer import MoELayer

    torch.manual_seed(3)
    d, f, E, k = 256, 128, 16, 4
    cfg = ModelConfig(hidden_size=d, intermediate_size=f, n_experts=E + 1, n_shared_experts=1,
                      n_experts_per_token=k)
    l32 = MoELayer(cfg).to(hip_device)
    l32.gate.expert_biases.data = (0.1 * torch.randn(E)).to(hip_device)
    l16 = MoELayer(cfg).to(hip_device)
    l16.load_state_dict(l32.state_dict())
    l16 = l16.to(torch.bfloat16)
    l16.gate.expert_biases.data = l32.gate.expert_biases.data.clone()
    T = 1000
    h = torch.randn(1, T, d, device=hip_device).to(torch.bfloat16).float()
    dout = torch.randn(1, T, d, device=hip_device).to(torch.bfloat16)
    x32 = h.clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        o32, i32 = l32(x32)
    o32.backward(dout)
    x16 = h.to(torch.bfloat16).requires_grad_(True)
    o16, i16 = l16(x16)
    o16.backward(dout)
    assert torch.equal(i32, i16) and torch.equal(o32, o16)
    assert x32.grad.dtype == torch.float32 and torch.equal(x32.grad.to(torch.bfloat16), x16.grad)
    for (n, p32), (_, p16) in zip(l32.named_parameters(), l16.named_parameters()):
        r = p32.grad.to(torch.bfloat16)
        same = (r == p16.grad).float().mean().item()
        assert same >= 0.99, (n, same)
        assert_close(np64(r), np64(p16.grad), rtol=2 ** -7, atol=1e-6, what=n)
