"""GPU parity of the whole MoE layer (gate -> sort -> GLU experts -> combine,
plus the shared expert) forward and backward against the float64 oracle.

Routing is compared bit-exactly from the logits the device's gate projection
produced (the projection itself is checked with the float tolerance); outputs
and gradients use the north-star tolerances.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from helpers import TOL, assert_close, assert_close_fro, gen, layer_inputs, np64

pytestmark = pytest.mark.gpu


def shared_width(f, n_shared):
    """Width of the layer's shared expert: the reference's ExpertMLP reads a width of
    0 (n_shared_experts = 0) as config.intermediate_size (expert_layer.py:10)."""
    return f * n_shared or f


def build_layer(P, d, E, k, f, n_shared, dtype, dev, fused=True):
    from modeling.model_config import ModelConfig
    from modeling.moe_layer import MoELayer

    cfg = ModelConfig(hidden_size=d, intermediate_size=f, n_experts=E + n_shared, n_shared_experts=n_shared,
                      n_experts_per_token=k)
    layer = MoELayer(cfg)
    layer.routed_experts.fused = fused
    with torch.no_grad():
        layer.gate.weight.copy_(P["Wg"])
        layer.gate.expert_biases.copy_(P["bias"])
        layer.routed_experts.experts.weight.copy_(P["W1"])
        layer.routed_experts.output_experts.weight.copy_(P["W2"])
        layer.shared_experts.gate_proj.weight.copy_(P["shared"][0])
        layer.shared_experts.up_proj.weight.copy_(P["shared"][1])
        layer.shared_experts.down_proj.weight.copy_(P["shared"][2])
    layer = layer.to(dev)
    if dtype != torch.float32:
        layer = layer.to(dtype)
        # .to(dtype) also rounds the fp32 buffer; restore the exact fp32 biases
        layer.gate.expert_biases.data = P["bias"].float().to(dev)
    return layer


def run_and_compare(T, d, E, k, f, n_shared, dtype, dev, fused=True, bias_std=0.1, seed=0):
    fs = shared_width(f, n_shared)
    P = layer_inputs(T, d, E, k, f, fs, seed=seed, dtype=dtype, bias_std=bias_std)
    layer = build_layer(P, d, E, k, f, n_shared, dtype, dev, fused=fused)
    x = P["x"].to(dtype).to(dev).view(1, T, d).requires_grad_(True)
    out, idx = layer(x)
    out.backward(P["dout"].to(dtype).to(dev).view(1, T, d))

    # the gate projection the device computed, re-run with the same call
    with torch.no_grad():
        logits = F.linear(x.detach().view(T, d), layer.gate.weight).float().cpu().numpy()
    ref_logits = (np64(P["x"]) @ np64(P["Wg"]).T)
    assert_close(logits, ref_logits, **TOL[dtype], what="gate logits")

    bf16 = dtype == torch.bfloat16
    # bf16: the oracle rounds where the path stores bf16; the whole-layer function applies
    # the routing weights to the activations, the module composition to the W2 outputs
    orc = O.MoELayerOracle(np64(P["Wg"]), P["bias"].numpy(), np64(P["W1"]), np64(P["W2"]), k,
                           shared=tuple(np64(w) for w in P["shared"]), round_probs_bf16=bf16,
                           store="bf16" if bf16 else None,
                           gate_scale_on="A" if (bf16 and fused and layer.fused_layer) else "Y")
    rout, ridx, _ = orc.forward(np64(P["x"]), logits=logits)
    np.testing.assert_array_equal(idx.view(T, k).cpu().numpy(), ridx)
    tol = TOL[dtype]
    assert_close(np64(out.view(T, d)), rout, **tol, what="out")
    g = orc.backward(np64(P["dout"]), rss=bf16)
    assert_close(np64(x.grad.view(T, d)), g["x"], **tol, what="dx")
    se = layer.shared_experts
    wgrads = (("d gate.weight", layer.gate.weight.grad, "gate_weight"),
              ("dW1", layer.routed_experts.experts.weight.grad, "W1"),
              ("dW2", layer.routed_experts.output_experts.weight.grad, "W2"),
              ("d shared gate", se.gate_proj.weight.grad, "shared_gate"),
              ("d shared up", se.up_proj.weight.grad, "shared_up"),
              ("d shared down", se.down_proj.weight.grad, "shared_down"))
    for what, got, key in wgrads:
        if bf16:  # bf16 sums over stored bf16 summands: + 2^-7 rss (see helpers.TOL)
            assert_close(np64(got), g[key], **tol, what=what, rss=g["rss"][key])
        else:  # fp32 sums over ~T rows: the norm-wise fp32 bound (see helpers.TOL)
            assert_close_fro(np64(got), g[key], what=what)
    return layer


def test_layer_c1_fp32(hip_device):
    """BASELINE config 1 (T=2048 d=256 E=8 k=2 f=512, n_shared_experts=0) in fp32; the
    reference layer still runs a shared expert of width f in that case."""
    run_and_compare(2048, 256, 8, 2, 512, 0, torch.float32, hip_device, bias_std=0.0)


@pytest.mark.parametrize("fused", [True, False])
def test_layer_small_c3_bf16(hip_device, fused):
    """C3's structure (shared expert, k=8) at a size the oracle finishes quickly."""
    run_and_compare(512, 512, 32, 8, 256, 2, torch.bfloat16, hip_device, fused=fused)


@pytest.mark.parametrize("k,E,fused", [(64, 80, True), (32, 40, False), (17, 24, False)])
def test_layer_large_top_k(hip_device, k, E, fused):
    """The largest top-k each path takes: 64 through the whole-layer function (the routing
    kernels' bound), 32 through the module composition, whose ParallelLinear backward forms
    the gates' grad in the combine's backward (one register slot per k, up to 32)."""
    run_and_compare(96, 128, E, k, 64, 1, torch.bfloat16, hip_device, fused=fused, seed=k)


@pytest.mark.parametrize("T,d,E,k,f,fused", [(1, 64, 1, 1, 32, True), (3, 64, 2, 2, 32, True),
                                              (5, 64, 1, 1, 32, False), (64, 128, 1024, 4, 32, True)])
def test_layer_extreme_small_shapes(hip_device, T, d, E, k, f, fused):
    """One token, one expert, every expert selected, and 1024 experts for 64 tokens (most of
    them empty) through the whole layer, forward and backward."""
    run_and_compare(T, d, E, k, f, 1, torch.bfloat16, hip_device, fused=fused, seed=T + E)


def test_layer_fused_matches_composition_fp32(hip_device):
    run_and_compare(700, 128, 16, 4, 96, 1, torch.float32, hip_device, fused=False, seed=3)


@pytest.mark.parametrize("unpad", [False, True])
def test_fused_layer_matches_composition_bf16(hip_device, unpad):
    """The layer as one autograd function (bf16) against the module composition: the same
    routing bit for bit and the same shared down-projection weight grad (same operands).
    The rest within the bf16 tolerance: the gates scale A before the W2 product instead
    of its output (so the output and dW2 round differently) and dA after its GEMM instead
    of before (dH, dW1, the gates' grad); the gate's and shared up/gate weight grads come
    from one split-K launch over their concatenated output grads, and the hidden states'
    grad sums its parts with one rounding."""
    from modeling.model_config import ModelConfig
    from modeling.moe_layer import MoELayer

    torch.manual_seed(2)
    cfg = ModelConfig(hidden_size=256, intermediate_size=128, n_experts=18, n_shared_experts=2,
                      n_experts_per_token=4)
    layer = MoELayer(cfg).to(hip_device).to(torch.bfloat16)
    layer.gate.expert_biases.data = (0.1 * torch.randn(16)).to(hip_device)
    B, S = 2, 300
    valid = torch.tensor([i for i in range(B * S) if (i % 9) != 4], device=hip_device) if unpad else None
    h = torch.randn(B, S, 256, device=hip_device).to(torch.bfloat16)
    dout = torch.randn(B, S, 256, device=hip_device).to(torch.bfloat16)
    runs = []
    for fused in (True, False):
        layer.fused_layer = fused
        layer.zero_grad(set_to_none=True)
        x = h.clone().requires_grad_(True)
        out, idx = layer(x, unpad_indices=valid)
        out.backward(dout)
        runs.append((out, idx, x.grad, {n: p.grad for n, p in layer.named_parameters()}))
    (o1, i1, g1, p1), (o0, i0, g0, p0) = runs
    assert torch.equal(i1, i0)
    assert_close(np64(o1), np64(o0), **TOL[torch.bfloat16], what="out fused vs composition")
    # weight grads are sums over bf16 summands that the two paths round at different
    # points: the allowance is the oracle's summand root-sum-square, once per path
    xv = h.reshape(B * S, 256) if valid is None else h.reshape(B * S, 256)[valid]
    se = layer.shared_experts
    orc = O.MoELayerOracle(np64(layer.gate.weight), layer.gate.expert_biases.cpu().numpy(),
                           np64(layer.routed_experts.experts.weight), np64(layer.routed_experts.output_experts.weight),
                           4, shared=(np64(se.gate_proj.weight), np64(se.up_proj.weight), np64(se.down_proj.weight)),
                           round_probs_bf16=True, store="bf16", gate_scale_on="A")
    with torch.no_grad():
        logits = F.linear(xv, layer.gate.weight).float().cpu().numpy()
    orc.forward(np64(xv), logits=logits)
    dv = dout.reshape(B * S, 256) if valid is None else dout.reshape(B * S, 256)[valid]
    rss = orc.backward(np64(dv), rss=True)["rss"]
    keys = {"gate.weight": "gate_weight", "routed_experts.experts.weight": "W1",
            "routed_experts.output_experts.weight": "W2", "shared_experts.gate_proj.weight": "shared_gate",
            "shared_experts.up_proj.weight": "shared_up"}
    for n in p0:
        if n == "shared_experts.down_proj.weight":
            assert torch.equal(p1[n], p0[n]), n
        else:
            assert_close(np64(p1[n]), np64(p0[n]), **TOL[torch.bfloat16], what=n, rss=2 * rss[keys[n]])
    assert_close(np64(g1), np64(g0), **TOL[torch.bfloat16], what="dx fused vs composition")


def test_layer_unpad_indices(hip_device):
    from modeling.model_config import ModelConfig
    from modeling.moe_layer import MoELayer

    torch.manual_seed(0)
    cfg = ModelConfig(hidden_size=128, intermediate_size=64, n_experts=10, n_shared_experts=2, n_experts_per_token=2)
    layer = MoELayer(cfg).to(hip_device)
    B, S = 3, 40
    h = torch.randn(B, S, 128, device=hip_device)
    valid = torch.tensor([i for i in range(B * S) if (i % 7) != 3], device=hip_device)
    out, idx = layer(h, unpad_indices=valid)
    ref_out, ref_idx = layer(h.view(1, B * S, 128)[:, valid])
    flat = out.view(B * S, 128)
    assert torch.equal(flat[valid], ref_out.view(-1, 128))
    pad = torch.ones(B * S, dtype=torch.bool, device=hip_device)
    pad[valid] = False
    assert (flat[pad] == 0).all() and (idx.view(B * S, -1)[pad] == 0).all()
    assert torch.equal(idx.view(B * S, -1)[valid], ref_idx.view(-1, 2))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_layer_unpad_backward_matches_unpadded(hip_device, dtype):
    """The re-pad folded into the combine (and the padded gradient read in place by its
    backward) gives the gradients of the unpadded computation: bit-identical parameter
    grads, hidden-state grads equal on valid rows and zero on padding."""
    from modeling.model_config import ModelConfig
    from modeling.moe_layer import MoELayer

    torch.manual_seed(1)
    cfg = ModelConfig(hidden_size=128, intermediate_size=64, n_experts=10, n_shared_experts=2, n_experts_per_token=2)
    layer = MoELayer(cfg).to(hip_device).to(dtype)
    layer.gate.expert_biases.data = layer.gate.expert_biases.data.float()
    B, S = 3, 40
    valid = torch.tensor([i for i in range(B * S) if (i % 5) != 1], device=hip_device)
    h = torch.randn(B, S, 128, device=hip_device).to(dtype).requires_grad_(True)
    dout = torch.randn(B, S, 128, device=hip_device).to(dtype)
    out, _ = layer(h, unpad_indices=valid)
    out.backward(dout)
    grads = {n: p.grad.clone() for n, p in layer.named_parameters()}
    layer.zero_grad(set_to_none=True)
    hu = h.detach().view(1, B * S, 128)[:, valid].clone().requires_grad_(True)
    ref, _ = layer(hu)
    ref.backward(dout.view(B * S, 128)[valid].view(1, -1, 128))
    for n, p in layer.named_parameters():
        assert torch.equal(grads[n], p.grad), n
    hg = h.grad.view(B * S, 128)
    assert torch.equal(hg[valid], hu.grad.view(-1, 128))
    pad = torch.ones(B * S, dtype=torch.bool, device=hip_device)
    pad[valid] = False
    assert (hg[pad] == 0).all()


def test_c3_full_size_properties(hip_device):
    """BASELINE config 3 at full size (T=32768 d=2048 E=128 k=8 f=768, shared 1536):
    sort invariants, linearity of the routed combine in the gates (exact for a
    power-of-two scale), and sampled tokens against the oracle."""
    from zmoe import ops
    from scattermoe.mlp import GLUExpertsFunction

    T, d, E, k, f = 32768, 2048, 128, 8, 768
    g = torch.Generator(device=hip_device)
    g.manual_seed(1)
    x = torch.randn(T, d, device=hip_device, generator=g).to(torch.bfloat16)
    W1 = (torch.randn(E, 2 * f, d, device=hip_device, generator=g) / d ** 0.5).to(torch.bfloat16)
    W2 = (torch.randn(E, d, f, device=hip_device, generator=g) / d ** 0.5).to(torch.bfloat16)
    Wg = (torch.randn(E, d, device=hip_device, generator=g) / d ** 0.5).to(torch.bfloat16)
    bias = torch.randn(E, device=hip_device, generator=g) * 0.1
    logits = F.linear(x, Wg)
    idx, w, _ = ops.route_topk(logits, bias, k, round_probs_bf16=True)
    se, ss, off, inv = ops.flatten_sort_count(idx, E)
    assert int(off[-1]) == T * k
    assert torch.equal(torch.sort(ss).values, torch.arange(T * k, device=hip_device))
    assert torch.equal(se, idx.view(-1)[ss])
    assert bool((se[1:] >= se[:-1]).all())
    y1, _ = GLUExpertsFunction.apply(x, w, idx, W1, W2, k, E)
    y2, _ = GLUExpertsFunction.apply(x, w * 2, idx, W1, W2, k, E)
    assert torch.equal(y2.float(), (y1.float() * 2))
    # sampled tokens vs the oracle (each token depends only on its own row)
    rows = torch.randperm(T, generator=gen(2))[:48].to(hip_device)
    sel_idx = idx[rows].cpu().numpy()
    xr, wr = np64(x[rows]), w[rows].double().cpu().numpy()
    ref = np.zeros((rows.numel(), d))
    for e in np.unique(sel_idx):
        W1e, W2e = np64(W1[int(e)]), np64(W2[int(e)])
        for t, j in zip(*np.nonzero(sel_idx == e)):
            hg = W1e @ xr[t]
            a = O.swiglu(hg[None, :])[0]
            ref[t] += wr[t, j] * (W2e @ a)
    assert_close(np64(y1[rows]), ref, **TOL[torch.bfloat16], what="C3 sampled tokens")
