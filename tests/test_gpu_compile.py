"""The layer under torch.compile, as the reference trainer compiles it (main.py:929).

Every HIP launch on the layer's paths is a ``zmoe::`` custom op with a fake
implementation (``zmoe/library.py``), so Dynamo traces the whole forward into one graph
(no graph break) and AOT autograd traces the backward through the fake shapes. The
compiled step must equal the eager one bit for bit (the same kernels run on the same
inputs). The backend is ``aot_eager``: it runs Dynamo and AOT autograd, and executes the
captured graphs op by op, without generating code for torch's own glue ops. The last test
uses the default inductor backend, as the reference does."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _layer(dev, fused_layer=True, fused_experts=True):
    """A small bf16 layer (C3-like structure) and a zero-centred RMSNorm."""
    from modeling.model_config import ModelConfig
    from modeling.moe_layer import MoELayer
    from modeling.zRMSNorm import ZeroCenteredRMSNorm

    torch.manual_seed(11)
    cfg = ModelConfig(hidden_size=256, intermediate_size=128, n_experts=18, n_shared_experts=2, n_experts_per_token=4)
    layer = MoELayer(cfg).to(dev).to(torch.bfloat16)
    layer.gate.expert_biases.data = (0.1 * torch.randn(16)).to(dev)
    layer.fused_layer = fused_layer
    layer.routed_experts.fused = fused_experts
    norm = ZeroCenteredRMSNorm(256).to(dev)
    with torch.no_grad():
        norm.weight.copy_(torch.randn(256) * 0.2)
    return layer, norm


def _step(fn, h, dout, params):
    for p in params:
        p.grad = None
    x = h.clone().requires_grad_(True)
    out, idx = fn(x)
    out.backward(dout)
    return out.detach(), idx, x.grad, [p.grad.clone() for p in params]


def _inputs(dev, B=2, S=150):
    h = torch.randn(B, S, 256, device=dev).to(torch.bfloat16)
    dout = torch.randn(B, S, 256, device=dev).to(torch.bfloat16)
    valid = torch.tensor([i for i in range(B * S) if (i % 9) != 4], device=dev)
    return h, dout, valid


CASES = {
    "whole-layer function": dict(fused_layer=True, norm=False, unpad=False),
    "whole-layer function, unpad + norm": dict(fused_layer=True, norm=True, unpad=True),
    "module composition": dict(fused_layer=False, norm=False, unpad=False),
    "module composition, unpad + norm": dict(fused_layer=False, norm=True, unpad=True),
}


def _fn(layer, norm, case, valid):
    def fn(x):
        return layer(x, unpad_indices=valid if case["unpad"] else None, norm=norm if case["norm"] else None)
    return fn


@pytest.mark.parametrize("name", list(CASES))
def test_layer_forward_has_no_graph_break(hip_device, name):
    import torch._dynamo

    case = CASES[name]
    layer, norm = _layer(hip_device, fused_layer=case["fused_layer"])
    h, dout, valid = _inputs(hip_device)
    torch._dynamo.reset()
    explanation = torch._dynamo.explain(_fn(layer, norm, case, valid))(h)
    assert explanation.graph_break_count == 0, explanation.break_reasons
    assert explanation.graph_count == 1


@pytest.mark.parametrize("name", list(CASES))
def test_compiled_step_equals_eager(hip_device, name):
    import torch._dynamo

    case = CASES[name]
    layer, norm = _layer(hip_device, fused_layer=case["fused_layer"])
    h, dout, valid = _inputs(hip_device)
    params = list(layer.parameters()) + ([norm.weight] if case["norm"] else [])
    fn = _fn(layer, norm, case, valid)
    ref = _step(fn, h, dout, params)
    torch._dynamo.reset()
    compiled = torch.compile(fn, backend="aot_eager", dynamic=True, fullgraph=True)
    for _ in range(2):  # the second call reuses the compiled graphs
        got = _step(compiled, h, dout, params)
        assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1]) and torch.equal(got[2], ref[2])
        for a, b in zip(got[3], ref[3]):
            assert torch.equal(a, b)
    # dynamic shapes: another token count through the same compiled function
    h2, dout2, valid2 = _inputs(hip_device, S=97)
    fn2 = _fn(layer, norm, case, valid2)
    ref2 = _step(fn2, h2, dout2, params)
    got2 = _step(torch.compile(fn2, backend="aot_eager", dynamic=True, fullgraph=True), h2, dout2, params)
    assert torch.equal(got2[0], ref2[0]) and torch.equal(got2[2], ref2[2])


def test_glumlp_compiles(hip_device):
    """The routed experts alone (GLUMLP's reference call, mlp.py:74)."""
    import torch._dynamo
    from scattermoe.mlp import GLUMLP

    torch.manual_seed(3)
    mlp = GLUMLP(128, 64, 8, 2).to(hip_device).to(torch.bfloat16)
    x = torch.randn(300, 128, device=hip_device).to(torch.bfloat16)
    p = torch.rand(300, 2, device=hip_device)
    idx = torch.argsort(torch.rand(300, 8, device=hip_device), dim=1)[:, :2].contiguous()
    dy = torch.randn(300, 128, device=hip_device).to(torch.bfloat16)

    def step(f):
        mlp.zero_grad(set_to_none=True)
        xx = x.clone().requires_grad_(True)
        y = f(xx, p, idx)
        y.backward(dy)
        return y.detach(), xx.grad, mlp.experts.weight.grad.clone(), mlp.output_experts.weight.grad.clone()

    ref = step(mlp)
    torch._dynamo.reset()
    got = step(torch.compile(mlp, backend="aot_eager", dynamic=True, fullgraph=True))
    for a, b in zip(got, ref):
        assert torch.equal(a, b)


def _amp_layer(dev):
    """The reference's training mode: fp32 master weights, run under bf16 autocast."""
    from modeling.model_config import ModelConfig
    from modeling.moe_layer import MoELayer

    torch.manual_seed(13)
    cfg = ModelConfig(hidden_size=256, intermediate_size=128, n_experts=18, n_shared_experts=2, n_experts_per_token=4)
    layer = MoELayer(cfg).to(dev)
    layer.gate.expert_biases.data = (0.1 * torch.randn(16)).to(dev)
    return layer


@pytest.mark.parametrize("mode", ["bf16", "autocast fp32 weights"])
def test_inductor_compiled_step(hip_device, mode):
    """torch.compile with the default (inductor) backend and dynamic shapes, as main.py:929
    compiles headless_forward, here around the layer with unpad indices; in the reference's
    own mode the forward runs under bf16 autocast with fp32 weights and an fp32 input.
    Inductor generates code for the glue ops around the ``zmoe::`` custom ops (which it calls
    as extern kernels); the glue is exact (casts, gathers, concatenation), so the compiled
    step equals eager bit for bit: routing, output, the input grad and every weight grad."""
    import torch._dynamo

    amp = mode != "bf16"
    if amp:
        layer = _amp_layer(hip_device)
    else:
        layer, _ = _layer(hip_device)
    h, dout, valid = _inputs(hip_device)
    if amp:
        h = h.float()
    params = list(layer.parameters())

    def fn(x):
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=amp):
            return layer(x, unpad_indices=valid)

    ref = _step(fn, h, dout, params)
    torch._dynamo.reset()
    compiled = torch.compile(fn, dynamic=True)
    for _ in range(2):
        got = _step(compiled, h, dout, params)
        assert torch.equal(got[1], ref[1]), "routing differs from eager"
        names = ["out", "d hidden"] + [n for n, _ in layer.named_parameters()]
        for what, a, b in zip(names, [got[0], got[2]] + got[3], [ref[0], ref[2]] + ref[3]):
            assert a.dtype == b.dtype and torch.equal(a, b), f"{what}: {int((a != b).sum())} elements differ"
