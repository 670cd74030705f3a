"""The MoE layer forward under HIP graph capture (torch.cuda.graph): the routing, sort,
grouped GEMMs (tiled and weight-streaming forms) and combine record no allocation, host
sync or memset, so the captured forward replays. Every replay is compared bit for bit
with the eager output, with eager runs of the same layer between the replays (a replay
that depended on state an eager run leaves behind, such as cleared scratch memory,
would show up here).
"""

import pytest
import torch

from helpers import layer_inputs

pytestmark = pytest.mark.gpu


def _layer(T, d, E, k, f, dev, seed):
    from modeling.model_config import ModelConfig
    from modeling.moe_layer import MoELayer

    P = layer_inputs(T, d, E, k, f, f, seed=seed, dtype=torch.bfloat16, bias_std=0.1)
    cfg = ModelConfig(hidden_size=d, intermediate_size=f, n_experts=E + 1, n_shared_experts=1,
                      n_experts_per_token=k)
    layer = MoELayer(cfg)
    with torch.no_grad():
        layer.gate.weight.copy_(P["Wg"])
        layer.routed_experts.experts.weight.copy_(P["W1"])
        layer.routed_experts.output_experts.weight.copy_(P["W2"])
        layer.shared_experts.gate_proj.weight.copy_(P["shared"][0])
        layer.shared_experts.up_proj.weight.copy_(P["shared"][1])
        layer.shared_experts.down_proj.weight.copy_(P["shared"][2])
    layer = layer.to(dev).to(torch.bfloat16)
    layer.gate.expert_biases.data = P["bias"].float().to(dev)
    x = P["x"].to(torch.bfloat16).to(dev).view(1, T, d)
    return layer, x


# T = 16 over E = 32 (k = 4: 64 routed rows, at most 8 per expert on average) takes the
# weight-streaming forward; T = 2048 over E = 8 (1024 rows per expert) the 256 x 256 tiles;
# T = 512 over E = 16 the 128 x 128 tiles
@pytest.mark.parametrize("T,d,E,k,f", [(16, 256, 32, 4, 128), (512, 256, 16, 4, 128), (2048, 512, 8, 2, 256)])
def test_forward_graph_replays_match_eager(hip_device, T, d, E, k, f):
    layer, x = _layer(T, d, E, k, f, hip_device, seed=T)
    with torch.no_grad():
        side = torch.cuda.Stream(hip_device)
        side.wait_stream(torch.cuda.current_stream(hip_device))
        with torch.cuda.stream(side):  # warm up off the capture stream, as torch asks
            for _ in range(2):
                layer(x)
        torch.cuda.current_stream(hip_device).wait_stream(side)
        ref, ref_idx = layer(x)
        ref, ref_idx = ref.clone(), ref_idx.clone()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out, idx = layer(x)
        for r in range(4):
            graph.replay()
            torch.cuda.synchronize(hip_device)
            assert torch.equal(idx, ref_idx), f"replay {r}: routing differs from eager"
            assert torch.equal(out, ref), f"replay {r}: output differs from eager"
            eager, _ = layer(x)
            torch.cuda.synchronize(hip_device)
            assert torch.equal(eager, ref), f"eager run after replay {r} differs"
        # new input written into the captured buffer: the replay follows it
        x2 = torch.randn(x.shape, generator=torch.Generator(device=hip_device).manual_seed(7), device=hip_device)
        x.copy_(x2.to(x.dtype))
        want, _ = layer(x)
        graph.replay()
        torch.cuda.synchronize(hip_device)
        assert torch.equal(out, want), "replay on a new input differs from eager"


# the training step (forward + backward into static .grad tensors): 128 x 128 and 256 x 256
# tiles, the small-expert weight-grad split and the shared expert's split-K weight grads
@pytest.mark.parametrize("T,d,E,k,f", [(512, 256, 16, 4, 128), (2048, 512, 8, 2, 256)])
def test_train_step_graph_replays_match_eager(hip_device, T, d, E, k, f):
    layer, x0 = _layer(T, d, E, k, f, hip_device, seed=T + 1)
    x = x0.clone().requires_grad_(True)
    dout = torch.randn(x.shape, generator=torch.Generator(device=hip_device).manual_seed(3),
                       device=hip_device).to(x.dtype)
    params = [p for p in layer.parameters() if p.requires_grad]
    leaves = [x] + params

    def eager_grads():
        out, _ = layer(x)
        return [out.detach().clone()] + [g.clone() for g in torch.autograd.grad(out, leaves, dout)]

    side = torch.cuda.Stream(hip_device)
    side.wait_stream(torch.cuda.current_stream(hip_device))
    with torch.cuda.stream(side):  # warm up off the capture stream
        for _ in range(2):
            eager_grads()
    torch.cuda.current_stream(hip_device).wait_stream(side)
    ref = eager_grads()
    for t in leaves:
        t.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out, _ = layer(x)
        out.backward(dout)
    names = ["out", "dx"] + [n for n, p in layer.named_parameters() if p.requires_grad]
    for r in range(3):
        graph.replay()
        torch.cuda.synchronize(hip_device)
        got = [out] + [t.grad for t in leaves]
        for name, g, want in zip(names, got, ref):
            assert g is not None and torch.equal(g, want), f"replay {r}: {name} differs from eager"
        again = eager_grads()
        torch.cuda.synchronize(hip_device)
        for name, g, want in zip(names, again, ref):
            assert torch.equal(g, want), f"eager run after replay {r}: {name} differs"
