"""GPU parity at the full sizes of BASELINE.json's configs C2, C4 and C5 for the
routed experts (GLUExpertsFunction, the module composition's fused path).

Routing is compared bit-exactly with the oracle; the sort through its invariants;
the routed GLU MLP forward and backward against the oracle's float64 restatement run
on the device (``oracle/torch_layer.py``; the numpy oracle would take minutes at these
sizes), under the bf16 storage model of this path (routing weights on the W2
outputs, ``gate_scale_on="Y"``), every element at the north star's fixed bf16
tolerance; the weight grads and the gates' grad (sums over stored bf16 summands) with
the summand allowance of ``helpers.TOL``.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from helpers import TOL, close_dev

BF16_TOL = TOL[torch.bfloat16]

pytestmark = pytest.mark.gpu


def close_t(got, ref, what, rss=None):
    """The bf16 bound elementwise on the device (helpers.close_dev)."""
    close_dev(got, ref, what, rtol=BF16_TOL["rtol"], atol=BF16_TOL["atol"], rss=rss)


def glu_reference(x, W1, W2, idx, w):
    """The oracle's routed experts (bf16 storage, weights on the W2 outputs) on the device."""
    from oracle.torch_layer import TorchGLURef

    return TorchGLURef(W1, W2, store="bf16", gate_scale_on="Y", grad_dtype=torch.bfloat16), (x, idx, w)


def make_weights(E, d, f, dev, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    std = d ** -0.5
    W1 = (torch.randn(E, 2 * f, d, device=dev, generator=g, dtype=torch.bfloat16) * std)
    W2 = (torch.randn(E, d, f, device=dev, generator=g, dtype=torch.bfloat16) * std)
    return W1, W2, g


def route_and_check(x, Wg, bias, k):
    """Gate logits on the device, routing on the device, compared bit-exactly with the oracle."""
    from zmoe import ops

    logits = F.linear(x, Wg)
    idx, w, p = ops.route_topk(logits, bias, k, round_probs_bf16=True)
    ridx, rw, rp = O.route_topk(logits.float().cpu().numpy(), bias.cpu().numpy(), k, round_probs_bf16=True)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_array_equal(p.cpu().numpy(), rp)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-6, atol=1e-7)
    return idx, w


def sort_invariants(idx, E):
    from zmoe import ops

    T, k = idx.shape
    se, ss, off, inv = ops.flatten_sort_count(idx, E)
    R = T * k
    counts = torch.bincount(idx.view(-1), minlength=E)
    assert torch.equal(off, torch.cumsum(counts, 0))
    assert torch.equal(se, idx.view(-1)[ss])
    assert torch.equal(torch.sort(ss).values, torch.arange(R, device=idx.device))
    # stable: within an expert, slot ids ascend
    same = se[1:] == se[:-1]
    assert bool((ss[1:][same] > ss[:-1][same]).all())
    assert torch.equal(inv.long()[ss], torch.arange(R, device=idx.device))
    return counts


def test_c2_forward_full(hip_device):
    """C2: T=16384 d=1024 E=64 k=8 f=512, selection bias ~ N(0, 0.1), bf16 forward."""
    from scattermoe.mlp import GLUExpertsFunction

    T, d, E, k, f = 16384, 1024, 64, 8, 512
    W1, W2, g = make_weights(E, d, f, hip_device, seed=21)
    x = torch.randn(T, d, device=hip_device, generator=g).to(torch.bfloat16)
    Wg = (torch.randn(E, d, device=hip_device, generator=g) * d ** -0.5).to(torch.bfloat16)
    bias = torch.randn(E, device=hip_device, generator=g) * 0.1
    idx, w = route_and_check(x, Wg, bias, k)
    sort_invariants(idx, E)
    with torch.no_grad():
        y, _ = GLUExpertsFunction.apply(x, w, idx, W1, W2, k, E)
    ref, args = glu_reference(x, W1, W2, idx, w)
    close_t(y, ref.forward(*args), "C2 output")


def test_c4_skewed_forward_backward(hip_device):
    """C4: T=8192 d=7168 E=256 k=8 f=2048 with Zipf(1.1)-skewed popularity, fwd + bwd."""
    import bench
    from scattermoe.mlp import GLUExpertsFunction

    T, d, E, k, f = 8192, 7168, 256, 8, 2048
    W1, W2, g = make_weights(E, d, f, hip_device, seed=41)
    x = torch.randn(T, d, device=hip_device, generator=g).to(torch.bfloat16)
    Wg = (torch.randn(E, d, device=hip_device, generator=g) * d ** -0.5).to(torch.bfloat16)
    bias, _, _ = bench.zipf_bias(F.linear(x, Wg), k)
    idx, w = route_and_check(x, Wg, bias, k)
    counts = sort_invariants(idx, E)
    assert int(counts.max()) > 4 * T * k // E  # the skew is real: the head expert gets > 4x the mean

    xg = x.clone().requires_grad_(True)
    wg = w.clone().requires_grad_(True)
    W1g = W1.clone().requires_grad_(True)
    W2g = W2.clone().requires_grad_(True)
    y, _ = GLUExpertsFunction.apply(xg, wg, idx, W1g, W2g, k, E)
    dout = torch.randn(T, d, device=hip_device, generator=g).to(torch.bfloat16)
    y.backward(dout)

    ref, args = glu_reference(x, W1, W2, idx, w)
    close_t(y, ref.forward(*args), "C4 output")
    ref_dx, ref_dW1, ref_dW2, ref_dg, rss = ref.backward(dout, rss=True)
    close_t(xg.grad, ref_dx, "C4 dx")
    # sums over stored bf16 summands: + 2^-7 rss (helpers.TOL)
    close_t(wg.grad, ref_dg, "C4 d_gates", rss=rss["d_gates"])
    close_t(W1g.grad, ref_dW1, "C4 dW1 (all experts)", rss=rss["W1"])
    close_t(W2g.grad, ref_dW2, "C4 dW2 (all experts)", rss=rss["W2"])
    for e in (counts == 0).nonzero().flatten().tolist():
        assert not bool(W1g.grad[e].any()) and not bool(W2g.grad[e].any())


@pytest.mark.parametrize("T", [32, 128, 512])
def test_c5_small_batch_forward(hip_device, T):
    """C5: T in {32, 128, 512}, d=2048 E=128 k=8 f=768 — most experts get 0-4 rows."""
    from scattermoe.mlp import GLUExpertsFunction

    d, E, k, f = 2048, 128, 8, 768
    W1, W2, g = make_weights(E, d, f, hip_device, seed=50 + T)
    x = torch.randn(T, d, device=hip_device, generator=g).to(torch.bfloat16)
    Wg = (torch.randn(E, d, device=hip_device, generator=g) * d ** -0.5).to(torch.bfloat16)
    bias = torch.randn(E, device=hip_device, generator=g) * 0.1
    idx, w = route_and_check(x, Wg, bias, k)
    sort_invariants(idx, E)
    with torch.no_grad():
        y, _ = GLUExpertsFunction.apply(x, w, idx, W1, W2, k, E)
    ref, args = glu_reference(x, W1, W2, idx, w)
    close_t(y, ref.forward(*args), f"C5 T={T} output")

