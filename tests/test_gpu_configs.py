"""GPU parity at the full sizes of BASELINE.json's configs C2, C4 and C5.

Routing is compared bit-exactly with the oracle; the sort through its invariants;
the routed GLU MLP forward and backward against a plain float32 torch reference of
the same computation (per expert, on the GPU: float64 on the CPU would take
minutes at these sizes), with the bf16 tolerance of the north star.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from helpers import TOL

BF16_TOL = TOL[torch.bfloat16]

pytestmark = pytest.mark.gpu


def close_t(got: torch.Tensor, ref: torch.Tensor, what: str, rtol=BF16_TOL["rtol"], atol=BF16_TOL["atol"]):
    """TOL[bf16] on the GPU: |got - ref| <= atol * max(1, max|ref|) + rtol * |ref|."""
    got = got.float()
    ref = ref.float()
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    a = atol * max(1.0, float(ref.abs().max()))
    err = (got - ref).abs()
    bad = err > a + rtol * ref.abs()
    if bool(bad.any()):
        i = int(torch.argmax((err - rtol * ref.abs()).flatten()))
        raise AssertionError(f"{what}: {int(bad.sum())}/{bad.numel()} outside tolerance; worst flat index {i}: "
                             f"got {got.flatten()[i].item()!r} ref {ref.flatten()[i].item()!r}")


def expert_rows(idx: torch.Tensor, E: int):
    """For each expert: (token ids, slot ids j) of its routed rows."""
    T, k = idx.shape
    flat = idx.reshape(-1)
    order = torch.argsort(flat, stable=True)
    counts = torch.bincount(flat, minlength=E).tolist()
    out, start = [], 0
    for e in range(E):
        sl = order[start:start + counts[e]]
        out.append((sl // k, sl % k))
        start += counts[e]
    return out


def glu_reference(x, W1, W2, idx, w, dout=None, dw_experts=()):
    """float32 reference of the routed GLU MLP (mlp.py:74-95, first half of W1 = h, second = gate).

    Returns out [T, d]; with ``dout``: also dx [T, d], d_gates [T, k] and {e: (dW1_e, dW2_e)}
    for the experts in ``dw_experts``.
    """
    T, d = x.shape
    E, two_f, _ = W1.shape
    f = two_f // 2
    out = torch.zeros(T, d, device=x.device)
    dx = torch.zeros(T, d, device=x.device) if dout is not None else None
    dg = torch.zeros(idx.shape, device=x.device) if dout is not None else None
    dws = {}
    for e, (tok, slot) in enumerate(expert_rows(idx, E)):
        if tok.numel() == 0:
            if e in dw_experts:
                dws[e] = (torch.zeros(two_f, d, device=x.device), torch.zeros(d, f, device=x.device))
            continue
        Xe = x[tok].float()
        W1e, W2e = W1[e].float(), W2[e].float()
        Hg = Xe @ W1e.t()
        h, g = Hg[:, :f], Hg[:, f:]
        A = F.silu(g) * h
        Y = A @ W2e.t()
        we = w[tok, slot].float()[:, None]
        out.index_add_(0, tok, we * Y)
        if dout is None:
            continue
        do = dout[tok].float()
        dg[tok, slot] = (Y * do).sum(1)
        dYg = we * do
        dA = dYg @ W2e
        s = torch.sigmoid(g)
        dH = torch.cat([dA * g * s, dA * h * s * (1 + g * (1 - s))], dim=1)
        dx.index_add_(0, tok, dH @ W1e)
        if e in dw_experts:
            dws[e] = (dH.t() @ Xe, dYg.t() @ A)
    if dout is None:
        return out
    return out, dx, dg, dws


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
        y = GLUExpertsFunction.apply(x, w, idx, W1, W2, k, E)
    close_t(y, glu_reference(x, W1, W2, idx, w), "C2 output")


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
    y = GLUExpertsFunction.apply(xg, wg, idx, W1g, W2g, k, E)
    dout = torch.randn(T, d, device=hip_device, generator=g).to(torch.bfloat16)
    y.backward(dout)

    nz = (counts > 0).nonzero().flatten()
    head, tail = int(torch.argmax(counts)), int(nz[torch.argmin(counts[nz])])
    empty = [int(e) for e in (counts == 0).nonzero().flatten()[:1]]
    check = sorted({head, tail, *empty, *range(0, E, 37)})
    ref_out, ref_dx, ref_dg, ref_dw = glu_reference(x, W1, W2, idx, w, dout, dw_experts=check)
    close_t(y, ref_out, "C4 output")
    close_t(xg.grad, ref_dx, "C4 dx")
    close_t(wg.grad, ref_dg, "C4 d_gates")
    for e in check:
        close_t(W1g.grad[e], ref_dw[e][0], f"C4 dW1[{e}] ({int(counts[e])} rows)")
        close_t(W2g.grad[e], ref_dw[e][1], f"C4 dW2[{e}] ({int(counts[e])} rows)")
    for e in empty:
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
        y = GLUExpertsFunction.apply(x, w, idx, W1, W2, k, E)
    close_t(y, glu_reference(x, W1, W2, idx, w), f"C5 T={T} output")

