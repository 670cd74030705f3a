"""The reference MoE layer as plain eager torch (float32): the CPU baseline of
BASELINE.json's configs[0] (C1: T=2048, d=256, E=8, top-2, SwiGLU f=512, no shared
expert; forward) and of the C3 fwd+bwd workload on a token sample (``moe_step``: the
same forward under autograd, then its backward).

TEST AND BASELINE INFRASTRUCTURE ONLY (like the rest of ``oracle/``): ``bench.py``'s
``cpu_baseline`` leg times it and ``tests/test_oracle.py`` pins it against the numpy
oracle. The product package never imports it.

It restates, op for op in torch, what the reference computes for one layer forward:
the gate (modeling/moe_gate.py:26-34: linear, sigmoid, +bias for selection only,
top-k, gather of the unbiased probabilities, L1 normalisation), the routed SwiGLU
experts over rows grouped by expert (scattermoe/mlp.py:74-95 with
scattermoe/parallel_experts.py:21-28 for the grouping: a stable sort of the flat
slots), and the weighted sum over the k slots of each token
(modeling/moe_layer.py:48-56). The reference runs the expert GEMMs as Triton
kernels; here each expert is one torch matmul pair, which is what an eager CPU
run of the same algorithm does.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


@torch.no_grad()
def moe_forward(x, Wg, bias, W1, W2, k: int, shared=None):
    """x [T, d]; Wg [E, d]; bias [E]; W1 [E, 2f, d] (rows 0..f-1: up, f..2f-1: gate);
    W2 [E, d, f]; shared = (gate [fs, d], up [fs, d], down [d, fs]) or None.
    Returns (out [T, d], topk_idx [T, k], topk_weight [T, k])."""
    return _forward(x, Wg, bias, W1, W2, k, shared)


def moe_step(x, Wg, bias, W1, W2, k: int, dout, shared=None):
    """One training step of the layer as eager torch: the forward of ``moe_forward`` under
    autograd, then ``out.backward(dout)``, as the reference's modules differentiate it (the
    gate's gradient flows through the gathered, normalised probabilities; the selection
    bias has none). Returns (out, {"x", "gate_weight", "W1", "W2"[, "shared_gate",
    "shared_up", "shared_down"]}: the grads)."""
    names = ["x", "gate_weight", "W1", "W2"] + (["shared_gate", "shared_up", "shared_down"] if shared else [])
    leaves = [t.detach().requires_grad_(True) for t in [x, Wg, W1, W2] + list(shared or ())]
    with torch.enable_grad():
        out, _, _ = _forward(leaves[0], leaves[1], bias, leaves[2], leaves[3], k,
                             tuple(leaves[4:]) if shared else None)
        out.backward(dout)
    return out.detach(), {n: t.grad for n, t in zip(names, leaves)}


def _forward(x, Wg, bias, W1, W2, k: int, shared=None):
    T, d = x.shape
    E, two_f, _ = W1.shape
    f = two_f // 2
    p = torch.sigmoid(F.linear(x, Wg))                          # moe_gate.py:26-27
    _, idx = torch.topk(p + bias, k, dim=-1, sorted=False)      # :29-30
    w = F.normalize(p.gather(-1, idx), p=1, dim=-1)             # :33-34
    flat = idx.reshape(-1)
    order = torch.argsort(flat, stable=True)                    # parallel_experts.py:21-28
    counts = torch.bincount(flat, minlength=E).tolist()
    xs = x[order // k]                                          # rows grouped by expert
    parts = []
    # split / unbind: under autograd their backwards are one concatenation each
    W1e, W2e, xe = W1.unbind(0), W2.unbind(0), xs.split(counts)
    for e, c in enumerate(counts):                              # mlp.py:80-87, one expert at a time
        if c:
            H = xe[e] @ W1e[e].t()
            A = F.silu(H[:, f:]) * H[:, :f]
            parts.append(A @ W2e[e].t())
    ys = torch.cat(parts) if parts else x.new_zeros(0, d)
    Y = ys[torch.argsort(order)]                                # back to slot order
    out = (Y.view(T, k, d) * w.unsqueeze(-1)).sum(dim=1)        # moe_layer.py:48-56
    if shared is not None:                                      # expert_layer.py:23-24
        g, u, dn = shared
        out = out + (F.silu(F.linear(x, g)) * F.linear(x, u)) @ dn.t()
    return out, idx, w


def c1_inputs(T=2048, d=256, E=8, f=512, seed=0):
    """Seeded C1 inputs as BASELINE.json configs[0] states them: x ~ N(0, 1), gate
    weight ~ N(0, 0.02), selection bias 0, expert weights ~ N(0, 1/sqrt(d))."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, d, generator=g)
    Wg = torch.randn(E, d, generator=g) * 0.02
    W1 = torch.randn(E, 2 * f, d, generator=g) * d ** -0.5
    W2 = torch.randn(E, d, f, generator=g) * d ** -0.5
    return x, Wg, torch.zeros(E), W1, W2
