"""The MoE-layer restatement of ``moe_oracle.MoELayerOracle`` in torch float64, for
device-side checks at full sizes.

TEST INFRASTRUCTURE ONLY (like the rest of ``oracle/``): imported by ``tests/``,
never by the product package. The numpy oracle takes minutes per step at the
BASELINE configs C3/C4 (7-17 TFLOP); this module runs the same arithmetic as torch
float64 operations on whatever device its tensors live on, so the full-size GPU
tests can check every output and gradient element. It follows the same reference
lines as the numpy oracle (modeling/moe_layer.py:38-59, scattermoe/mlp.py:74-95,
scattermoe/parallel_experts.py:34-135, modeling/moe_gate.py:27-34,
modeling/expert_layer.py:23-24) and the same rounding model (``store``,
``gate_scale_on``; see ``moe_oracle.storage_rounder`` and ``glu_mlp_forward``).
``tests/test_oracle.py`` pins it against the numpy oracle on the CPU.

Routing is an input here (idx, w, p from ``moe_oracle.route_topk``, which the tests
check bit-exactly against the device); the expert order within each expert is the
stable one (by flat slot id), as in ``moe_oracle.flatten_sort_count``.
"""

from __future__ import annotations

import torch

F64 = torch.float64


def bf16_store(t: torch.Tensor) -> torch.Tensor:
    """float64 -> float32 -> bfloat16 -> float64: the stored-bf16 rounding of
    ``moe_oracle.storage_rounder("bf16")`` (round to nearest even at each step)."""
    return t.to(torch.float32).to(torch.bfloat16).to(F64)


def rounder(store):
    if store is None:
        return lambda t: t
    if store == "bf16":
        return bf16_store
    raise ValueError(f"unknown store {store!r}")


def _swiglu(H: torch.Tensor) -> torch.Tensor:
    f = H.shape[1] // 2
    return torch.nn.functional.silu(H[:, f:]) * H[:, :f]


def _swiglu_backward(dA: torch.Tensor, H: torch.Tensor) -> torch.Tensor:
    f = H.shape[1] // 2
    h, g = H[:, :f], H[:, f:]
    s = torch.sigmoid(g)
    return torch.cat([dA * g * s, dA * h * s * (1.0 + g * (1.0 - s))], dim=1)


def route_topk_backward(d_weight, p_selected, idx, E: int) -> torch.Tensor:
    """``moe_oracle.route_topk_backward`` (autograd of moe_gate.py:27,33-34), float64."""
    dw = d_weight.to(F64)
    p = p_selected.to(F64)
    S_raw = p.abs().sum(dim=1, keepdim=True)
    S = S_raw.clamp_min(1e-12)
    w = p / S
    inner = (dw * w).sum(dim=1, keepdim=True)
    dp = torch.where(S_raw > 1e-12, (dw - inner * torch.sign(p)) / S, dw / S)
    dz = torch.zeros(dw.shape[0], E, dtype=F64, device=dw.device)
    dz.scatter_(1, idx.to(torch.int64), dp * p * (1.0 - p))
    return dz


def expert_rows(idx, E: int):
    """Per expert: (token ids, slot ids j) of its rows, stable by flat slot id."""
    T, k = idx.shape
    flat = idx.reshape(-1)
    order = torch.argsort(flat, stable=True)
    counts = torch.bincount(flat, minlength=E).tolist()
    out, start = [], 0
    for c in counts:
        sl = order[start:start + c]
        out.append((sl // k, sl % k))
        start += c
    return out


class TorchGLURef:
    """The routed experts (``moe_oracle.glu_mlp_forward`` / ``glu_mlp_backward``) in
    float64 torch ops. W1 [E, 2f, d] and W2 [E, d, f] in parameter storage, any float
    dtype; each expert's weights are taken to float64 when used. ``grad_dtype`` is the
    dtype of the returned weight grads (bfloat16 holds them exactly when
    ``store="bf16"``, which saves memory at C4)."""

    def __init__(self, W1, W2, store=None, gate_scale_on="Y", grad_dtype=F64):
        if gate_scale_on not in ("Y", "A"):
            raise ValueError("gate_scale_on must be 'Y' or 'A'")
        self.W1, self.W2 = W1, W2
        self.store = store
        self.r = rounder(store)
        self.gate_scale_on = gate_scale_on
        self.grad_dtype = grad_dtype

    @torch.no_grad()
    def forward(self, x, idx, w, residual=None):
        """y = r(residual + sum_j w Y) (mlp.py:74-95, moe_layer.py:53)."""
        r = self.r
        x64 = x.to(F64)
        T, d = x64.shape
        self.rows = expert_rows(idx, self.W1.shape[0])
        w64 = w.to(F64)
        acc = torch.zeros(T, d, dtype=F64, device=x.device) if residual is None else residual.to(F64).clone()
        self.H, self.A = [], []
        for e, (tok, slot) in enumerate(self.rows):
            if tok.numel() == 0:
                self.H.append(None)
                self.A.append(None)
                continue
            H = r(x64[tok] @ self.W1[e].to(F64).T)                              # mlp.py:80-85
            we = w64[tok, slot][:, None]
            A = r(_swiglu(H)) if self.gate_scale_on == "Y" else r(we * _swiglu(H))   # mlp.py:86
            Y = r(A @ self.W2[e].to(F64).T)                                     # mlp.py:87-93
            acc.index_add_(0, tok, we * Y if self.gate_scale_on == "Y" else Y)  # parallel_experts.py:50-52
            self.H.append(H)
            self.A.append(A)
        self.x64, self.w64, self.k = x64, w64, idx.shape[1]
        return r(acc)

    @torch.no_grad()
    def backward(self, dout, rss=False):
        """(dx unrounded, dW1, dW2, d_gates) as ``moe_oracle.glu_mlp_backward``; with
        ``rss=True`` a fifth item maps "W1", "W2", "d_gates" to each element's summand
        root-sum-square (``moe_oracle.summand_rss``), W1/W2 ones in ``grad_dtype``."""
        r = self.r
        dout64 = dout.to(F64)
        T, d = dout64.shape
        dev = dout.device
        dW1 = torch.empty(self.W1.shape, dtype=self.grad_dtype, device=dev)
        dW2 = torch.empty(self.W2.shape, dtype=self.grad_dtype, device=dev)
        d_gates = torch.zeros(T, self.k, dtype=F64, device=dev)
        dx = torch.zeros(T, d, dtype=F64, device=dev)
        if rss:
            rW1 = torch.zeros(self.W1.shape, dtype=self.grad_dtype, device=dev)
            rW2 = torch.zeros(self.W2.shape, dtype=self.grad_dtype, device=dev)
            rg = torch.zeros(T, self.k, dtype=F64, device=dev)
        for e, (tok, slot) in enumerate(self.rows):
            if tok.numel() == 0:
                dW1[e].zero_()
                dW2[e].zero_()
                continue
            W1e, W2e = self.W1[e].to(F64), self.W2[e].to(F64)
            H, A = self.H[e], self.A[e]
            we = self.w64[tok, slot][:, None]
            if self.gate_scale_on == "Y":
                Y = r(A @ W2e.T)
                d_gates[tok, slot] = (Y * dout64[tok]).sum(1)                   # parallel_experts.py:82
                G = r(we * dout64[tok])                                         # :95-97
                dA = r(G @ W2e)                                                 # :112-120
                dH = r(_swiglu_backward(dA, H))
            else:
                G = dout64[tok]
                dA = r(G @ W2e)
                d_gates[tok, slot] = (dA * _swiglu(H)).sum(1)
                dH = r(_swiglu_backward(we * dA, H))
            dW2[e] = r(G.T @ A).to(self.grad_dtype)                             # :105-110
            dW1[e] = r(dH.T @ self.x64[tok]).to(self.grad_dtype)
            dx.index_add_(0, tok, r(dH @ W1e))                                  # :112-125
            if rss:
                rW2[e] = ((G * G).T @ (A * A)).sqrt().to(self.grad_dtype)
                rW1[e] = ((dH * dH).T @ (self.x64[tok] ** 2)).sqrt().to(self.grad_dtype)
                terms = Y * dout64[tok] if self.gate_scale_on == "Y" else dA * _swiglu(H)
                rg[tok, slot] = (terms * terms).sum(1).sqrt()
        if rss:
            return dx, dW1, dW2, d_gates, {"W1": rW1, "W2": rW2, "d_gates": rg}
        return dx, dW1, dW2, d_gates


class TorchLayerRef:
    """Forward and backward of the MoE layer (valid tokens), ``moe_oracle.MoELayerOracle``
    with the routing given: the shared expert, the routed experts (TorchGLURef) and the
    gate's backward."""

    def __init__(self, Wgate, W1, W2, k, shared=None, store=None, gate_scale_on="Y", grad_dtype=F64):
        self.Wgate, self.k = Wgate, int(k)
        self.glu = TorchGLURef(W1, W2, store=store, gate_scale_on=gate_scale_on, grad_dtype=grad_dtype)
        self.shared = shared
        self.r = rounder(store)
        self.gate_scale_on = gate_scale_on

    @torch.no_grad()
    def forward(self, x, idx, w, p_sel):
        r = self.r
        x64 = x.to(F64)
        S = None
        if self.shared is not None:                                            # moe_layer.py:47
            Wg, Wu, Wd = (t.to(F64) for t in self.shared)
            g = r(x64 @ Wg.T)
            u = r(x64 @ Wu.T)
            a = r(torch.nn.functional.silu(g) * u)
            S = r(a @ Wd.T)
            self._shared = (g, u, a)
        self.x64, self.idx, self.p_sel = x64, idx, p_sel
        return self.glu.forward(x, idx, w, residual=S)                         # moe_layer.py:51-53

    @torch.no_grad()
    def backward(self, dout, rss=False):
        """Grads keyed as ``moe_oracle.MoELayerOracle.backward``; with ``rss=True`` also
        "rss": the summand root-sum-square of every weight grad and of d_gates."""
        r = self.r
        dout64 = dout.to(F64)
        res = self.glu.backward(dout, rss=rss)
        dx, dW1, dW2, d_gates = res[:4]
        E = self.Wgate.shape[0]
        dz = r(route_topk_backward(d_gates, self.p_sel, self.idx, E))
        grads = {"gate_weight": r(dz.T @ self.x64)}
        sq = lambda a, b: ((a * a).T @ (b * b)).sqrt()  # noqa: E731
        if rss:
            grads["rss"] = dict(res[4], gate_weight=sq(dz, self.x64))
        dx_dense = dz @ self.Wgate.to(F64)
        if self.shared is not None:
            Wg, Wu, Wd = (t.to(F64) for t in self.shared)
            g, u, a = self._shared
            grads["shared_down"] = r(dout64.T @ a)
            da = r(dout64 @ Wd)
            s = torch.sigmoid(g)
            du = r(da * g * s)
            dg = r(da * u * s * (1.0 + g * (1.0 - s)))
            dx_dense = dx_dense + dg @ Wg + du @ Wu
            grads["shared_gate"] = r(dg.T @ self.x64)
            grads["shared_up"] = r(du.T @ self.x64)
            if rss:
                grads["rss"].update(shared_gate=sq(dg, self.x64), shared_up=sq(du, self.x64),
                                    shared_down=sq(dout64, a))
        if self.gate_scale_on == "A":
            dx_dense = r(dx_dense)
        grads.update(x=r(dx + dx_dense), W1=dW1, W2=dW2, d_gates=d_gates, d_logits=dz)
        return grads
