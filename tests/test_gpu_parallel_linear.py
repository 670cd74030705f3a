"""GPU parity of ParallelLinear / parallel_linear (reference scattermoe/parallel_experts.py:34-147)
against the oracle's parallel_linear_forward / parallel_linear_backward, in every caller mode:
gathered or grouped input, slot-order or grouped output, gates, bias; fp32 and bf16.

bf16 is compared at the north-star bound rtol = atol = 2e-2 with the oracle's bf16 storage
model (store="bf16": rounded where the path stores a bf16 tensor, pinned against torch's own
bf16 arithmetic in tests/test_oracle.py). The relative Frobenius error against the exact
oracle (no rounding) is printed beside it.
"""

import numpy as np
import pytest
import torch

import oracle as O
from helpers import TOL, assert_close, gen, np64, random_topk

pytestmark = pytest.mark.gpu

# (fan, grouped_in, grouped_out, gates, bias): as tests/test_oracle.py's _PL_MODES
MODES = [
    (4, False, False, False, False),
    (1, False, False, False, True),
    (3, False, True, False, True),
    (4, False, False, True, False),
    (3, False, False, True, True),
    (4, True, False, False, True),
    (4, True, True, False, False),
    (3, True, False, True, True),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("fan,grouped_in,grouped_out,gates,bias", MODES)
def test_parallel_linear_fwd_bwd(hip_device, dtype, fan, grouped_in, grouped_out, gates, bias):
    from scattermoe.parallel_experts import flatten_sort_count, parallel_linear

    T, E, K, N = 160, 8, 256, 192
    R = T * fan
    k = 1 if grouped_in else fan
    idx = random_topk(T, E, fan, seed=fan * 10 + int(grouped_in))
    se, ss, off = flatten_sort_count(idx.to(hip_device), E)
    g = gen(7 * fan + 3 * int(gates) + int(bias))
    x = torch.randn(R if grouped_in else T, K, generator=g).to(dtype)
    Wp = (torch.randn(E, N, K, generator=g) / K ** 0.5).to(dtype)  # nn.Parameter layout [E, out, in]
    b = (torch.randn(E, N, generator=g) * 0.5).to(dtype) if bias else None
    gw = (torch.rand(T, fan, generator=g) + 0.2).to(dtype) if gates else None
    dy_shape = (T, N) if gates else (R, N)
    dy = torch.randn(*dy_shape, generator=g).to(dtype)

    xd = x.to(hip_device).requires_grad_(True)
    Wd = Wp.to(hip_device).requires_grad_(True)
    bd = b.to(hip_device).requires_grad_(True) if bias else None
    gd = gw.to(hip_device).requires_grad_(True) if gates else None
    out = parallel_linear(xd, Wd.permute(0, 2, 1), k, se, ss, off, expert_biases=bd, gates=gd,
                          grouped_in=grouped_in, grouped_out=grouped_out)
    out.backward(dy.to(hip_device))

    sen, ssn, offn = se.cpu().numpy(), ss.cpu().numpy(), off.cpu().numpy()
    Wl = np64(Wp).transpose(0, 2, 1)
    kw = dict(b=None if b is None else np64(b), gates=None if gw is None else np64(gw),
              grouped_in=grouped_in, grouped_out=grouped_out)

    def oracle(store):
        rout, expanded = O.parallel_linear_forward(np64(x), Wl, k, sen, ssn, offn, store=store, **kw)
        rdx, rdW, rdb, rdg = O.parallel_linear_backward(np64(dy), np64(x), Wl, k, sen, ssn, offn,
                                                        output_expanded=expanded, store=store, **kw)
        return dict(out=rout, dx=rdx, dW=rdW.transpose(0, 2, 1), db=rdb, dg=rdg)

    bf16 = dtype == torch.bfloat16
    ref = oracle("bf16" if bf16 else None)
    got = dict(out=np64(out), dx=np64(xd.grad), dW=np64(Wd.grad), db=np64(bd.grad) if bias else None,
               dg=np64(gd.grad) if gates else None)
    tol = TOL[dtype]
    what = f"fan={fan} gin={grouped_in} gout={grouped_out} gates={gates} bias={bias} {dtype}"
    exact = oracle(None) if bf16 else ref
    for name in ("out", "dx", "dW", "db", "dg"):
        if got[name] is None:
            continue
        assert_close(got[name], ref[name], **tol, what=f"{name} {what}")
        if bf16:
            e = np.linalg.norm(got[name] - exact[name]) / max(np.linalg.norm(exact[name]), 1e-30)
            print(f"  {name}: rel. Frobenius error vs the unrounded oracle {e:.2e}")
    counts = np.diff(np.concatenate([[0], offn]))
    for e in np.nonzero(counts == 0)[0]:
        assert not Wd.grad[e].any(), f"empty expert {e} must get exact zeros"
