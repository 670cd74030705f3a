"""Shared test helpers: seeded inputs for the BASELINE configs and tolerances."""

from __future__ import annotations

import math

import numpy as np
import torch

# bf16 paths rtol = atol = 2e-2 against the float64
# reference; fp32 paths rtol = atol = 1e-5. The absolute part is taken relative
# to the tensor's largest magnitude when that exceeds 1 (atol * max(1, max|ref|)):
# a reduction over n terms carries ~sqrt(n) roundings of its partial sums, so
# elements that cancel to near zero inside a large tensor (weight grads summed
# over hundreds of rows, bf16 gradients of magnitude ~20 whose ulp is 0.125)
# cannot meet a fixed absolute bound in that precision. Index/wrong-row bugs
# produce errors of the order of the values themselves and still fail.
TOL = {
    torch.bfloat16: dict(rtol=2e-2, atol=2e-2, scale_atol=True),
    torch.float32: dict(rtol=1e-5, atol=1e-5, scale_atol=True),
}


def np64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def assert_close(got, ref, rtol, atol, what="", scale_atol=False):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    if scale_atol and ref.size:
        atol = atol * max(1.0, float(np.abs(ref).max()))
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    if bad.any():
        i = np.unravel_index(np.argmax(err - rtol * np.abs(ref)), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.size} outside rtol={rtol} atol={atol}; "
            f"worst at {i}: got {got[i]!r} ref {ref[i]!r}; max abs err {err.max():.3e}, "
            f"max |ref| {np.abs(ref).max():.3e}")


def rel_err(got, ref) -> float:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def random_topk(T: int, E: int, k: int, seed: int, skew: float = 0.0) -> torch.Tensor:
    """[T, k] distinct expert ids per row; ``skew`` > 0 biases towards low ids (Zipf-like)."""
    g = gen(seed)
    if skew > 0:
        w = torch.tensor([1.0 / (e + 1) ** skew for e in range(E)])
        return torch.multinomial(w.expand(T, E), k, replacement=False, generator=g)
    return torch.argsort(torch.rand(T, E, generator=g), dim=1)[:, :k].contiguous()


def layer_inputs(T, d, E, k, f, fs, seed, dtype, bias_std=0.0):
    """Seeded synthetic layer inputs following the BASELINE.json recipes."""
    g = gen(seed)
    std = 1.0 / math.sqrt(d)
    P = dict(
        x=torch.randn(T, d, generator=g),
        Wg=torch.randn(E, d, generator=g) * std,
        bias=torch.randn(E, generator=g) * bias_std,
        W1=torch.randn(E, 2 * f, d, generator=g) * std,
        W2=torch.randn(E, d, f, generator=g) * std,
        shared=None,
        dout=torch.randn(T, d, generator=g),
    )
    if fs:
        P["shared"] = tuple(torch.randn(*s, generator=g) * std for s in ((fs, d), (fs, d), (d, fs)))
    # round once to the compute dtype so both sides see identical inputs
    for key in ("x", "Wg", "W1", "W2", "dout"):
        P[key] = P[key].to(dtype).float()
    if P["shared"] is not None:
        P["shared"] = tuple(w.to(dtype).float() for w in P["shared"])
    return P
