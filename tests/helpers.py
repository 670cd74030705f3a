"""Shared test helpers: seeded inputs for the BASELINE configs and tolerances."""

from __future__ import annotations

import math

import numpy as np
import torch

# North-star tolerances, elementwise: |got - ref| <= atol + rtol |ref| with
# bf16 paths rtol = atol = 2e-2 and fp32 paths rtol = atol = 1e-5, against the
# float64 oracle. Where the path stores bf16 intermediates (H, A, Y, dA, dH, the
# per-slot input grads) the oracle rounds at the same points (store="bf16").
#
# Two kinds of result get a stated allowance on top, because no implementation in
# that precision can meet the bare bound on every element:
#
# * bf16 reductions over stored bf16 summands (weight grads, the gates' grad): the
#   path and the oracle accumulate in a different order (fp32 vs float64), so about
#   2e-4 of the bf16 values each GEMM stores land one ulp apart (measured on MI355X for
#   this build's GEMMs and hipBLASLt alike), and one such flip in a large summand moves
#   a sum that cancels to near zero by up to 2^-8 max|summand|. These elements are
#   bounded by atol + rtol |ref| + 2^-7 rss, with rss the root-sum-square of the
#   element's own summands from the oracle (rss >= max|summand|: two flips allowed).
#   An element built from a wrong row or expert still fails: its error is a whole
#   summand, not 2^-8 of one.
# * fp32 weight grads that sum thousands of products (|dW| ~ 100, where the fp32 ulp is
#   7.6e-6 and the rounding error of the sum grows like sqrt(n) ulps of its partial
#   sums; numpy's own float32 BLAS misses 1e-5 there by 1.7-5x at C1) are compared
#   norm-wise, ||got - ref||_F <= 1e-5 ||ref||_F (assert_close_fro), which still fails a
#   single wrong element larger than 1e-5 of the tensor's norm.
TOL = {
    torch.bfloat16: dict(rtol=2e-2, atol=2e-2),
    torch.float32: dict(rtol=1e-5, atol=1e-5),
}
FRO_F32 = 1e-5
FLIP_RSS = 2.0 ** -7   # allowance per unit of summand root-sum-square (two bf16 ulps)


def np64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def assert_close(got, ref, rtol, atol, what="", rss=None):
    """|got - ref| <= atol + rtol |ref| (+ FLIP_RSS * rss for bf16 reductions); NaN
    must sit in the same places on both sides."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    nan_g, nan_r = np.isnan(got), np.isnan(ref)
    if not np.array_equal(nan_g, nan_r):
        raise AssertionError(f"{what}: NaN in {int(nan_g.sum())} elements of got, {int(nan_r.sum())} of ref, "
                             f"{int((nan_g != nan_r).sum())} placed differently")
    got = np.where(nan_r, 0.0, got)
    ref = np.where(nan_r, 0.0, ref)
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    if rss is not None:
        bound = bound + FLIP_RSS * np.asarray(rss, dtype=np.float64)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.size} outside rtol={rtol} atol={atol}"
            f"{' + 2^-7 rss' if rss is not None else ''}; worst at {i}: got {got[i]!r} ref {ref[i]!r} "
            f"bound {bound[i]!r}; max abs err {err.max():.3e}, max |ref| {np.abs(ref).max():.3e}")


def assert_close_fro(got, ref, rel=FRO_F32, what=""):
    """Norm-wise ||got - ref||_F <= rel ||ref||_F (fp32 weight grads of long sums)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    e, n = float(np.linalg.norm(got - ref)), float(np.linalg.norm(ref))
    if e > rel * n:
        raise AssertionError(f"{what}: ||got - ref||_F = {e:.3e} > {rel} x ||ref||_F = {rel * n:.3e}")


def close_dev(got: torch.Tensor, ref: torch.Tensor, what: str, rtol=2e-2, atol=2e-2, rss=None,
              chunk_elems=1 << 28, verbose=True) -> float:
    """assert_close on the device, in float64, over chunks of the leading dim (a C4 weight
    grad holds 7.5e9 elements). Returns the worst |err| / bound."""
    assert got.shape == ref.shape, (what, tuple(got.shape), tuple(ref.shape))
    got, ref = got.detach(), ref.detach()
    if rss is not None:
        assert rss.shape == ref.shape, (what, "rss", tuple(rss.shape))
        rss = rss.detach()
    lead = got.shape[0] if got.dim() else 1
    per = max(1, got.numel() // max(lead, 1))
    step = max(1, chunk_elems // per)
    worst, where, n_bad, maxref = 0.0, None, 0, 0.0
    for i0 in range(0, lead, step):
        g = got[i0:i0 + step].double()
        r = ref[i0:i0 + step].double()
        if not torch.equal(torch.isnan(g), torch.isnan(r)):
            raise AssertionError(f"{what}: NaN placed differently")
        g = torch.nan_to_num(g, nan=0.0)
        r = torch.nan_to_num(r, nan=0.0)
        bound = atol + rtol * r.abs()
        if rss is not None:
            bound = bound + FLIP_RSS * rss[i0:i0 + step].double()
        ratio = (g - r).abs() / bound
        m = float(ratio.max())
        n_bad += int((ratio > 1.0).sum())
        maxref = max(maxref, float(r.abs().max()))
        if m > worst:
            j = int(torch.argmax(ratio.flatten()))
            worst, where = m, (i0 * per + j, g.flatten()[j].item(), r.flatten()[j].item(), bound.flatten()[j].item())
        del g, r, bound, ratio
    if verbose:
        print(f"  {what}: worst |err| / bound = {worst:.3f}; max |ref| {maxref:.3g}"
              f"{' (bound includes 2^-7 rss)' if rss is not None else ''}", flush=True)
    if n_bad:
        raise AssertionError(f"{what}: {n_bad}/{got.numel()} outside rtol={rtol} atol={atol}"
                             f"{' + 2^-7 rss' if rss is not None else ''}; worst flat index {where[0]}: "
                             f"got {where[1]!r} ref {where[2]!r} bound {where[3]!r}")
    return worst


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
