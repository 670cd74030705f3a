"""GPU parity: routing (bit-exact given logits), the stable expert sort, counts."""

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, gen, random_topk

pytestmark = pytest.mark.gpu


def _route_case(T, E, k, seed, dtype, bias_std, ties=False, nan=False):
    g = gen(seed)
    logits = torch.randn(T, E, generator=g) * 2
    if ties:
        logits[: T // 2] = torch.round(logits[: T // 2] * 2) / 2  # many equal logits per row
    if nan:
        logits[3, E // 2] = float("nan")
    logits = logits.to(dtype)
    bias = torch.randn(E, generator=g) * bias_std
    if ties:
        bias[: E // 2] = 0.0
    return logits, bias


@pytest.mark.parametrize("T,E,k", [(2048, 8, 2), (1000, 64, 8), (777, 128, 8), (300, 256, 8), (64, 1024, 16),
                                   (33, 5, 5), (16, 70, 1),
                                   # bf16 four-tokens-per-wave kernel: partial 16-expert lanes, one
                                   # occupied lane, k = 16, token counts not divisible by 4
                                   (513, 200, 8), (99, 136, 16), (50, 8, 8), (1001, 120, 3), (64, 256, 16),
                                   # eight tokens per wave (8-lane rows) for E <= 128 and k <= 8, 16-lane
                                   # rows of 8 experts for k in 9..16 at E <= 128
                                   (301, 128, 12), (77, 64, 16), (263, 16, 5),
                                   # the largest k (one slot per lane of the one-row-per-wave kernel)
                                   (40, 100, 64), (9, 64, 64)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_route_topk_bit_exact(hip_device, T, E, k, dtype):
    logits, bias = _route_case(T, E, k, seed=T + E, dtype=dtype, bias_std=0.1, ties=True, nan=T > 3)
    from zmoe import ops

    rb = dtype == torch.bfloat16
    idx, w, p = ops.route_topk(logits.to(hip_device), bias.to(hip_device), k, round_probs_bf16=rb)
    ridx, rw, rp = O.route_topk(logits.float().numpy(), bias.numpy(), k, round_probs_bf16=rb)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_array_equal(p.cpu().numpy(), rp)  # sigmoid evaluated identically (f64, one rounding)
    ok = ~np.isnan(rw).any(axis=1)
    assert_close(w.cpu().numpy()[ok], rw[ok], rtol=1e-6, atol=1e-7, what="topk_weight")


@pytest.mark.parametrize("T,E,k", [(777, 128, 8), (301, 128, 12), (130, 64, 8), (99, 200, 8)])
def test_route_topk_bf16_logits_fp32_probs(hip_device, T, E, k):
    """bf16 logits with probabilities kept in fp32 (round_probs_bf16=False): the several-tokens-per-wave
    kernels evaluate the sigmoid in double instead of reading the bf16 table."""
    logits, bias = _route_case(T, E, k, seed=3 * T + E, dtype=torch.bfloat16, bias_std=0.1, ties=True, nan=True)
    from zmoe import ops

    idx, w, p = ops.route_topk(logits.to(hip_device), bias.to(hip_device), k, round_probs_bf16=False)
    ridx, rw, rp = O.route_topk(logits.float().numpy(), bias.numpy(), k, round_probs_bf16=False)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_array_equal(p.cpu().numpy(), rp)
    ok = ~np.isnan(rw).any(axis=1)
    assert_close(w.cpu().numpy()[ok], rw[ok], rtol=1e-6, atol=1e-7, what="topk_weight")


@pytest.mark.parametrize("bias_std,rb", [(0.0, True), (0.3, True), (0.3, False)])
def test_route_topk_every_bf16_logit(hip_device, bias_std, rb):
    """Every one of the 65536 bf16 values as a logit (NaNs, infinities, subnormals, both
    zeros and the saturated logits included), all selected (k = E = 64): each probability
    equals the oracle's bf16(fp32(sigmoid in float64)) (or, with rb False, the fp32 value)
    bit for bit, whichever evaluation the kernel used."""
    from zmoe import ops

    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    logits = bits.view(torch.bfloat16).reshape(1024, 64)
    bias = torch.randn(64, generator=gen(9)) * bias_std
    idx, w, p = ops.route_topk(logits.to(hip_device), bias.to(hip_device), 64, round_probs_bf16=rb)
    ridx, rw, rp = O.route_topk(logits.float().numpy(), bias.numpy(), 64, round_probs_bf16=rb)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_array_equal(p.cpu().numpy(), rp)


def _hard_fp32_logits(n_mid: int, seed: int) -> np.ndarray:
    """fp32 logits where a bf16 probability is hardest to get right from fp32 arithmetic:
    z = logit(midpoint between two adjacent bf16 probabilities), nudged by -24..24 fp32 ulps,
    so sigmoid(z) lies within a few fp32 ulps of a bf16 rounding midpoint; |z| around 80
    (where the kernel's fp32 evaluation hands over to double); the saturation edge
    (-88.7228...: fp32 exp(-z) overflows from there on, p = 0); and NaN / +-inf."""
    r = np.random.default_rng(seed)
    m = O.bf16_round(r.uniform(1e-6, 0.99, n_mid).astype(np.float32))  # stays below 1 after rounding
    ulp = (m.view(np.uint32) & 0x7F800000).view(np.float32) * np.float32(2.0 ** -7)  # bf16 ulp of m
    mid = m.astype(np.float64) + ulp.astype(np.float64) / 2
    z0 = np.log(mid / (1.0 - mid)).astype(np.float32)
    nudge = r.integers(-24, 25, n_mid).astype(np.int64)
    z = (z0.view(np.int32).astype(np.int64) + np.where(z0 < 0, -nudge, nudge)).astype(np.int32).view(np.float32)
    edge = np.float32(O.SIGMOID_ZERO_BELOW)
    around = [np.nextafter(edge, np.float32(0)), edge, np.nextafter(edge, np.float32(-200))]
    special = np.array([80.0, -80.0, 79.99999, -79.99999, 80.00001, -80.00001, 88.0, -88.0, 88.75, -88.75,
                        -89.0, -92.5, -103.0, -110.0, 110.0, 0.0, -0.0, np.inf, -np.inf, np.nan] + around,
                       dtype=np.float32)
    band = r.uniform(-90.0, -78.0, 400).astype(np.float32)
    return np.concatenate([z, special, band, -band[:100]])


@pytest.mark.parametrize("k,rb", [(64, True), (8, True), (64, False)])
def test_route_topk_fp32_logits_hard_cases(hip_device, k, rb):
    """fp32 logits at the hard cases. With bf16-rounded probabilities (round_probs_bf16=True,
    as a bf16 gate over an fp32 projection) the kernel's fp32 sigmoid with its guard band
    around bf16 midpoints and its double fallback must give the oracle's bf16(fp32(sigmoid))
    bit for bit, and so the same selection; with fp32 probabilities the double evaluation,
    0 from the saturation edge on."""
    from zmoe import ops

    E = 64
    z = _hard_fp32_logits(64 * 300, seed=k)
    n = (z.size // E) * E
    logits = torch.from_numpy(z[:n].copy()).reshape(-1, E)
    perm = torch.randperm(n, generator=gen(k)).reshape(-1, E)  # mix the kinds within rows
    logits = logits.reshape(-1)[perm.reshape(-1)].reshape(-1, E).contiguous()
    bias = torch.zeros(E) if k == E else torch.randn(E, generator=gen(5)) * 1e-3
    idx, w, p = ops.route_topk(logits.to(hip_device), bias.to(hip_device), k, round_probs_bf16=rb)
    ridx, rw, rp = O.route_topk(logits.numpy(), bias.numpy(), k, round_probs_bf16=rb)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    got, ref = p.cpu().numpy(), rp
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(got[ok].view(np.uint32), ref[ok].view(np.uint32))


def test_route_equal_scores_and_forced_bias(hip_device):
    from zmoe import ops

    T, E, k = 128, 32, 4
    logits = torch.zeros(T, E, device=hip_device)
    bias = torch.zeros(E, device=hip_device)
    idx, w, _ = ops.route_topk(logits, bias, k)
    assert (idx.cpu() == torch.arange(k)).all()
    assert torch.allclose(w.cpu(), torch.full((T, k), 0.25))
    bias[17] = 50.0
    idx, w, p = ops.route_topk(torch.randn(T, E, device=hip_device), bias, k)
    assert (idx[:, 0] == 17).all()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("E,k", [(64, 8), (100, 40), (128, 64)])
def test_route_backward(hip_device, dtype, E, k):
    """Up to 16 slots per token through scalar registers, more through lane shuffles."""
    from zmoe import ops

    T = 500
    logits, bias = _route_case(T, E, k, seed=5, dtype=dtype, bias_std=0.1)
    idx, w, p = ops.route_topk(logits.to(hip_device), bias.to(hip_device), k,
                               round_probs_bf16=dtype == torch.bfloat16)
    dw = torch.randn(T, k, generator=gen(6))
    dz = ops.route_topk_backward(dw.to(hip_device), p, idx, E, torch.float32)
    ref = O.route_topk_backward(dw.numpy(), p.cpu().numpy(), idx.cpu().numpy(), E)
    assert_close(dz.cpu().numpy(), ref, rtol=1e-5, atol=1e-6, what="d_logits")
    # into the trailing columns of a wider buffer (rows 40 + E apart); the rest is left alone
    buf = torch.full((T, 40 + E), 7.0, device=hip_device)
    ops.route_topk_backward(dw.to(hip_device), p, idx, E, torch.float32, out=buf[:, 40:])
    assert torch.equal(buf[:, 40:], dz) and bool((buf[:, :40] == 7.0).all())


@pytest.mark.parametrize("T,E,k,skew", [(2048, 8, 2, 0.0), (16384, 64, 8, 0.0), (32768, 128, 8, 0.0),
                                        (8192, 256, 8, 1.1), (32, 128, 8, 0.0), (1, 1, 1, 0.0),
                                        (5000, 1024, 3, 1.5),
                                        # 512 tiles x 129 buckets: above the single-scatter table
                                        # bound, so the histogram / scan / scatter launches run
                                        (65536, 128, 8, 0.0)])
def test_flatten_sort_count_bit_exact(hip_device, T, E, k, skew):
    from zmoe import ops

    idx = random_topk(T, E, k, seed=T + E, skew=skew)
    se, ss, off, inv, ws = ops.flatten_sort_count(idx.to(hip_device), E, return_workspace=True)
    rse, rss, roff = O.flatten_sort_count(idx.numpy(), E)
    np.testing.assert_array_equal(se.cpu().numpy(), rse)
    np.testing.assert_array_equal(ss.cpu().numpy(), rss)
    np.testing.assert_array_equal(off.cpu().numpy(), roff)
    np.testing.assert_array_equal(inv.cpu().numpy(), O.inverse_permutation(rss))
    assert not ops.sort_out_of_range(ws)
    np.testing.assert_array_equal(ops.bincount(idx.to(hip_device), E).cpu().numpy(), O.expert_counts(idx.numpy(), E))
    np.testing.assert_array_equal(ops.offsets_from_sorted(se, E).cpu().numpy(), roff)


def test_sort_empty_and_out_of_range(hip_device):
    from zmoe import ops

    empty = torch.empty(0, 8, dtype=torch.int64, device=hip_device)
    se, ss, off, inv = ops.flatten_sort_count(empty, 16)
    assert se.numel() == 0 and (off.cpu() == 0).all()
    bad = torch.tensor([[0, 3], [7, 1], [2, -1]], device=hip_device)
    se, ss, off, inv, ws = ops.flatten_sort_count(bad, 4, return_workspace=True)
    assert ops.sort_out_of_range(ws)
    # valid slots sorted first, the out-of-range ones after them; still a permutation
    assert off.cpu().tolist() == [1, 2, 3, 4]
    assert sorted(ss.cpu().tolist()) == list(range(6))
    assert se.cpu().tolist()[:4] == [0, 1, 2, 3]


def test_bias_update_matches_reference_rule(hip_device):
    from zmoe import ops

    T, E, k = 4096, 64, 8
    idx = random_topk(T, E, k, seed=3, skew=0.7)
    _, _, off, _ = ops.flatten_sort_count(idx.to(hip_device), E)
    b0 = (torch.randn(E, generator=gen(4)) * 0.01).float()
    b = b0.to(hip_device).clone()
    ops.bias_update_(b, off, 1e-3)
    np.testing.assert_array_equal(b.cpu().numpy(), O.bias_update(b0.numpy(), idx.numpy(), E, 1e-3))
