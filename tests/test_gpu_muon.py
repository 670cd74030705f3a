"""GPU parity of the Newton-Schulz orthogonalisation (optimizer/muon.py:6-32) through
the C ABI (``zmoe_newton_schulz5`` via ``zmoe.ops.newton_schulz5``).

Comparisons are against the oracle's bf16 mode, which rounds where the reference's
bf16 tensor arithmetic rounds (pinned against torch's own bf16 ops on the CPU).
The normalisation alone (steps = 0) is compared bit for bit. One and two steps are
compared by relative Frobenius error per matrix against 2e-3: the only differences
left are fp32 accumulation order inside the GEMMs (and, for the symmetric products,
the mirrored tiles), which flip a few bf16 roundings. The iteration amplifies such
flips about tenfold per step from the third step on (its slope at 0 is a = 3.44), so
after five steps two correct bf16 implementations already differ by up to ~1.5% (the
oracle against torch's own CPU bf16 arithmetic on these shapes); five steps are
compared against 5e-2. At the C3 stack sizes the check is the same on sampled
matrices, plus the singular values of the result against the exact-arithmetic closed
form U phi^5(S / ||G||) V^T, which the rounding noise does not move.
"""

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

REL_FRO = {1: 2e-3, 2: 2e-3, 5: 5e-2}  # by step count (see the module docstring)


def rel_fro(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(got - ref) / np.linalg.norm(ref))


def make_stack(shape, seed, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return torch.randn(*shape, device=dev, generator=g)


@pytest.mark.parametrize("shape", [(3, 64, 128), (2, 128, 64), (1, 256, 256), (4, 40, 72), (2, 512, 768), (3, 200, 264), (2, 648, 1024)])
def test_normalisation_bit_exact(hip_device, shape):
    from zmoe import ops

    G = make_stack(shape, 1, hip_device)
    got = ops.newton_schulz5(G, 0)
    assert got.dtype == torch.bfloat16 and got.shape == G.shape
    np.testing.assert_array_equal(got.float().cpu().numpy(), O.newton_schulz5(G.cpu().numpy(), 0))


# (2, 512, 768), (3, 200, 264) and (2, 648, 1024) span several tiles per matrix (128 and 256
# tiles, full and partial), so the symmetric products' mirrored tiles are exercised
@pytest.mark.parametrize("shape", [(3, 64, 128), (2, 128, 64), (1, 256, 256), (4, 40, 72), (2, 512, 768), (3, 200, 264), (2, 648, 1024)])
@pytest.mark.parametrize("steps", [1, 2, 5])
def test_steps_match_oracle(hip_device, shape, steps):
    from zmoe import ops

    G = make_stack(shape, 2 + steps, hip_device)
    got = ops.newton_schulz5(G, steps).float().cpu().numpy()
    ref = O.newton_schulz5(G.cpu().numpy(), steps)
    for e in range(shape[0]):
        err = rel_fro(got[e], ref[e])
        assert err <= REL_FRO[steps], (shape, steps, e, err)


def test_input_untouched_and_dropin_name(hip_device):
    from zmoe.muon import zeropower_via_newtonschulz5

    G = make_stack((2, 64, 96), 5, hip_device).bfloat16()
    G0 = G.clone()
    out = zeropower_via_newtonschulz5(G, 5)
    assert torch.equal(G, G0)  # the bf16 input is not overwritten
    assert out.dtype == torch.bfloat16 and out.shape == G.shape
    assert rel_fro(out.float().cpu().numpy()[1], O.newton_schulz5(G.float().cpu().numpy(), 5)[1]) <= REL_FRO[5]


def test_rejects_unaligned_sizes(hip_device):
    from zmoe import ops
    from zmoe._lib import ZmoeError

    with pytest.raises((ZmoeError, ValueError)):
        ops.newton_schulz5(torch.randn(2, 20, 36, device=hip_device), 5)


@pytest.mark.parametrize("name,shape", [("W1 stack [E, 2f, d]", (128, 1536, 2048)),
                                        ("W2 stack [E, d, f] (tall)", (128, 2048, 768))])
def test_c3_expert_stack(hip_device, name, shape):
    """MuonMD on the C3 routed-expert weights: E=128, d=2048, f=768, 5 steps."""
    from zmoe import ops

    G = make_stack(shape, 11, hip_device)
    out = ops.newton_schulz5(G, 5)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out.float()).all())
    for e in (0, 127):
        g = G[e].cpu().numpy()
        got = out[e].float().cpu().numpy()
        ref = O.newton_schulz5(g[None], 5)[0]
        assert rel_fro(got, ref) <= REL_FRO[5], (name, e, rel_fro(got, ref))
        s_got = np.linalg.svd(got.astype(np.float64), compute_uv=False)
        S = np.linalg.svd(g.astype(np.float64), compute_uv=False)
        s = S / (np.linalg.norm(g.astype(np.float64)) + 1e-7)
        a, b, c = O.NS_COEFFS
        for _ in range(5):
            s = a * s + b * s**3 + c * s**5
        s_exact = np.sort(s)[::-1]
        assert np.max(np.abs(s_got - s_exact)) < 0.1, (name, e, np.max(np.abs(s_got - s_exact)))


@pytest.mark.parametrize("shape", [(1100, 256, 4096),   # 2.3 GB: passes of 1023 and 77 matrices
                                   (1030, 64, 64)])     # more than 1024 matrices of one tile
def test_stack_beyond_one_pass(hip_device, shape):
    """Stacks that span more than 2 GiB or hold more than 1024 matrices run in passes over
    one pass-sized workspace. Each matrix is independent, so every matrix of the whole
    stack equals, bit for bit, the same matrix run in a small stack of its own; sampled
    matrices on both sides of a pass boundary are also checked against the oracle."""
    from zmoe import ops

    E, m, n = shape
    G = make_stack(shape, 21, hip_device).to(torch.bfloat16)
    out = ops.newton_schulz5(G, 5)
    torch.cuda.synchronize()
    chunk = min(1024, (0x7FFF0000) // (m * n * 2))
    picks = sorted({0, chunk - 1, min(chunk, E - 1), E - 1})
    alone = ops.newton_schulz5(G[picks].contiguous(), 5)
    assert torch.equal(out[picks], alone), (shape, picks)
    for e in picks[:2] + picks[-1:]:
        got = out[e].float().cpu().numpy()
        ref = O.newton_schulz5(G[e].float().cpu().numpy()[None], 5)[0]
        assert rel_fro(got, ref) <= REL_FRO[5], (shape, e, rel_fro(got, ref))
