"""Newton-Schulz orthogonalisation for the MuonMD step (reference optimizer/muon.py).

``zeropower_via_newtonschulz5(G, steps)`` has the reference's signature and result
(muon.py:6-32): a bf16 tensor of G's shape, each trailing matrix driven towards
U S' V^T. It runs as one C-ABI call (``zmoe_newton_schulz5``): a deterministic
Frobenius normalisation, then per step three grouped bf16 MFMA GEMMs whose
epilogues also form the scaled and summed terms, so a step has no separate
elementwise passes. The reference's ``md_decoupled_step`` (muon.py:399-508) calls
the function by its module-global name at :449, so binding this one in that
module's namespace routes the expert stacks' orthogonalisation here.
"""

from __future__ import annotations

import torch

from . import ops

NS_COEFFS = ops.NS_COEFFS


def zeropower_via_newtonschulz5(G: torch.Tensor, steps: int) -> torch.Tensor:
    assert G.ndim >= 2  # muon.py:17
    return ops.newton_schulz5(G, steps, NS_COEFFS)
