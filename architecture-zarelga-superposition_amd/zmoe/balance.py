"""Aux-loss-free load balancing and MoE load metrics on the GPU.

Drop-in counterparts of the reference's trainer-side helpers:

* ``auxillary_loss_free_update(model, all_topk_indices, update_rate, attention_mask=None)``
  (main.py:161-175): ``b += update_rate * sign(mean(counts) - counts)`` per MoE layer, over
  the valid tokens only. Counts come from the HIP histogram (``zmoe_bincount``), the
  update from ``zmoe_bias_update``; nothing syncs the host.
* ``log_moe_metrics(moe_layers, all_topk_indices, step, attention_mask=None)``
  (utils/trainutils.py:110-142, the method body with the registered ``(layer_idx, gate)``
  list passed in): the same four metrics per layer under the same keys, read back with one
  host transfer for all layers instead of four ``.item()`` calls per layer.
* ``update_biases_from_layers(moe_layers, update_rate)``: the same bias update from the
  expert offsets the routed experts' sort already produced in the last forward
  (``GLUMLP.last_expert_offsets``), so no pass over topk_idx at all. It equals the
  reference's masked update when the layer saw only valid tokens (the unpadded path, or no
  padding); with padded inputs use ``auxillary_loss_free_update`` and the mask.
"""

from __future__ import annotations

from typing import Dict, Iterable, Optional, Sequence, Tuple

import torch

from . import ops


def expert_counts(topk_idx: torch.Tensor, n_experts: int, valid: Optional[torch.Tensor] = None) -> torch.Tensor:
    """bincount(topk_idx[valid].flatten(), minlength=E) as int64 [E] on the device."""
    if valid is not None:
        topk_idx = topk_idx[valid]
    return ops.bincount(topk_idx.reshape(-1), n_experts)


def auxillary_loss_free_update(model, all_topk_indices: Sequence[torch.Tensor], update_rate: float,
                               attention_mask: Optional[torch.Tensor] = None) -> None:
    valid = attention_mask.bool() if attention_mask is not None else None
    with torch.no_grad():
        for layer_idx, topk_idx in enumerate(all_topk_indices):
            idx = topk_idx[valid] if valid is not None else topk_idx
            if idx.numel() == 0:  # main.py:170-171
                continue
            gate = model.layers[layer_idx].mlp.gate
            counts = ops.bincount(idx.reshape(-1), gate.n_routed_experts)
            ops.bias_update_(gate.expert_biases, torch.cumsum(counts, 0), update_rate)


def update_biases_from_layers(moe_layers: Iterable, update_rate: float) -> None:
    """Bias update for each MoELayer from the offsets its last forward's sort produced."""
    with torch.no_grad():
        for layer in moe_layers:
            off = getattr(layer.routed_experts, "last_expert_offsets", None)
            if off is None:
                raise RuntimeError("update_biases_from_layers: the layer has not run a forward pass")
            ops.bias_update_(layer.gate.expert_biases, off, update_rate)


def moe_load_metrics(counts: torch.Tensor, total: int) -> Dict[str, torch.Tensor]:
    """utils/trainutils.py:124-135 from an expert histogram: 0-d float tensors, on the device."""
    E = counts.numel()
    c = counts.float()
    expected = total / E
    return {
        "pct_experts_used": 100.0 * (counts > 0).sum().float() / E,
        "load_imbalance": (c / expected - 1.0).abs().mean(),
        "max_expert_pct": c.max() * 100.0 / total,
        "min_expert_pct": c.min() * 100.0 / total,
    }


def log_moe_metrics(moe_layers: Sequence[Tuple[int, torch.nn.Module]], all_topk_indices: Sequence[torch.Tensor],
                    step: int, attention_mask: Optional[torch.Tensor] = None) -> Dict[str, float]:
    del step  # the reference takes it for its logger; the values do not depend on it
    if not moe_layers or not all_topk_indices:
        return {}
    valid = attention_mask.bool() if attention_mask is not None else None
    keys, vals = [], []
    for (layer_idx, gate), topk_idx in zip(moe_layers, all_topk_indices):
        idx = topk_idx[valid] if valid is not None else topk_idx
        if idx.numel() == 0:
            continue
        m = moe_load_metrics(ops.bincount(idx.reshape(-1), gate.n_routed_experts), idx.numel())
        for name in ("pct_experts_used", "load_imbalance", "max_expert_pct", "min_expert_pct"):
            keys.append(f"experts/layer_{layer_idx}_{name}")
            vals.append(m[name])
    if not vals:
        return {}
    return dict(zip(keys, torch.stack(vals).tolist()))
