"""Checkpoint compatibility of the MoE layer (CPU).

The reference saves ``model.state_dict()`` with safetensors (utils/trainutils.py:33-43);
the MoE sublayer sits under ``layers.{i}.mlp``. Its keys, shapes and dtypes here must be
the reference's, so checkpoints load both ways:

  gate.weight                          [E, d]      moe_gate.py:15
  gate.expert_biases                   [E] fp32    moe_gate.py:16 (persistent buffer)
  shared_experts.gate_proj.weight      [fs, d]     expert_layer.py:12-14
  shared_experts.up_proj.weight        [fs, d]
  shared_experts.down_proj.weight      [d, fs]
  routed_experts.experts.weight        [E, 2f, d]  mlp.py:58 + parallel_experts.py:152
  routed_experts.output_experts.weight [E, d, f]   mlp.py:59

with fs = intermediate_size * n_shared_experts (moe_layer.py:18-19; 0 reads as f,
expert_layer.py:10).
"""

import pytest
import torch
from safetensors.torch import load_file, save_file


def reference_layout(d, f, E, n_shared):
    fs = f * n_shared or f
    return {
        "gate.weight": (E, d),
        "gate.expert_biases": (E,),
        "shared_experts.gate_proj.weight": (fs, d),
        "shared_experts.up_proj.weight": (fs, d),
        "shared_experts.down_proj.weight": (d, fs),
        "routed_experts.experts.weight": (E, 2 * f, d),
        "routed_experts.output_experts.weight": (E, d, f),
    }


def make_layer(d, f, E, k, n_shared):
    from modeling.model_config import ModelConfig
    from modeling.moe_layer import MoELayer

    cfg = ModelConfig(hidden_size=d, intermediate_size=f, n_experts=E + n_shared, n_shared_experts=n_shared,
                      n_experts_per_token=k)
    return MoELayer(cfg)


@pytest.mark.parametrize("d,f,E,k,n_shared", [(256, 512, 8, 2, 0), (2048, 768, 128, 8, 2), (64, 32, 4, 2, 1)])
def test_state_dict_keys_shapes_dtypes(d, f, E, k, n_shared):
    sd = make_layer(d, f, E, k, n_shared).state_dict()
    want = reference_layout(d, f, E, n_shared)
    assert set(sd) == set(want)
    for key, shape in want.items():
        assert tuple(sd[key].shape) == shape, key
        assert sd[key].dtype == torch.float32, key


def test_safetensors_round_trip_under_model_prefix(tmp_path):
    torch.manual_seed(0)
    layer = make_layer(64, 32, 4, 2, 1)
    with torch.no_grad():
        layer.gate.expert_biases.normal_()
    sd = {f"layers.3.mlp.{k}": v.contiguous() for k, v in layer.state_dict().items()}
    path = tmp_path / "checkpoint.safetensors"
    save_file(sd, str(path))
    loaded = load_file(str(path))
    fresh = make_layer(64, 32, 4, 2, 1)
    prefix = "layers.3.mlp."
    missing, unexpected = fresh.load_state_dict({k[len(prefix):]: v for k, v in loaded.items()}, strict=True)
    assert not missing and not unexpected
    for k, v in layer.state_dict().items():
        assert torch.equal(fresh.state_dict()[k], v), k


def test_runtime_attributes_stay_out_of_the_state_dict():
    layer = make_layer(64, 32, 4, 2, 1)
    layer.routed_experts.last_expert_offsets = torch.arange(4)
    assert "routed_experts.last_expert_offsets" not in layer.state_dict()
