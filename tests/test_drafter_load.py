"""Drafter checkpoint reading (host only): ParallelDrafter's parameter names
(src/pe/drafter.py:62-76, src/pe/nn.py:59-117) mapped to DeviceDrafter's layout."""
import pytest
import torch

from parallel_eagle_amd.drafter import _LAYER_KEYS, weights_from_state_dict


def _sd(n_layers, h=8):
    sd = {"feat_norm.weight": torch.ones(h), "feat_proj.weight": torch.randn(h, 3 * h),
          "in_proj.weight": torch.randn(h, 2 * h), "mask_emb": torch.randn(h), "h_shared": torch.randn(h)}
    for i in range(n_layers):
        for theirs in _LAYER_KEYS.values():
            sd[f"layers.{i}.{theirs}"] = torch.randn(h, h)
    return sd


def test_state_dict_names_map_to_the_layout():
    sd = _sd(2)
    w = weights_from_state_dict(sd, 2)
    assert w["in_proj"] is sd["in_proj.weight"] and w["mask_emb"] is sd["mask_emb"]
    assert len(w["layers"]) == 2
    assert w["layers"][1]["q"] is sd["layers.1.attn.q_proj.weight"]
    assert w["layers"][0]["attn_norm"] is sd["layers.0.input_norm.weight"]
    assert w["layers"][0]["mlp_norm"] is sd["layers.0.post_norm.weight"]
    assert w["layers"][1]["down"] is sd["layers.1.mlp.down_proj.weight"]


def test_checkpoint_round_trip_through_a_safe_load(tmp_path):
    sd = _sd(1)
    path = tmp_path / "drafter.pt"
    torch.save({"state_dict": sd, "num_layers": 1, "max_depth": 5, "target_name": "x"}, path)
    ck = torch.load(path, map_location="cpu", weights_only=True)
    w = weights_from_state_dict(ck["state_dict"], ck["num_layers"])
    assert torch.equal(w["layers"][0]["gate"], sd["layers.0.mlp.gate_proj.weight"])


def test_missing_parameter_is_named():
    sd = _sd(2)
    del sd["layers.1.attn.v_proj.weight"]
    with pytest.raises(KeyError, match="layers.1.attn.v_proj.weight"):
        weights_from_state_dict(sd, 2)
