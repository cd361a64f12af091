"""The MLX checkpoint loader on CPU: names, fusion, validation (Q36/checkpoint/loader.py,
Q36/checkpoint/inventory.py) -- on synthetic checkpoints written in the mlx_lm layout."""

from __future__ import annotations

import json
import os

import pytest
import torch

from jitengine_amd import checkpoint
from jitengine_amd.checkpoint import CheckpointError
from tests.ckpt_util import config_dict, write_checkpoint


def _same(a, b):
    return a.dtype == b.dtype and a.shape == b.shape and torch.equal(a.cpu().view(torch.uint8),
                                                                      b.cpu().contiguous().view(torch.uint8))


@pytest.mark.parametrize("prefix", ["", "language_model."])
def test_load_fuses_and_keeps_bytes(tmp_path, prefix):
    cfg = config_dict()
    src = write_checkpoint(str(tmp_path), cfg, prefix=prefix)
    lm = checkpoint.load(str(tmp_path), "cpu", prepack=False)
    assert lm.vocab == 64 and lm.eos_ids == (63,) and len(lm.layers) == 2
    assert lm.cfg.hidden == 256 and lm.cfg.experts == 4 and lm.cfg.top_k == 2 and lm.cfg.inter == 64
    for i, layer in enumerate(lm.layers):
        p = f"model.layers.{i}."
        for part in ("weight", "scales", "biases"):
            qkv = torch.cat([src[p + f"self_attn.{m}_proj.{part}"] for m in "qkv"], 0)
            assert _same(getattr(layer.qkv, part), qkv)
            gu = torch.cat([src[p + f"mlp.switch_mlp.{m}_proj.{part}"] for m in ("gate", "up")], 1)
            assert _same(getattr(layer.moe.gate_up, part), gu)
            assert _same(getattr(layer.moe.down, part), src[p + f"mlp.switch_mlp.down_proj.{part}"])
            assert _same(getattr(layer.moe.router, part), src[p + f"mlp.gate.{part}"])
            assert _same(getattr(layer.o, part), src[p + f"self_attn.o_proj.{part}"])
        assert _same(layer.input_norm, src[p + "input_layernorm.weight"])
        assert _same(layer.k_norm, src[p + "self_attn.k_norm.weight"])
    assert _same(lm.embed.weight, src["model.embed_tokens.weight"])
    assert _same(lm.lm_head.scales, src["lm_head.scales"])
    assert _same(lm.final_norm, src["model.norm.weight"])


def test_tied_head_and_layer_limit(tmp_path):
    write_checkpoint(str(tmp_path), config_dict(tie=True, L=3))
    lm = checkpoint.load(str(tmp_path), "cpu", layers=1, prepack=False)
    assert lm.lm_head is lm.embed and len(lm.layers) == 1 and lm.cfg.layers == 1


@pytest.mark.parametrize("drop", [("partial_rotary_factor",), ("partial_rotary_factor", "rope_theta")])
def test_config_without_rope_keys_takes_the_reference_defaults(tmp_path, drop):
    """A config.json that leaves out the RoPE keys means the reference config's defaults
    (partial_rotary_factor 0.25, rope_theta 1e7): a quarter-head rotation, rejected, never silently
    read as a whole-head rotation at 1e6."""
    cfg = config_dict()
    for key in drop:
        del cfg[key]
    with open(os.path.join(tmp_path, "config.json"), "w") as f:
        json.dump(cfg, f)
    with pytest.raises(CheckpointError, match="partial_rotary_factor 0.25"):
        checkpoint.read_config(str(tmp_path))


def test_config_theta_default_is_the_reference_one(tmp_path):
    cfg = config_dict()
    del cfg["rope_theta"]
    with open(os.path.join(tmp_path, "config.json"), "w") as f:
        json.dump(cfg, f)
    assert checkpoint.read_config(str(tmp_path)).model.rope_theta == checkpoint.REF_ROPE_THETA == 1e7


@pytest.mark.parametrize("change, what", [
    ({"quantization": {"group_size": 64, "bits": 8}}, "bits=8"),
    ({"quantization": {"group_size": 32, "bits": 4}}, "group_size=32"),
    ({"quantization": {"group_size": 64, "bits": 4, "model.layers.0.mlp.gate": {"bits": 8, "group_size": 64}}},
     "model.layers.0.mlp.gate"),
    ({"quantization": {"group_size": 64, "bits": 4, "lm_head": False}}, "unquantized"),
    ({"head_dim": 64}, "head_dim 64"),
    ({"mlp_only_layers": [1]}, "dense MLP"),
    ({"layer_types": ["linear_attention", "full_attention"]}, "linear-attention"),
    ({"shared_expert_intermediate_size": 512}, "shared experts"),
    ({"partial_rotary_factor": 0.25}, "partial_rotary_factor"),
    ({"rope_parameters": {"rope_theta": 1e6, "partial_rotary_factor": 0.5}}, "partial_rotary_factor"),
    ({"rope_scaling": {"type": "yarn", "factor": 4.0}}, "RoPE scaling"),
    ({"rope_parameters": {"rope_theta": 1e6, "rope_type": "yarn"}}, "RoPE scaling"),
])
def test_config_rejections(tmp_path, change, what):
    cfg = config_dict()
    cfg.update(change)
    os.makedirs(tmp_path, exist_ok=True)
    with open(os.path.join(tmp_path, "config.json"), "w") as f:
        json.dump(cfg, f)
    with pytest.raises(CheckpointError, match=what):
        checkpoint.read_config(str(tmp_path))


def test_unquantized_and_missing_config(tmp_path):
    with pytest.raises(CheckpointError, match="does not exist"):
        checkpoint.read_config(str(tmp_path))
    cfg = config_dict()
    del cfg["quantization"]
    with open(os.path.join(tmp_path, "config.json"), "w") as f:
        json.dump(cfg, f)
    with pytest.raises(CheckpointError, match="not quantized"):
        checkpoint.read_config(str(tmp_path))


def test_missing_tensor_and_bad_dtype(tmp_path):
    write_checkpoint(str(tmp_path / "a"), config_dict(), drop=["model.layers.1.self_attn.k_norm.weight"])
    with pytest.raises(CheckpointError, match="model.layers.1.self_attn.k_norm.weight"):
        checkpoint.load(str(tmp_path / "a"), "cpu", prepack=False)
    write_checkpoint(str(tmp_path / "b"), config_dict(), drop=["lm_head.weight", "lm_head.scales", "lm_head.biases"])
    with pytest.raises(CheckpointError, match="lm_head"):
        checkpoint.load(str(tmp_path / "b"), "cpu", prepack=False)
    # a packed weight stored as I32 instead of U32
    from safetensors.torch import load_file, save_file
    write_checkpoint(str(tmp_path / "c"), config_dict(), shards=1)
    f = str(tmp_path / "c" / "model-00000.safetensors")
    d = load_file(f)
    d["model.layers.0.self_attn.o_proj.weight"] = d["model.layers.0.self_attn.o_proj.weight"].view(torch.int32)
    save_file(d, f)
    with pytest.raises(CheckpointError, match="U32"):
        checkpoint.load(str(tmp_path / "c"), "cpu", prepack=False)


def test_shape_mismatch(tmp_path):
    write_checkpoint(str(tmp_path), config_dict())
    cfg = json.load(open(tmp_path / "config.json"))
    cfg["moe_intermediate_size"] = 128  # the stacks on disk are 64 wide
    json.dump(cfg, open(tmp_path / "config.json", "w"))
    with pytest.raises(CheckpointError, match="switch_mlp.gate_proj"):
        checkpoint.load(str(tmp_path), "cpu", prepack=False)


def test_config_rope_parameters_and_generation_eos(tmp_path):
    """rope_parameters.rope_theta wins over a top-level rope_theta, and generation_config.json's stop
    tokens replace config.json's (Q36/model/config.py:91-103)."""
    cfg = config_dict()
    cfg["rope_theta"] = 5e5
    cfg["rope_parameters"] = {"rope_theta": 1e7, "rope_type": "default", "partial_rotary_factor": 1.0}
    cfg["eos_token_id"] = 7
    with open(os.path.join(tmp_path, "config.json"), "w") as f:
        json.dump(cfg, f)
    cc = checkpoint.read_config(str(tmp_path))
    assert cc.model.rope_theta == 1e7 and cc.eos_ids == (7,)
    with open(os.path.join(tmp_path, "generation_config.json"), "w") as f:
        json.dump({"eos_token_id": [3, 9]}, f)
    assert checkpoint.read_config(str(tmp_path)).eos_ids == (3, 9)
