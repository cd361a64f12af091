"""Synthetic MLX-layout checkpoints for the loader tests: config.json plus safetensors shards with
the sanitized mlx_lm names (un-fused q/k/v and gate/up, U32 packed weights, BF16 scales/biases)."""

from __future__ import annotations

import json
import os

import torch
from safetensors.torch import save_file

from jitengine_amd.quant import random_quantized


def config_dict(D=256, H=2, Hkv=1, E=4, k=2, I=64, V=64, L=2, tie=False, **extra):
    c = {"model_type": "qwen3_moe", "hidden_size": D, "num_attention_heads": H, "num_key_value_heads": Hkv,
         "head_dim": 128, "num_experts": E, "num_experts_per_tok": k, "moe_intermediate_size": I,
         "rope_theta": 1000000.0, "partial_rotary_factor": 1.0, "rms_norm_eps": 1e-6, "num_hidden_layers": L,
         "vocab_size": V, "norm_topk_prob": True, "tie_word_embeddings": tie, "decoder_sparse_step": 1, "mlp_only_layers": [],
         "eos_token_id": [V - 1], "quantization": {"group_size": 64, "bits": 4}}
    c.update(extra)
    return c


def write_checkpoint(path: str, cfg: dict, seed: int = 5, prefix: str = "", shards: int = 2, drop=(),
                     device="cpu") -> dict:
    """Write the checkpoint; returns {canonical name: tensor} of what was written (packed weights
    as int32 views)."""
    os.makedirs(path, exist_ok=True)
    D, H, Hkv, E, I, V = (cfg[k] for k in ("hidden_size", "num_attention_heads", "num_key_value_heads",
                                            "num_experts", "moe_intermediate_size", "vocab_size"))
    hd = cfg["head_dim"]
    out = {}
    n = [seed * 1000]

    def q(name, shape):
        n[0] += 1
        lin = random_quantized(shape, n[0], device=device)
        out[name + ".weight"], out[name + ".scales"], out[name + ".biases"] = lin.weight, lin.scales, lin.biases

    def vec(name, size):
        n[0] += 1
        g = torch.Generator(device=device)
        g.manual_seed(n[0])
        out[name] = (1.0 + 0.02 * torch.randn(size, generator=g, device=device)).to(torch.bfloat16)

    q("model.embed_tokens", (V, D))
    if not cfg.get("tie_word_embeddings"):
        q("lm_head", (V, D))
    vec("model.norm.weight", D)
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}."
        vec(p + "input_layernorm.weight", D)
        vec(p + "post_attention_layernorm.weight", D)
        q(p + "self_attn.q_proj", (H * hd, D))
        q(p + "self_attn.k_proj", (Hkv * hd, D))
        q(p + "self_attn.v_proj", (Hkv * hd, D))
        q(p + "self_attn.o_proj", (D, H * hd))
        vec(p + "self_attn.q_norm.weight", hd)
        vec(p + "self_attn.k_norm.weight", hd)
        q(p + "mlp.gate", (E, D))
        q(p + "mlp.switch_mlp.gate_proj", (E, I, D))
        q(p + "mlp.switch_mlp.up_proj", (E, I, D))
        q(p + "mlp.switch_mlp.down_proj", (E, D, I))
    for name in drop:
        out.pop(name)
    names = sorted(out)
    wm = {}
    for s in range(shards):
        part = {}
        for nm in names[s::shards]:
            t = out[nm].cpu()
            part[prefix + nm] = t.view(torch.uint32) if t.dtype == torch.int32 else t
            wm[prefix + nm] = f"model-{s:05d}.safetensors"
        if s == 0:  # tensors the loader must skip
            part["vision_tower.blocks.0.w"] = torch.zeros(4, dtype=torch.bfloat16)
            part[prefix + "mtp.layers.0.w"] = torch.zeros(4, dtype=torch.bfloat16)
            wm["vision_tower.blocks.0.w"] = wm[prefix + "mtp.layers.0.w"] = "model-00000.safetensors"
        save_file(part, os.path.join(path, f"model-{s:05d}.safetensors"))
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wm}, f)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg, f)
    return out
