"""MLX 4-bit checkpoints of the Qwen3-MoE geometry: config, validation and loading.

Reads the sanitized mlx_lm layout the reference loads (Q36/checkpoint/loader.py:21-65;
header-only validation in Q36/checkpoint/inventory.py): safetensors shards listed by
`model.safetensors.index.json` (or every `*.safetensors`), tensor names with an optional
`language_model.` prefix, quantized modules as `<name>.weight` U32 [out, in / 8] +
`<name>.scales` / `<name>.biases` BF16 [out, in / 64], expert stacks as
`mlp.switch_mlp.{gate,up,down}_proj` [E, out, in / 8].  Vision and multi-token-prediction
tensors are skipped as the reference's loader skips them.

Only what the HIP path computes is accepted: every layer full attention with q/k RMSNorm and a
routed MoE (no shared expert, no dense MLP layers), affine 4-bit group-64 quantization for every
matrix, head_dim 128.  Anything else raises CheckpointError naming what is wrong, before any
tensor is read, as the reference's inventory does (Q36/checkpoint/inventory.py:40-66,101-120).
"""

from __future__ import annotations

import dataclasses
import glob
import json
import os
from dataclasses import dataclass

import torch

from .model import MoEConfig
from .quant import QLinear

LANG_PREFIX = "language_model."
VISION_PREFIXES = ("vision_tower.", "model.visual.", "visual.")


class CheckpointError(ValueError):
    """The checkpoint is not one this build can serve (the message says why)."""


# The reference config's RoPE defaults, used when config.json names neither key
# (Qwen3_5MoeConfig.rope_theta / partial_rotary_factor, Q36/model/config.py:22-23).
REF_ROPE_THETA = 1e7
REF_PARTIAL_ROTARY = 0.25


@dataclass(frozen=True)
class CheckpointConfig:
    model: MoEConfig
    vocab: int
    tie_embeddings: bool
    eos_ids: tuple


def canonical(name: str) -> str:
    """Strip the vision-language conversion's `language_model.` prefix."""
    return name[len(LANG_PREFIX):] if name.startswith(LANG_PREFIX) else name


def _skipped(name: str) -> bool:
    c = canonical(name)
    return name.startswith(VISION_PREFIXES) or c.startswith("mtp.") or ".mtp." in c or c.startswith("model.mtp")


def read_config(model_path: str) -> CheckpointConfig:
    """Parse and validate config.json (a `text_config` block, when present, holds the language
    model's fields)."""
    path = os.path.join(model_path, "config.json")
    try:
        with open(path) as f:
            raw = json.load(f)
    except FileNotFoundError:
        raise CheckpointError(f"{path} does not exist") from None
    t = dict(raw.get("text_config") or raw)
    q = raw.get("quantization") or raw.get("quantization_config") or t.get("quantization")
    if not q:
        raise CheckpointError("the checkpoint is not quantized (this build serves MLX 4-bit affine)")
    if not isinstance(q, dict):
        raise CheckpointError("quantization block is not an object")
    bits, group, mode = q.get("bits"), q.get("group_size"), q.get("mode", "affine")
    if bits != 4 or group != 64 or mode != "affine":
        raise CheckpointError(f"quantization bits={bits} group_size={group} mode={mode!r}: only 4-bit affine "
                              "group 64 is served")
    for k, v in q.items():
        if isinstance(v, dict) and (v.get("bits", 4) != 4 or v.get("group_size", 64) != 64
                                    or v.get("mode", "affine") != "affine"):
            raise CheckpointError(f"{canonical(k)}: quantization override {v} (only 4-bit affine group 64 is served)")
        if v is False:
            raise CheckpointError(f"{canonical(k)} is left unquantized (only 4-bit matrices are served)")

    def need(key):
        if key not in t:
            raise CheckpointError(f"config lacks {key!r}")
        return t[key]

    L = int(need("num_hidden_layers"))
    H, Hkv = int(need("num_attention_heads")), int(need("num_key_value_heads"))
    D = int(need("hidden_size"))
    hd = int(t.get("head_dim", D // H))
    if hd != 128:
        raise CheckpointError(f"head_dim {hd}: the attention kernels serve 128")
    if t.get("mlp_only_layers") or int(t.get("decoder_sparse_step", 1)) != 1:
        raise CheckpointError("dense MLP layers are not served (every layer must be a routed MoE)")
    types = t.get("layer_types")
    if types and any(x != "full_attention" for x in types):
        raise CheckpointError("linear-attention layers are not served (every layer must be full attention)")
    if int(t.get("shared_expert_intermediate_size", 0) or 0):
        raise CheckpointError("shared experts are not served")
    # RoPE as the reference reads it (Q36/model/config.py:91-95): rope_parameters first, then the
    # top-level keys, then the reference config's defaults (rope_theta 1e7, partial_rotary_factor
    # 0.25; Q36/model/config.py:22-23) -- so a config.json that names neither key means a quarter-head
    # rotation at 1e7, which the kernels do not serve.  They rotate the whole head with plain
    # frequencies only.
    rp = t.get("rope_parameters") or {}
    if not isinstance(rp, dict):
        raise CheckpointError("rope_parameters is not an object")
    theta = float(rp.get("rope_theta", t.get("rope_theta", REF_ROPE_THETA)))
    prf = float(rp.get("partial_rotary_factor", t.get("partial_rotary_factor", REF_PARTIAL_ROTARY)))
    if prf != 1.0:
        raise CheckpointError(f"partial_rotary_factor {prf}: the kernels rotate the whole head (1.0)")
    scaling = t.get("rope_scaling") or rp.get("rope_scaling")
    rtype = rp.get("rope_type", rp.get("type", "default"))
    if scaling or rtype not in ("default", None):
        raise CheckpointError(f"RoPE scaling ({scaling or rtype}) is not served: plain RoPE frequencies only")
    cfg = MoEConfig(hidden=D, heads=H, kv_heads=Hkv, head_dim=hd, experts=int(need("num_experts")),
                    top_k=int(need("num_experts_per_tok")), inter=int(need("moe_intermediate_size")),
                    rope_theta=theta, eps=float(t.get("rms_norm_eps", 1e-6)),
                    layers=L, norm_topk=bool(t.get("norm_topk_prob", True)))
    # stop tokens: config.json's, replaced by generation_config.json's when that file names them
    # (the reference's order, Q36/model/config.py:98-103)
    eos = raw.get("eos_token_id", t.get("eos_token_id", ()))
    gen_path = os.path.join(model_path, "generation_config.json")
    if os.path.exists(gen_path):
        try:
            with open(gen_path) as f:
                g = json.load(f)
        except ValueError as exc:
            raise CheckpointError(f"{gen_path} is not valid JSON: {exc}") from None
        eos = g.get("eos_token_id", eos)
    eos = tuple(int(e) for e in (eos if isinstance(eos, (list, tuple)) else [eos]) if e is not None)
    return CheckpointConfig(cfg, int(need("vocab_size")),
                            bool(raw.get("tie_word_embeddings", t.get("tie_word_embeddings", False))), eos)


def shard_files(model_path: str) -> list:
    idx = os.path.join(model_path, "model.safetensors.index.json")
    if os.path.exists(idx):
        with open(idx) as f:
            files = sorted({os.path.join(model_path, v) for v in json.load(f)["weight_map"].values()})
        if files:
            return files
    return sorted(glob.glob(os.path.join(model_path, "*.safetensors")))


class _Tensors:
    """Lazy name -> tensor access over the shards (each tensor read when first asked for)."""

    def __init__(self, model_path: str):
        from safetensors import safe_open

        self.where = {}
        self._open = {}
        files = shard_files(model_path)
        if not files:
            raise CheckpointError(f"no safetensors shards under {model_path}")
        for path in files:
            h = safe_open(path, framework="pt", device="cpu")
            self._open[path] = h
            for k in h.keys():
                if not _skipped(k):
                    self.where[canonical(k)] = (path, k)

    def has(self, name: str) -> bool:
        return name in self.where

    def get(self, name: str) -> torch.Tensor:
        if name not in self.where:
            raise CheckpointError(f"missing tensor {name!r}")
        path, raw = self.where[name]
        return self._open[path].get_tensor(raw)


def _quant(ts: _Tensors, name: str, shape: tuple, device) -> QLinear:
    """The quantized module `name` with logical shape (..., out, in), validated."""
    w, s, b = ts.get(name + ".weight"), ts.get(name + ".scales"), ts.get(name + ".biases")
    *lead, n, k = shape
    if w.dtype != torch.uint32:
        raise CheckpointError(f"{name}.weight is {w.dtype}, packed weights are U32")
    if s.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise CheckpointError(f"{name}.scales/.biases must be BF16")
    if tuple(w.shape) != (*lead, n, k // 8) or tuple(s.shape) != (*lead, n, k // 64) or s.shape != b.shape:
        raise CheckpointError(f"{name}: weight {tuple(w.shape)} scales {tuple(s.shape)} do not fit a 4-bit g64 "
                              f"matrix {tuple(shape)}")
    return QLinear(w.view(torch.int32).contiguous().to(device), s.contiguous().to(device),
                   b.contiguous().to(device))


def _vec(ts: _Tensors, name: str, n: int, device) -> torch.Tensor:
    t = ts.get(name)
    if tuple(t.shape) != (n,):
        raise CheckpointError(f"{name} is {tuple(t.shape)}, expected ({n},)")
    return t.to(torch.bfloat16).contiguous().to(device)


def _cat(parts: list) -> QLinear:
    """Fuse quantized matrices along the output rows (the last-but-one axis)."""
    return QLinear(torch.cat([p.weight for p in parts], -2).contiguous(),
                   torch.cat([p.scales for p in parts], -2).contiguous(),
                   torch.cat([p.biases for p in parts], -2).contiguous())


def layer_weights(ts: _Tensors, cfg: MoEConfig, i: int, device) -> dict:
    """Layer i's weights in this build's fused form: q, k, v rows concatenated into one qkv matrix
    [(H + 2 Hkv) * 128, D] and each expert's gate and up rows into one gate||up stack [E, 2I, D]."""
    D, H, Hkv, hd, E, I = cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.experts, cfg.inter
    p = f"model.layers.{i}."
    a, m = p + "self_attn.", p + "mlp."
    if ts.has(m + "shared_expert.gate_proj.weight"):
        raise CheckpointError(f"layer {i} has a shared expert (not served)")
    return {
        "input_norm": _vec(ts, p + "input_layernorm.weight", D, device),
        "qkv": _cat([_quant(ts, a + "q_proj", (H * hd, D), device), _quant(ts, a + "k_proj", (Hkv * hd, D), device),
                     _quant(ts, a + "v_proj", (Hkv * hd, D), device)]),
        "q_norm": _vec(ts, a + "q_norm.weight", hd, device),
        "k_norm": _vec(ts, a + "k_norm.weight", hd, device),
        "o": _quant(ts, a + "o_proj", (D, H * hd), device),
        "post_norm": _vec(ts, p + "post_attention_layernorm.weight", D, device),
        "router": _quant(ts, m + "gate", (E, D), device),
        "gate_up": _cat([_quant(ts, m + "switch_mlp.gate_proj", (E, I, D), device),
                         _quant(ts, m + "switch_mlp.up_proj", (E, I, D), device)]),
        "down": _quant(ts, m + "switch_mlp.down_proj", (E, D, I), device),
    }


def load(model_path: str, device, layers: int | None = None, prepack: bool = True):
    """The checkpoint as a CausalLM on `device` (the first `layers` layers when given), loaded layer
    by layer so no layer is resident twice."""
    from .model import CausalLM, DecoderLayer, Model

    cc = read_config(model_path)
    cfg = cc.model if layers is None else dataclasses.replace(cc.model, layers=int(layers))
    ts = _Tensors(model_path)
    D, V = cfg.hidden, cc.vocab
    embed = _quant(ts, "model.embed_tokens", (V, D), device)
    if ts.has("lm_head.weight"):
        head = _quant(ts, "lm_head", (V, D), device)
    elif cc.tie_embeddings:
        head = embed
    else:
        raise CheckpointError("missing tensor 'lm_head.weight' (and the embeddings are not tied)")
    model = Model.__new__(Model)
    model.cfg, model.layers = cfg, []
    for i in range(cfg.layers):
        model.layers.append(DecoderLayer(cfg, layer_weights(ts, cfg, i, device), prepack))
    return CausalLM(model, embed, _vec(ts, "model.norm.weight", D, device), head, V, cc.eos_ids, prepack)
