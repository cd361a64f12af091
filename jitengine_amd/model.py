"""The decode step of the BASELINE geometry on the HIP kernels: decoder layers and decode_step.

Mirrors the reference's batched decode call chain (Q36/model/model.py:504-517 `decode_step` ->
`Qwen3_5MoeDecoderLayer.step` :77-80): input RMSNorm -> fused qkv projection -> q/k RMSNorm +
RoPE + KV append (Q36/model/attention.py:99-119, here into the paged pool) -> decode attention
(Q36/kernels/sdpa_decode.py:462-476, here paged split-K) -> o_proj -> residual -> post-attention
RMSNorm -> MoE block (Q36/model/moe.py:255-289) with the residual.  The geometry (Qwen3-MoE-style:
hidden 2048, 32 q / 4 kv heads of 128, 128 experts top-8 of intermediate 768, RoPE theta 1e6) has
no output gate and no shared expert.  Embedding and lm_head are outside the step.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import ops
from .moe import MoEBlock
from .quant import QLinear, random_quantized


@dataclass(frozen=True)
class MoEConfig:
    hidden: int = 2048
    heads: int = 32
    kv_heads: int = 4
    head_dim: int = 128
    experts: int = 128
    top_k: int = 8
    inter: int = 768
    rope_theta: float = 1e6
    eps: float = 1e-6
    layers: int = 48
    norm_topk: bool = True

    @property
    def qkv_rows(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim


def rope_inv_freq(theta: float, dims: int) -> np.ndarray:
    """fp32 inverse frequencies theta^(-2i/dims), i < dims/2 (evaluated in float64, rounded)."""
    return (float(theta) ** (-np.arange(0, dims, 2, dtype=np.float64) / dims)).astype(np.float32)


def random_layer_weights(cfg: MoEConfig, seed: int, device, std: float = 0.02) -> dict:
    """Synthetic weights of one layer: N(0, std) bf16 matrices quantized to 4-bit g64 (MLX
    layout) and RMSNorm weights 1 + N(0, std) in bf16; seeded, generated on `device`."""
    D, I, E = cfg.hidden, cfg.inter, cfg.experts
    gen = torch.Generator(device=device)
    gen.manual_seed(int(seed))

    def norm_w(n):
        return (1.0 + std * torch.randn(n, generator=gen, device=device)).to(torch.bfloat16)

    def stack(shape, s):
        parts = [random_quantized((min(16, shape[0] - e0), *shape[1:]), s * 1000 + e0, std, device)
                 for e0 in range(0, shape[0], 16)]
        return QLinear(torch.cat([p.weight for p in parts]), torch.cat([p.scales for p in parts]),
                       torch.cat([p.biases for p in parts]))

    return {
        "input_norm": norm_w(D),
        "qkv": random_quantized((cfg.qkv_rows, D), seed * 10 + 1, std, device),
        "q_norm": norm_w(cfg.head_dim),
        "k_norm": norm_w(cfg.head_dim),
        "o": random_quantized((D, cfg.heads * cfg.head_dim), seed * 10 + 2, std, device),
        "post_norm": norm_w(D),
        "router": random_quantized((E, D), seed * 10 + 3, std, device),
        "gate_up": stack((E, 2 * I, D), seed * 10 + 4),
        "down": stack((E, D, I), seed * 10 + 5),
    }


@dataclass
class StepState:
    """Per-step inputs shared by every layer: positions, page table, split plan, buffers."""

    pos: torch.Tensor          # int32 [B]: the position each row writes (its length so far)
    page_table: torch.Tensor   # int32 [B, max_pages]
    plan: ops.AttnPlan         # over lens = pos + 1
    workspace: torch.Tensor    # attention partials


def make_step_state(cfg: MoEConfig, pos_host, page_table: torch.Tensor) -> StepState:
    """Plan one decode step: row b writes position pos_host[b] and attends to pos + 1 keys (the
    plan and its workspace serve every layer of the step)."""
    pos_host = np.asarray(pos_host, np.int32)
    dev = page_table.device
    plan = ops.attn_plan(pos_host + 1, dev)
    ws = torch.empty(max(ops.attn_workspace_bytes(plan.total, cfg.heads), 4), dtype=torch.uint8, device=dev)
    return StepState(ops.upload(pos_host, dev), page_table, plan, ws)


@dataclass
class MixedState:
    """Per-step inputs of a mixed chunked-prefill + decode step.  Rows: the prefill chunks' tokens
    in chunk order, then one row per decode sequence.  Every row writes its K/V at pos_rows[r]
    through its own page-table row; the prefill rows attend causally over their sequence's keys,
    the decode rows over pos + 1 keys."""

    P: int                       # prefill rows (the first P rows)
    pos_rows: torch.Tensor       # int32 [T]
    table_rows: torch.Tensor     # int32 [T, max_pages]: row r's sequence's pages
    seq_table: torch.Tensor      # int32 [S, max_pages]: the prefill sequences' pages
    prefill: ops.PrefillPlan     # chunks (seq index into seq_table, ctx, length)
    dec_table: torch.Tensor      # int32 [D, max_pages]: the decode sequences' pages
    decode: ops.AttnPlan         # decode lens = pos + 1
    workspace: torch.Tensor


def make_mixed_state(cfg: MoEConfig, chunks, seq_table_host, dec_pos_host, dec_table_host, device) -> MixedState:
    """chunks [(seq, ctx, length)] over the rows of seq_table_host [S, max_pages]; decode sequence d
    writes position dec_pos_host[d] through dec_table_host[d] (both tables of equal width)."""
    seq_table_host = np.asarray(seq_table_host, np.int32)
    dec_table_host = np.asarray(dec_table_host, np.int32)
    dec_pos = np.asarray(dec_pos_host, np.int32)
    pos, rows = [], []
    for seq, ctx, length in chunks:
        pos += range(ctx, ctx + length)
        rows += [seq_table_host[seq]] * length
    P = len(pos)
    pos_rows = np.concatenate([np.asarray(pos, np.int32), dec_pos]).astype(np.int32)
    table_rows = np.concatenate([np.stack(rows) if rows else np.zeros((0, dec_table_host.shape[1]), np.int32),
                                 dec_table_host]).astype(np.int32)
    dplan = ops.attn_plan(dec_pos + 1, device)
    ws = torch.empty(max(ops.attn_workspace_bytes(dplan.total, cfg.heads), 4), dtype=torch.uint8, device=device)
    # (pinned, asynchronous uploads: the host does not wait for the steps still queued)
    return MixedState(P, ops.upload(pos_rows, device), ops.upload(table_rows, device),
                      ops.upload(seq_table_host, device), ops.prefill_plan(chunks, cfg.heads, cfg.kv_heads, device),
                      ops.upload(dec_table_host, device), dplan, ws)


class DecoderLayer:
    """One decoder layer over B ragged decode rows; weights stay resident (packed layout)."""

    def __init__(self, cfg: MoEConfig, w: dict, prepack: bool = True):
        self.cfg = cfg
        pk = ops.prepack if prepack else (lambda q: q)
        self.input_norm = w["input_norm"].contiguous()
        self.qkv = pk(w["qkv"])
        self.q_norm = w["q_norm"].contiguous()
        self.k_norm = w["k_norm"].contiguous()
        self.o = pk(w["o"])
        self.post_norm = w["post_norm"].contiguous()
        self.moe = MoEBlock(w["router"], w["gate_up"], w["down"], cfg.top_k, cfg.norm_topk, prepack=prepack)
        self.inv_freq = torch.from_numpy(rope_inv_freq(cfg.rope_theta, cfg.head_dim)).to(self.input_norm.device)

    def step(self, x: torch.Tensor, pool: torch.Tensor, st: StepState, debug: dict | None = None) -> torch.Tensor:
        """x [B, D] -> the layer's output rows (Q36/model/model.py:65-80 order: attention
        sub-block, residual, MoE sub-block, residual); `debug` receives every intermediate."""
        return self.run(x, pool, st, debug=debug)[0]

    def run(self, x: torch.Tensor | None, pool: torch.Tensor, st: StepState, xn: torch.Tensor | None = None,
            next_norm: torch.Tensor | None = None, debug: dict | None = None, carry: tuple | None = None,
            defer: bool = False):
        """(y, xn_next): the layer on rows x whose input norm xn = rmsnorm(x) may come from the
        previous layer; with next_norm (the next layer's input-norm weight) the closing combine
        also returns that layer's normed input in the same launch, else xn_next is None.

        One-token steps (the same bits, fewer launches): carry = (r, pk, scores, h) is the previous
        layer's combine left undone, run here with this layer's input norm inside the qkv
        projection (x is None then: the launch writes it); defer=True leaves this layer's combine
        undone and returns (None, carry) for the next layer to take in."""
        cfg = self.cfg
        moe = self.moe
        if carry is not None:
            r0, pk0, sc0, h0 = carry
            x, qkv = ops.qmm_combine_rmsnorm(r0, pk0, sc0, h0, self.input_norm, cfg.eps, self.qkv)
        else:
            if xn is None:
                xn = ops.rmsnorm(x, self.input_norm, cfg.eps)
            # decode rows take the decode kernels at any batch size (seg=False): a row's bits never
            # depend on how many other rows the step carries
            qkv = ops.qmm(xn, self.qkv, seg=False)
        B = x.shape[0]
        if defer and B != 1:
            raise ValueError("defer takes a one-token step")
        scale = cfg.head_dim ** -0.5
        if debug is None:  # q/k norm + RoPE + append inside the attention launch (the same bits)
            q = None
            attn = ops.paged_decode_attention_qkv(qkv, cfg.heads, cfg.kv_heads, self.q_norm, self.k_norm, cfg.eps,
                                                  self.inv_freq, pool, st.page_table, st.plan, scale, st.workspace)
        else:  # the two launches, which also show q
            q = ops.qk_norm_rope_append(qkv, cfg.heads, cfg.kv_heads, self.q_norm, self.k_norm, cfg.eps,
                                        self.inv_freq, st.pos, st.page_table, pool)
            attn = ops.paged_decode_attention(q, pool, st.page_table, st.plan, scale, st.workspace)
        o = ops.qmm(attn.view(B, -1), self.o, seg=False)
        if B == 1 and ops.row_prologue_fits(moe.router, cfg.hidden):  # the add + norm inside the router launch
            logits, h, hn = ops.qmm_add_rmsnorm(o, x, self.post_norm, cfg.eps, moe.router)
        else:
            hn, h = ops.rmsnorm(o, self.post_norm, cfg.eps, resid=x, return_sum=True)
            logits = ops.qmm(hn, moe.router, seg=False)
        E, k = moe.num_experts, moe.top_k
        if B == 1 and isinstance(moe.gate_up, ops.PackedQ4) and E % 32 == 0 and E <= 128 and k < E and k <= 64:
            # one token: its top-k and packing inside the gate||up launch (the same bits)
            inds, scores, pk, hh = ops.route_gate_up(hn, logits, moe.gate_up, k, moe.norm_topk)
            r = ops.expert_down(hh, moe.down, pk)
        else:
            if B <= ops.ROUTE_PACK_MAX_ROWS and E <= 128:  # one launch for a small step
                inds, scores, pk = ops.route_pack(logits, k, moe.norm_topk)
            else:
                inds, scores = ops.router_topk(logits, k, moe.norm_topk)
                pk = ops.moe_pack(inds, E)
            hh, r = moe.expert_mlp(hn, pk)
        if defer:
            y, xn_next = None, None
        elif next_norm is None:
            y, xn_next = ops.moe_combine(r, pk, scores, h), None
        else:
            y, xn_next = ops.moe_combine_rmsnorm(r, pk, scores, h, next_norm, cfg.eps)
        if debug is not None:
            debug.update(x=x, xn=xn, qkv=qkv, q=q, attn=attn, o=o, h=h, hn=hn, logits=logits, inds=inds,
                         scores=scores, pk=pk, hh=hh, r=r, y=y)
        if defer:
            return None, (r, pk, scores, h)
        return y, xn_next


    def mixed(self, x: torch.Tensor, pool: torch.Tensor, ms: MixedState, debug: dict | None = None) -> torch.Tensor:
        """One mixed chunked-prefill + decode step of the layer over rows x [T, D]: the decode
        step's block with the prefill rows' attention causal over their chunks
        (Q36/model/attention.py:70-74) and the MoE on the segment GEMM when the batch is long
        (Q36/model/moe.py:161-190)."""
        cfg = self.cfg
        T = x.shape[0]
        xn = ops.rmsnorm(x, self.input_norm, cfg.eps)
        qkv = ops.qmm(xn, self.qkv)
        q = ops.qk_norm_rope_append(qkv, cfg.heads, cfg.kv_heads, self.q_norm, self.k_norm, cfg.eps,
                                    self.inv_freq, ms.pos_rows, ms.table_rows, pool)
        scale = cfg.head_dim ** -0.5
        parts = []
        if ms.P:
            parts.append(ops.paged_prefill_attention(q[:ms.P], pool, ms.seq_table, ms.prefill, scale))
        if T > ms.P:
            parts.append(ops.paged_decode_attention(q[ms.P:], pool, ms.dec_table, ms.decode, scale, ms.workspace))
        attn = torch.cat(parts) if len(parts) > 1 else parts[0]
        o = ops.qmm(attn.view(T, -1), self.o)
        hn, h = ops.rmsnorm(o, self.post_norm, cfg.eps, resid=x, return_sum=True)
        moe = self.moe
        logits = ops.qmm(hn, moe.router)
        inds, scores = ops.router_topk(logits, moe.top_k, moe.norm_topk)
        pk = ops.moe_pack(inds, moe.num_experts)
        hh, r = moe.expert_mlp(hn, pk, prefill=True)
        y = ops.moe_combine(r, pk, scores, h)
        if debug is not None:
            debug.update(x=x, xn=xn, qkv=qkv, q=q, attn=attn, o=o, h=h, hn=hn, logits=logits, inds=inds,
                         scores=scores, pk=pk, hh=hh, r=r, y=y)
        return y


class Model:
    """A stack of decoder layers and the ragged batched decode step."""

    def __init__(self, cfg: MoEConfig, layer_weights: list, prepack: bool = True):
        self.cfg = cfg
        self.layers = [DecoderLayer(cfg, w, prepack) for w in layer_weights]

    def make_state(self, pos_host, page_table: torch.Tensor) -> StepState:
        return make_step_state(self.cfg, pos_host, page_table)

    def decode_step(self, x: torch.Tensor, pools: list, st: StepState) -> torch.Tensor:
        """x [B, D] bf16 hidden rows -> the last layer's output rows; pools[l] is layer l's KV pool."""
        one = x.shape[0] == 1
        xn, carry = None, None
        for i, (layer, pool) in enumerate(zip(self.layers, pools)):
            nxt = self.layers[i + 1] if i + 1 < len(self.layers) else None
            # one token: the layer's combine runs inside the next layer's qkv launch
            defer = one and nxt is not None and ops.row_prologue_fits(nxt.qkv, self.cfg.hidden)
            y, out = layer.run(x, pool, st, xn=xn, carry=carry, defer=defer,
                               next_norm=None if (defer or nxt is None) else nxt.input_norm)
            x, xn, carry = (None, None, out) if defer else (y, out, None)
        return x


class CausalLM:
    """The whole model around the decoder stack: 4-bit embedding table, final RMSNorm, 4-bit lm_head
    and the greedy draw (Q36/model/model.py:248-270 `forward`: embed.lookup -> layers -> norm ->
    lm_head; Q36/sampler.py:371-374 with temperature 0).  A tied head reads the embedding table."""

    def __init__(self, model: Model, embed: QLinear, final_norm: torch.Tensor, lm_head: QLinear, vocab: int,
                 eos_ids=(), prepack: bool = True):
        embed.validate()
        if embed.weight.dim() != 2 or embed.out_dims != vocab or embed.in_dims != model.cfg.hidden:
            raise ValueError(f"embedding table must be [{vocab}, {model.cfg.hidden}]")
        if lm_head.out_dims != vocab or lm_head.in_dims != model.cfg.hidden:
            raise ValueError(f"lm_head must be [{vocab}, {model.cfg.hidden}]")
        self.model, self.cfg = model, model.cfg
        self.embed = embed
        self.final_norm = final_norm.contiguous()
        self.lm_head = ops.prepack(lm_head) if prepack else lm_head
        self.vocab = int(vocab)
        self.eos_ids = tuple(int(e) for e in eos_ids)

    @property
    def layers(self) -> list:
        return self.model.layers

    def embed_tokens(self, ids: torch.Tensor) -> torch.Tensor:
        """ids int32 [B] -> hidden rows [B, D] bf16."""
        return ops.embed_q4(ids, self.embed)

    def logits(self, h: torch.Tensor) -> torch.Tensor:
        """Last-layer rows [B, D] -> logits [B, V] bf16 (the decode kernel at any row count, so a row's
        logits do not depend on the batch)."""
        return ops.qmm(ops.rmsnorm(h, self.final_norm, self.cfg.eps), self.lm_head, seg=False)

    def greedy(self, h: torch.Tensor) -> torch.Tensor:
        """Last-layer rows -> the greedy token of each row, int32 [B]."""
        return ops.argmax_rows(self.logits(h))


def random_causal_lm(cfg: MoEConfig, vocab: int, seed: int, device, std: float = 0.02,
                     prepack: bool = True) -> CausalLM:
    """A seeded synthetic model of the geometry: random_layer_weights per layer, an N(0, std)
    embedding table and lm_head quantized to 4-bit, a final norm 1 + N(0, std)."""
    layers = [random_layer_weights(cfg, seed * 100 + l, device, std) for l in range(cfg.layers)]
    model = Model(cfg, layers, prepack)
    gen = torch.Generator(device=device)
    gen.manual_seed(int(seed) * 7 + 3)
    final_norm = (1.0 + std * torch.randn(cfg.hidden, generator=gen, device=device)).to(torch.bfloat16)
    embed = random_quantized((vocab, cfg.hidden), seed * 10 + 8, std, device)
    head = random_quantized((vocab, cfg.hidden), seed * 10 + 9, std, device)
    return CausalLM(model, embed, final_norm, head, vocab, (), prepack)
