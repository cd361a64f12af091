"""The hot path's operators registered with torch as torch.ops.jitengine.* (torch.library custom
ops), the form the survey of the reference names for this boundary: the same C-ABI calls as
jitengine_amd.ops, each with a fake kernel that gives its output shapes and dtypes without
running it, so that torch.compile traces through the operators instead of breaking its graph at
an opaque ctypes call, and meta/fake tensors propagate through them.

Host-side structures of jitengine_amd.ops are passed as their tensors and sizes:
  * a packed 4-bit matrix or expert stack (ops.PackedQ4) as its uint8 tensor and (E, N, K);
  * the packing tables (ops.Packing) as the single int32 buffer moe_pack returns, with (k, E);
  * a decode attention plan (ops.AttnPlan) as its three int32 tensors, its chunk count and the
    longest sequence (plan_args);
  * a prefill plan (ops.PrefillPlan) as its two int32 tables, its chunks flattened into (seq, ctx,
    length) triples, its most key parts of a token and its longest chunk (prefill_plan_args).
Importing this module registers the operators; it needs the HIP library only when one runs.
"""

from __future__ import annotations

import numpy as np
import torch

from . import ops

_NS = "jitengine"


def _packed(data: torch.Tensor, E: int, N: int, K: int) -> ops.PackedQ4:
    return ops.PackedQ4(data, E, N, K, E > 1)


def packing_from_buffer(buf: torch.Tensor, k: int, E: int) -> ops.Packing:
    """The packing tables over moe_pack's int32 buffer [3 P + 5 E + 4] (views, no copy)."""
    P = (buf.shape[0] - 5 * E - 4) // 3
    parts = torch.split(buf, [P, P, P, E, E, E, E, E, 4])
    return ops.Packing(*parts, P=P, k=k, E=E)


def _packing_buffer(P: int, E: int, device) -> torch.Tensor:
    """A zeroed packing buffer: the launches define the segment tables only up to the segment count
    (meta[0]), and an operator's outputs must not depend on what the memory held before."""
    return torch.zeros(3 * P + 5 * E + 4, dtype=torch.int32, device=device)


# ----------------------------------------------------------------------------- router
@torch.library.custom_op(f"{_NS}::router_topk", mutates_args=())
def router_topk(logits: torch.Tensor, k: int, norm: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """(inds int32 [B, k], scores bf16 [B, k]) of router logits [B, E] (jit_router_topk)."""
    return ops.router_topk(logits, k, norm)


@router_topk.register_fake
def _(logits, k, norm):
    B = logits.shape[0]
    return logits.new_empty((B, k), dtype=torch.int32), logits.new_empty((B, k), dtype=torch.bfloat16)


@torch.library.custom_op(f"{_NS}::moe_pack", mutates_args=())
def moe_pack(inds: torch.Tensor, n_experts: int) -> torch.Tensor:
    """The packing tables of inds [B, k] as one int32 buffer [3 P + 5 E + 4] (jit_moe_pack;
    packing_from_buffer splits it; segment entries past the segment count are zero)."""
    P, E = inds.numel(), int(n_experts)
    buf = _packing_buffer(P, E, inds.device)
    ops.moe_pack_into(inds, packing_from_buffer(buf, inds.shape[-1], E))
    return buf


@moe_pack.register_fake
def _(inds, n_experts):
    P = inds.shape[0] * inds.shape[1]
    return inds.new_empty((3 * P + 5 * n_experts + 4,), dtype=torch.int32)


@torch.library.custom_op(f"{_NS}::route_pack", mutates_args=())
def route_pack(logits: torch.Tensor, k: int, norm: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(inds, scores, packing buffer) of at most 4 router rows in one launch (jit_route_pack): the
    router_topk and moe_pack results."""
    rows, E = logits.shape
    buf = _packing_buffer(rows * k, E, logits.device)
    inds, scores, _ = ops.route_pack(logits, k, norm, pk=packing_from_buffer(buf, k, E))
    return inds, scores, buf


@route_pack.register_fake
def _(logits, k, norm):
    rows, E = logits.shape
    return (logits.new_empty((rows, k), dtype=torch.int32), logits.new_empty((rows, k), dtype=torch.bfloat16),
            logits.new_empty((3 * rows * k + 5 * E + 4,), dtype=torch.int32))


# ----------------------------------------------------------------------------- experts
@torch.library.custom_op(f"{_NS}::expert_gate_up", mutates_args=())
def expert_gate_up(x: torch.Tensor, packed: torch.Tensor, E: int, N: int, K: int, pack_buf: torch.Tensor,
                   k: int, seg: bool) -> torch.Tensor:
    """h bf16 [P, N / 2] of the fused gate||up stack [E, N, K] with SwiGLU, in sorted pair order
    (jit_moe_gate_up_swiglu_packed, or the segment GEMM with seg)."""
    return ops.expert_gate_up(x, _packed(packed, E, N, K), packing_from_buffer(pack_buf, k, E), seg=seg)


@expert_gate_up.register_fake
def _(x, packed, E, N, K, pack_buf, k, seg):
    P = (pack_buf.shape[0] - 5 * E - 4) // 3
    return x.new_empty((P, N // 2), dtype=torch.bfloat16)


@torch.library.custom_op(f"{_NS}::route_gate_up", mutates_args=())
def route_gate_up(x: torch.Tensor, logits: torch.Tensor, packed: torch.Tensor, E: int, N: int, K: int, k: int,
                  norm: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(inds, scores, packing buffer, h) of one token: route_pack and expert_gate_up in one launch
    (jit_moe_gate_up_swiglu_routed_packed)."""
    buf = _packing_buffer(k, E, x.device)
    inds, scores, _, h = ops.route_gate_up(x, logits, _packed(packed, E, N, K), k, norm,
                                           pk=packing_from_buffer(buf, k, E))
    return inds, scores, buf, h


@route_gate_up.register_fake
def _(x, logits, packed, E, N, K, k, norm):
    return (x.new_empty((1, k), dtype=torch.int32), x.new_empty((1, k), dtype=torch.bfloat16),
            x.new_empty((3 * k + 5 * E + 4,), dtype=torch.int32), x.new_empty((k, N // 2), dtype=torch.bfloat16))


@torch.library.custom_op(f"{_NS}::expert_down", mutates_args=())
def expert_down(h: torch.Tensor, packed: torch.Tensor, E: int, N: int, K: int, pack_buf: torch.Tensor, k: int,
                seg: bool) -> torch.Tensor:
    """r bf16 [P, N] of the down stack [E, N, K] in sorted pair order (jit_moe_down_packed, or
    the segment GEMM with seg)."""
    return ops.expert_down(h, _packed(packed, E, N, K), packing_from_buffer(pack_buf, k, E), seg=seg)


@expert_down.register_fake
def _(h, packed, E, N, K, pack_buf, k, seg):
    return h.new_empty((h.shape[0], N), dtype=torch.bfloat16)


@torch.library.custom_op(f"{_NS}::moe_combine", mutates_args=())
def moe_combine(r: torch.Tensor, pack_buf: torch.Tensor, k: int, E: int, scores: torch.Tensor,
                resid: torch.Tensor | None) -> torch.Tensor:
    """y bf16 [B, D]: the slot-order weighted sum of the pair rows r, plus resid (jit_moe_combine)."""
    return ops.moe_combine(r, packing_from_buffer(pack_buf, k, E), scores, resid)


@moe_combine.register_fake
def _(r, pack_buf, k, E, scores, resid):
    return r.new_empty((scores.shape[0], r.shape[1]), dtype=torch.bfloat16)


@torch.library.custom_op(f"{_NS}::moe_combine_rmsnorm", mutates_args=())
def moe_combine_rmsnorm(r: torch.Tensor, pack_buf: torch.Tensor, k: int, E: int, scores: torch.Tensor,
                        resid: torch.Tensor | None, w: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(y, xn): moe_combine and the RMSNorm of its rows in one launch (jit_moe_combine_rmsnorm)."""
    return ops.moe_combine_rmsnorm(r, packing_from_buffer(pack_buf, k, E), scores, resid, w, eps)


@moe_combine_rmsnorm.register_fake
def _(r, pack_buf, k, E, scores, resid, w, eps):
    y = r.new_empty((scores.shape[0], r.shape[1]), dtype=torch.bfloat16)
    return y, torch.empty_like(y)


# ----------------------------------------------------------------------------- dense, norms
@torch.library.custom_op(f"{_NS}::qmm", mutates_args=())
def qmm(x: torch.Tensor, packed: torch.Tensor, N: int, K: int) -> torch.Tensor:
    """x [T, K] bf16 against a packed 4-bit matrix [N, K] (jit_qmm_packed, or jit_qmm_seg for a
    long batch)."""
    return ops.qmm(x, _packed(packed, 1, N, K))


@qmm.register_fake
def _(x, packed, N, K):
    return x.new_empty((x.shape[0], N), dtype=torch.bfloat16)


@torch.library.custom_op(f"{_NS}::rmsnorm", mutates_args=())
def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm rows of x (jit_rmsnorm)."""
    return ops.rmsnorm(x, w, eps)


@rmsnorm.register_fake
def _(x, w, eps):
    return torch.empty_like(x)


@torch.library.custom_op(f"{_NS}::rmsnorm_add", mutates_args=())
def rmsnorm_add(x: torch.Tensor, resid: torch.Tensor, w: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(RMSNorm of h, h) for h = x + resid, in one launch (jit_rmsnorm with a residual)."""
    return ops.rmsnorm(x, w, eps, resid, return_sum=True)


@rmsnorm_add.register_fake
def _(x, resid, w, eps):
    return torch.empty_like(x), torch.empty_like(x)


@torch.library.custom_op(f"{_NS}::qmm_add_rmsnorm", mutates_args=())
def qmm_add_rmsnorm(a: torch.Tensor, resid: torch.Tensor, w: torch.Tensor, eps: float, packed: torch.Tensor, N: int,
                    K: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(y, h, hn) of one row: h = a + resid, hn its RMSNorm, y = hn against a packed 4-bit [N, K]
    matrix, in one launch (jit_qmm_packed_add_rmsnorm)."""
    return ops.qmm_add_rmsnorm(a, resid, w, eps, _packed(packed, 1, N, K))


@qmm_add_rmsnorm.register_fake
def _(a, resid, w, eps, packed, N, K):
    return a.new_empty((1, N), dtype=torch.bfloat16), torch.empty_like(a), torch.empty_like(a)


@torch.library.custom_op(f"{_NS}::qmm_combine_rmsnorm", mutates_args=())
def qmm_combine_rmsnorm(r: torch.Tensor, pack_buf: torch.Tensor, k: int, E: int, scores: torch.Tensor,
                        resid: torch.Tensor | None, w: torch.Tensor, eps: float, packed: torch.Tensor, N: int,
                        K: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(y, out) of one row: y = moe_combine, out = its RMSNorm against a packed 4-bit [N, K] matrix,
    in one launch (jit_qmm_packed_combine_rmsnorm)."""
    return ops.qmm_combine_rmsnorm(r, packing_from_buffer(pack_buf, k, E), scores, resid, w, eps,
                                   _packed(packed, 1, N, K))


@qmm_combine_rmsnorm.register_fake
def _(r, pack_buf, k, E, scores, resid, w, eps, packed, N, K):
    return r.new_empty((1, r.shape[1]), dtype=torch.bfloat16), r.new_empty((1, N), dtype=torch.bfloat16)


# ----------------------------------------------------------------------------- attention
@torch.library.custom_op(f"{_NS}::qk_norm_rope_append", mutates_args=("pool",))
def qk_norm_rope_append(qkv: torch.Tensor, H: int, Hkv: int, q_norm: torch.Tensor, k_norm: torch.Tensor,
                        eps: float, inv_freq: torch.Tensor, pos: torch.Tensor, page_table: torch.Tensor,
                        pool: torch.Tensor) -> torch.Tensor:
    """q bf16 [B, H, 128] (normed, rotated); k and v of every row written into the pool
    (jit_qk_norm_rope_append)."""
    return ops.qk_norm_rope_append(qkv, H, Hkv, q_norm, k_norm, eps, inv_freq, pos, page_table, pool)


@qk_norm_rope_append.register_fake
def _(qkv, H, Hkv, q_norm, k_norm, eps, inv_freq, pos, page_table, pool):
    return qkv.new_empty((qkv.shape[0], H, ops.HEAD_DIM), dtype=torch.bfloat16)


@torch.library.custom_op(f"{_NS}::paged_decode_attention", mutates_args=("workspace",))
def paged_decode_attention(q: torch.Tensor, pool: torch.Tensor, page_table: torch.Tensor, lens: torch.Tensor,
                           chunk_start: torch.Tensor, chunk_seq: torch.Tensor, total: int, max_len: int,
                           scale: float, workspace: torch.Tensor) -> torch.Tensor:
    """out bf16 [B, H, 128] of split-K paged decode attention under an attention plan given by its
    tensors (jit_paged_decode_attn; workspace of attn_workspace_bytes(total, H) bytes).  max_len is
    the plan's longest sequence (plan_args gives it): the page table's width is checked against it,
    the device tensors are not read on the host."""
    plan = ops.AttnPlan(lens, chunk_start, chunk_seq, int(total), np.array([int(max_len)], np.int32))
    return ops.paged_decode_attention(q, pool, page_table, plan, scale, workspace)


@paged_decode_attention.register_fake
def _(q, pool, page_table, lens, chunk_start, chunk_seq, total, max_len, scale, workspace):
    return torch.empty_like(q)


@torch.library.custom_op(f"{_NS}::paged_decode_attention_qkv", mutates_args=("pool", "workspace"))
def paged_decode_attention_qkv(qkv: torch.Tensor, H: int, Hkv: int, q_norm: torch.Tensor, k_norm: torch.Tensor,
                               eps: float, inv_freq: torch.Tensor, pool: torch.Tensor, page_table: torch.Tensor,
                               lens: torch.Tensor, chunk_start: torch.Tensor, chunk_seq: torch.Tensor, total: int,
                               max_len: int, scale: float, workspace: torch.Tensor) -> torch.Tensor:
    """out bf16 [B, H, 128] of the step's raw qkv rows: qk_norm_rope_append of each token at position
    lens[b] - 1 and split-K paged decode attention in one launch (jit_paged_decode_attn_qkv).  The
    plan's tensors and max_len as for paged_decode_attention."""
    plan = ops.AttnPlan(lens, chunk_start, chunk_seq, int(total), np.array([int(max_len)], np.int32))
    return ops.paged_decode_attention_qkv(qkv, H, Hkv, q_norm, k_norm, eps, inv_freq, pool, page_table, plan, scale,
                                          workspace)


@paged_decode_attention_qkv.register_fake
def _(qkv, H, Hkv, q_norm, k_norm, eps, inv_freq, pool, page_table, lens, chunk_start, chunk_seq, total, max_len,
      scale, workspace):
    return qkv.new_empty((qkv.shape[0], H, ops.HEAD_DIM), dtype=torch.bfloat16)


@torch.library.custom_op(f"{_NS}::paged_prefill_attention", mutates_args=("workspace",))
def paged_prefill_attention(q: torch.Tensor, pool: torch.Tensor, page_table: torch.Tensor, tables: torch.Tensor,
                            blocks: torch.Tensor, chunks: list[int], pmax: int, max_len: int, scale: float,
                            workspace: torch.Tensor) -> torch.Tensor:
    """out bf16 [T, H, 128]: causal attention of prefill chunks over the paged pool, under a prefill
    plan given by its tensors and its chunks flattened as (seq, ctx, length) triples
    (jit_paged_prefill_attn; workspace of prefill_workspace_bytes bytes)."""
    trip = [tuple(chunks[i:i + 3]) for i in range(0, len(chunks), 3)]
    plan = ops.PrefillPlan(trip, tables, blocks, sum(c[2] for c in trip), int(pmax), int(max_len))
    return ops.paged_prefill_attention(q, pool, page_table, plan, scale, workspace)


@paged_prefill_attention.register_fake
def _(q, pool, page_table, tables, blocks, chunks, pmax, max_len, scale, workspace):
    return torch.empty_like(q)


def prefill_plan_args(plan: ops.PrefillPlan) -> tuple:
    """(tables, blocks, chunks, pmax, max_len) of a prefill plan, for
    torch.ops.jitengine.paged_prefill_attention."""
    return plan.tables, plan.blocks, [int(v) for c in plan.chunks for v in c], plan.pmax, plan.max_len


# ----------------------------------------------------------------------------- paged KV
@torch.library.custom_op(f"{_NS}::kv_append_paged", mutates_args=("pool",))
def kv_append_paged(pool: torch.Tensor, k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor,
                    page_table: torch.Tensor) -> None:
    """k, v [B, Hkv, 128] written at positions pos [B] of the paged pool (jit_kv_append_paged)."""
    ops.kv_append_paged(pool, k, v, pos, page_table)


@kv_append_paged.register_fake
def _(pool, k, v, pos, page_table):
    return None


@torch.library.custom_op(f"{_NS}::kv_copy_pages", mutates_args=("pool",))
def kv_copy_pages(pool: torch.Tensor, src: torch.Tensor, dst: torch.Tensor) -> None:
    """Pages src[i] copied to dst[i] inside one layer's pool (jit_kv_copy_pages)."""
    ops.kv_copy_pages(pool, src, dst)


@kv_copy_pages.register_fake
def _(pool, src, dst):
    return None


def plan_args(plan: ops.AttnPlan) -> tuple:
    """(lens, chunk_start, chunk_seq, total, max_len) of an attention plan, for
    torch.ops.jitengine.paged_decode_attention."""
    mx = int(plan.lens_host.max()) if plan.lens_host.size else 0
    return plan.lens, plan.chunk_start, plan.chunk_seq, plan.total, mx


# ----------------------------------------------------------------------------- sampler
@torch.library.custom_op(f"{_NS}::logprobs_rows", mutates_args=())
def logprobs_rows(logits: torch.Tensor) -> torch.Tensor:
    """bf16 [B, V] log-probabilities (jit_logprobs_rows)."""
    return ops.logprobs_rows(logits)


@logprobs_rows.register_fake
def _(logits):
    return torch.empty_like(logits)


@torch.library.custom_op(f"{_NS}::argmax_rows", mutates_args=())
def argmax_rows(logits: torch.Tensor) -> torch.Tensor:
    """int32 [B] greedy draws (jit_argmax_rows)."""
    return ops.argmax_rows(logits)


@argmax_rows.register_fake
def _(logits):
    return logits.new_empty((logits.shape[0],), dtype=torch.int32)


@torch.library.custom_op(f"{_NS}::sample_rows", mutates_args=())
def sample_rows(logits: torch.Tensor, temperature: float, top_p: float, top_k: int, u: torch.Tensor) -> torch.Tensor:
    """int32 [B] draws under shared temperature / top-p / top-k given uniforms u [B] (jit_sample_rows)."""
    return ops.sample_rows(logits, temperature, top_p, top_k, u)


@sample_rows.register_fake
def _(logits, temperature, top_p, top_k, u):
    return logits.new_empty((logits.shape[0],), dtype=torch.int32)


@torch.library.custom_op(f"{_NS}::threefry_uniform", mutates_args=())
def threefry_uniform(keys: torch.Tensor) -> torch.Tensor:
    """fp32 [B] uniforms of uint32 key pairs [B, 2] (jit_threefry_uniform)."""
    return ops.threefry_uniform(keys)


@threefry_uniform.register_fake
def _(keys):
    return keys.new_empty((keys.shape[0],), dtype=torch.float32)


OPS = ("router_topk", "moe_pack", "route_pack", "expert_gate_up", "route_gate_up", "expert_down", "moe_combine",
       "moe_combine_rmsnorm", "qmm", "rmsnorm", "rmsnorm_add", "qmm_add_rmsnorm", "qmm_combine_rmsnorm",
       "qk_norm_rope_append", "paged_decode_attention", "paged_decode_attention_qkv", "paged_prefill_attention",
       "kv_append_paged", "kv_copy_pages", "logprobs_rows", "argmax_rows", "sample_rows", "threefry_uniform")
