"""The MoE block's routed-expert path on the HIP kernels.

Mirrors the call sites of Qwen3_5MoeSparseMoeBlock (Q36/model/moe.py): the router logits
(`_route_logits`, :296-302), the fused router top-k (`_route_top_k`, :304-315), token-to-expert
packing (`_sort_pairs`, :151-159), gate||up + SwiGLU and down over the packed pairs (:191-193), and
the slot-order weighted combine (:286) with the residual (`with_residual`, :119-123).  The
BASELINE geometry has no shared expert, so there is no shared branch.
"""

from __future__ import annotations

import torch

from . import ops
from .quant import QLinear


class MoEBlock:
    """Router + routed experts over ragged token rows x [B, D] (bf16, on the GPU)."""

    def __init__(self, router: QLinear, gate_up: QLinear, down: QLinear, top_k: int = 8,
                 norm_topk: bool = True, prepack: bool = True):
        for lin in (router, gate_up, down):
            lin.validate()
        if gate_up.weight.dim() != 3 or down.weight.dim() != 3:
            raise ValueError("gate_up and down must be expert stacks [E, N, K]")
        E = gate_up.weight.shape[0]
        if down.weight.shape[0] != E or router.out_dims != E:
            raise ValueError("router, gate_up and down disagree on the number of experts")
        if down.in_dims * 2 != gate_up.out_dims or down.out_dims != gate_up.in_dims:
            raise ValueError("down must be [E, D, I] for a gate_up stack [E, 2I, D]")
        if prepack:  # one-time reorder into the MFMA tile layout (coalesced weight streaming)
            router, gate_up, down = ops.prepack(router), ops.prepack(gate_up), ops.prepack(down)
        self.router, self.gate_up, self.down = router, gate_up, down
        self.top_k = int(top_k)
        self.norm_topk = bool(norm_topk)
        self.num_experts = E

    def route(self, x: torch.Tensor):
        """(inds int32 [B, k], scores bf16 [B, k]) for rows x [B, D]."""
        logits = ops.qmm(x, self.router)
        return ops.router_topk(logits, self.top_k, self.norm_topk)

    def use_seg(self, P: int, prefill: bool) -> bool:
        """Whether a prefill batch of P pairs takes the segment GEMM: at least 4 pairs per expert
        on average (the reference's switch, Q36/model/moe.py:161-175) on prepacked stacks.  Decode
        steps always take the decode kernels, as the reference's decode path does."""
        packed = isinstance(self.gate_up, ops.PackedQ4) and isinstance(self.down, ops.PackedQ4)
        return prefill and packed and P >= 16 and P // self.num_experts >= 4

    def experts(self, x: torch.Tensor, inds: torch.Tensor, scores: torch.Tensor,
                resid: torch.Tensor | None = None, prefill: bool = False) -> torch.Tensor:
        """Every selected expert applied and combined: y [B, D] (+ resid)."""
        pk = ops.moe_pack(inds, self.num_experts)
        _, r = self.expert_mlp(x, pk, prefill)
        return ops.moe_combine(r, pk, scores, resid)

    def expert_mlp(self, x: torch.Tensor, pk: ops.Packing, prefill: bool = False):
        """(h [P, I], r [P, D]) in sorted pair order: gate||up + SwiGLU and down over packed pairs."""
        seg = self.use_seg(pk.P, prefill)
        h = ops.expert_gate_up(x, self.gate_up, pk, seg=seg)
        return h, ops.expert_down(h, self.down, pk, seg=seg)

    def __call__(self, x: torch.Tensor, resid: torch.Tensor | None = None, prefill: bool = False) -> torch.Tensor:
        inds, scores = self.route(x)
        return self.experts(x, inds, scores, resid, prefill)

    def with_residual(self, x: torch.Tensor, resid: torch.Tensor) -> torch.Tensor:
        """resid + moe(x)."""
        return self(x, resid)
