"""On-device self-check of the hot path's kernels, once per device before the first step.

The reference runs small cases of its custom kernels against stock MLX ops when an engine loads and
turns off any kernel that disagrees (Q36/kernels/selfcheck.py:123-144, called from
Q36/engine/engine.py:355-375).  This build has no other compute path to fall back to, so a kernel
that disagrees raises SelfCheckError instead.  Each case is tiny and compares the HIP kernel with a
plain torch fp32 computation of the same op on the same device (integer outputs exactly, bf16
outputs within the north-star tolerance: max-abs <= 2e-2 or 2 bf16 ulps, cosine >= 0.9995).  The
torch computations are the checker only; nothing here feeds a result back into a step.

Opt in with Engine(..., selfcheck=True) or JITENGINE_SELFCHECK=1 in the environment.
"""

from __future__ import annotations

import os
import threading

import torch

from . import ops
from .quant import dequantize4, random_quantized

_done: set = set()
_lock = threading.Lock()


class SelfCheckError(RuntimeError):
    """A kernel disagreed with its torch reference on the device (the message names the case)."""


def enabled_by_env() -> bool:
    return os.environ.get("JITENGINE_SELFCHECK", "") not in ("", "0")


def _close(name: str, got: torch.Tensor, want: torch.Tensor) -> None:
    g, w = got.float().flatten(), want.float().flatten()
    if not torch.isfinite(g).all():
        raise SelfCheckError(f"{name}: non-finite outputs")
    ulp = torch.where(w == 0, torch.full_like(w, 2.0**-133), w.abs()) * 2.0**-7
    bound = torch.maximum(torch.full_like(w, 2e-2), 2 * ulp)
    err = (g - w).abs()
    cos = float(g @ w / (g.norm() * w.norm()).clamp_min(1e-30)) if g.numel() else 1.0
    if bool((err > bound).any()) or cos < 0.9995:
        raise SelfCheckError(f"{name}: max |err| {float(err.max()):.3g}, cosine {cos:.6f} against the torch reference")


def _equal(name: str, got: torch.Tensor, want: torch.Tensor) -> None:
    if not torch.equal(got.to(want.dtype), want):
        raise SelfCheckError(f"{name}: integer outputs differ from the torch reference")


def _router_and_pack(dev) -> None:
    B, E, k = 4, 128, 8
    g = torch.Generator(device="cpu").manual_seed(1)
    # distinct logits k / 8: every gate differs from its neighbours in bf16, so the order is unambiguous
    logits = torch.stack([torch.randperm(E, generator=g) for _ in range(B)]).float().sub(64).div(8)
    lt = logits.to(torch.bfloat16).to(dev)
    inds, scores = ops.router_topk(lt, k, True)
    gates = torch.softmax(lt.float(), dim=-1)
    top = torch.topk(gates, k, dim=-1)  # descending; the kernel's slots run ascending (slot 0 = k-th largest)
    _equal("router_topk indices", inds, top.indices.flip(-1).to(torch.int32))
    want = top.values.flip(-1)
    _close("router_topk scores", scores, want / want.sum(-1, keepdim=True))
    pk = ops.moe_pack(inds, E)
    flat = inds.reshape(-1).long()
    order = torch.sort(flat, stable=True).indices
    _equal("moe_pack order", pk.order, order.to(torch.int32))
    _equal("moe_pack pair_row", pk.pair_row, (order // k).to(torch.int32))
    _equal("moe_pack expert_cnt", pk.expert_cnt, torch.bincount(flat, minlength=E).to(torch.int32))


def _projections(dev) -> None:
    g = torch.Generator(device=dev).manual_seed(2)
    x = torch.randn((5, 512), generator=g, device=dev).to(torch.bfloat16)
    w = random_quantized((64, 512), 3, device=dev)
    want = x.float() @ dequantize4(w).t()
    _close("qmm (MLX layout)", ops.qmm(x, w, seg=False), want)
    _close("qmm (packed)", ops.qmm(x, ops.prepack(w), seg=False), want)
    E, D, I, k = 8, 512, 256, 2
    gu, dn = random_quantized((E, 2 * I, D), 4, device=dev), random_quantized((E, D, I), 5, device=dev)
    inds = torch.stack([torch.randperm(E, device=dev)[:k] for _ in range(3)]).to(torch.int32)
    pk = ops.moe_pack(inds, E)
    xe = torch.randn((3, D), generator=g, device=dev).to(torch.bfloat16)
    h = ops.expert_gate_up(xe, gu, pk)
    wgu, wdn = dequantize4(gu), dequantize4(dn)
    e_of = inds.reshape(-1)[pk.order.long()].long()
    rows = xe[pk.pair_row.long()].float()
    gu_out = torch.einsum("pk,pnk->pn", rows, wgu[e_of])
    gate, up = gu_out[:, :I], gu_out[:, I:]
    _close("gate_up + SwiGLU", h, torch.nn.functional.silu(gate) * up)
    r = ops.expert_down(h, dn, pk)
    _close("down", r, torch.einsum("pk,pnk->pn", h.float(), wdn[e_of]))


def _norm_and_attention(dev) -> None:
    g = torch.Generator(device=dev).manual_seed(6)
    x = torch.randn((3, 2048), generator=g, device=dev).to(torch.bfloat16)
    wn = (1 + 0.02 * torch.randn(2048, generator=g, device=dev)).to(torch.bfloat16)
    xf = x.float()
    _close("rmsnorm", ops.rmsnorm(x, wn, 1e-6), xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) * wn.float())
    H, Hkv, lens = 8, 2, [5, 40, 1600]
    pool, table, npg, K, V = _paged_kv(g, dev, lens, Hkv)
    q = torch.randn((len(lens), H, ops.HEAD_DIM), generator=g, device=dev).to(torch.bfloat16)
    out = ops.paged_decode_attention(q, pool, table, ops.attn_plan(lens, dev), ops.HEAD_DIM ** -0.5)
    want = torch.empty((len(lens), H, ops.HEAD_DIM), device=dev)
    for b, L in enumerate(lens):
        kb, vb = _keys_of(K, V, table, npg, b, L, Hkv)
        qb = q[b].float().reshape(Hkv, H // Hkv, ops.HEAD_DIM)
        p = torch.softmax(qb @ kb.transpose(1, 2) * ops.HEAD_DIM ** -0.5, dim=-1)
        want[b] = (p @ vb).reshape(H, ops.HEAD_DIM)
    _close("paged decode attention", out, want)


def _paged_kv(g, dev, keys, Hkv):
    """A pool holding each sequence's keys in permuted pages, its table, and the K and V views
    [pages, Hkv, 16, 128] (fp32) of its two parts (K chunk-major, V dim-major)."""
    npg = [-(-n // ops.PAGE) for n in keys]
    pool = torch.randn((sum(npg) + 1, Hkv, 2, ops.PAGE * ops.HEAD_DIM), generator=g, device=dev).to(torch.bfloat16)
    perm = torch.randperm(sum(npg), device=dev).to(torch.int32)
    table = torch.zeros((len(keys), max(npg)), dtype=torch.int32, device=dev)
    at = 0
    for b, n in enumerate(npg):
        table[b, :n] = perm[at:at + n]
        at += n
    pf = pool.float()
    K = pf[:, :, 0].reshape(-1, Hkv, 4, ops.PAGE, 32).permute(0, 1, 3, 2, 4).reshape(-1, Hkv, ops.PAGE, ops.HEAD_DIM)
    V = pf[:, :, 1].reshape(-1, Hkv, ops.HEAD_DIM, ops.PAGE).transpose(2, 3)
    return pool, table, npg, K, V


def _keys_of(K, V, table, npg, b, L, Hkv):
    pages = table[b, :npg[b]].long()
    kb = K[pages].permute(1, 0, 2, 3).reshape(Hkv, -1, ops.HEAD_DIM)[:, :L]
    vb = V[pages].permute(1, 0, 2, 3).reshape(Hkv, -1, ops.HEAD_DIM)[:, :L]
    return kb, vb


def _prefill(dev) -> None:
    """Causal prefill attention of two chunks, one across the first key cut (partials and merge)."""
    g = torch.Generator(device=dev).manual_seed(7)
    H, Hkv, cut = 8, 2, int(ops._lib.lib().jit_prefill_part_keys())
    chunks = [(0, 0, 20), (1, cut - 10, 24)]
    pool, table, npg, K, V = _paged_kv(g, dev, [ctx + n for _, ctx, n in chunks], Hkv)
    T = sum(n for *_, n in chunks)
    q = torch.randn((T, H, ops.HEAD_DIM), generator=g, device=dev).to(torch.bfloat16)
    scale = ops.HEAD_DIM ** -0.5
    out = ops.paged_prefill_attention(q, pool, table, ops.prefill_plan(chunks, H, Hkv, dev), scale)
    want = torch.empty((T, H, ops.HEAD_DIM), device=dev)
    row = 0
    for seq, ctx, n in chunks:
        kb, vb = _keys_of(K, V, table, npg, seq, ctx + n, Hkv)
        qb = q[row:row + n].float().reshape(n, Hkv, H // Hkv, ops.HEAD_DIM).permute(1, 0, 2, 3)
        s = torch.einsum("hngd,hkd->hngk", qb, kb) * scale
        pos = ctx + torch.arange(n, device=dev)
        s = s.masked_fill(torch.arange(ctx + n, device=dev)[None, None, None, :] > pos[None, :, None, None], -torch.inf)
        o = torch.einsum("hngk,hkd->hngd", torch.softmax(s, dim=-1), vb)
        want[row:row + n] = o.permute(1, 0, 2, 3).reshape(n, H, ops.HEAD_DIM)
        row += n
    _close("paged prefill attention", out, want)


def _segment(dev) -> None:
    """The segment GEMMs of long expert segments (bf16 weights, bf16(s q + b)) with SwiGLU."""
    g = torch.Generator(device=dev).manual_seed(8)
    E, D, I, k, B = 8, 512, 256, 2, 48
    gu, dn = random_quantized((E, 2 * I, D), 9, device=dev), random_quantized((E, D, I), 10, device=dev)
    inds = torch.stack([torch.randperm(E, device=dev)[:k] for _ in range(B)]).to(torch.int32)
    pk = ops.moe_pack(inds, E)
    xe = torch.randn((B, D), generator=g, device=dev).to(torch.bfloat16)
    h = ops.expert_gate_up(xe, ops.prepack(gu), pk, seg=True)
    wgu = dequantize4(gu).to(torch.bfloat16).float()
    wdn = dequantize4(dn).to(torch.bfloat16).float()
    e_of = inds.reshape(-1)[pk.order.long()].long()
    gu_out = torch.einsum("pk,pnk->pn", xe[pk.pair_row.long()].float(), wgu[e_of])
    _close("segment gate_up + SwiGLU", h, torch.nn.functional.silu(gu_out[:, :I]) * gu_out[:, I:])
    r = ops.expert_down(h, ops.prepack(dn), pk, seg=True)
    _close("segment down", r, torch.einsum("pk,pnk->pn", h.float(), wdn[e_of]))


def _sampler(dev) -> None:
    x = torch.zeros((2, 1000), device=dev)
    x[0, 417], x[1, 3] = 5.0, 7.0
    _equal("greedy draw", ops.argmax_rows(x.to(torch.bfloat16)), torch.tensor([417, 3], dtype=torch.int32, device=dev))


CASES = (("router + packing", _router_and_pack), ("projections + experts", _projections),
         ("rmsnorm + attention", _norm_and_attention), ("prefill attention", _prefill),
         ("segment GEMMs", _segment), ("sampler", _sampler))


def run(device=None, force: bool = False) -> list:
    """Run every case on `device` (default: the current one) unless it already passed there;
    returns the names of the cases run.  Raises SelfCheckError on the first disagreement."""
    dev = torch.device(device if device is not None else f"cuda:{torch.cuda.current_device()}")
    if dev.type != "cuda":
        raise ValueError("the self-check runs the HIP kernels: give it a GPU device")
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    with _lock:
        if key in _done and not force:
            return []
        with torch.cuda.device(key):
            for _, fn in CASES:
                fn(dev)
            torch.cuda.synchronize(key)
        _done.add(key)
    return [name for name, _ in CASES]
