"""The segment GEMM of long expert segments (row a9; chunked prefill) vs the CPU oracle (MI355X only).

Its arithmetic is the reference's prefill tile GEMM (Q36/kernels/gather_qmm_prefill.py): weights
dequantized to bf16, bf16 products accumulated in fp32.  The oracle restates it with float64 sums
over the same bf16 weights (oracle.moe_gate_up / moe_down with bf16w), so the bar is the north-star
float tolerance; the integer tables are shared with the decode path (jit_moe_pack)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from jitengine_amd import ops
from jitengine_amd.moe import MoEBlock
from jitengine_amd.quant import QLinear, random_quantized
from tests.helpers import assert_close_bf16, bf16_tensor, normal_bf16, router_logits, stack_np, u16

pytestmark = pytest.mark.gpu
DEV = "cuda"
D, I, K_TOP = 2048, 768, 8


def _stack(E, N, K, seed):
    parts = [random_quantized((min(8, E - e0), N, K), seed * 100 + e0) for e0 in range(0, E, 8)]
    return QLinear(torch.cat([p.weight for p in parts]), torch.cat([p.scales for p in parts]),
                   torch.cat([p.biases for p in parts]))


def _skewed_inds(B, E, seed):
    """Each row picks 8 distinct experts from 0..E-3 with a skewed preference (expert 0 is in
    nearly every row: up to three 160-token chunks); expert E-2 gets exactly one pair and
    expert E-1 none."""
    rng = np.random.default_rng(seed)
    w = 1.0 / (1.0 + np.arange(E - 2)) ** 1.5
    w[0] = 50.0
    inds = np.stack([rng.choice(E - 2, K_TOP, replace=False, p=w / w.sum()) for _ in range(B)]).astype(np.int32)
    inds[0, K_TOP - 1] = E - 2
    return inds


@pytest.fixture(scope="module")
def seg_case():
    B, E = 420, 20
    gu_h, dn_h = _stack(E, 2 * I, D, 31), _stack(E, D, I, 32)
    gu, dn = ops.prepack(gu_h.to(DEV)), ops.prepack(dn_h.to(DEV))
    x = normal_bf16((B, D), seed=33)
    inds = _skewed_inds(B, E, seed=34)
    return B, E, gu_h, dn_h, gu, dn, x, inds


def test_segment_gemm_parity(seg_case):
    B, E, gu_h, dn_h, gu, dn, x, inds = seg_case
    pk = ops.moe_pack(torch.from_numpy(inds).to(DEV), E)
    cnt = pk.expert_cnt.cpu().numpy()
    assert cnt[0] > 320 and cnt[E - 2] == 1 and cnt[E - 1] == 0  # 3 chunks, a 1-row segment, an empty one
    h = ops.expert_gate_up(bf16_tensor(x, DEV), gu, pk, seg=True)
    torch.cuda.synchronize()
    opk = oracle.moe_pack(inds.view(np.uint32), E)
    want_h = oracle.moe_gate_up(x, inds.view(np.uint32), opk, *stack_np(gu_h), bf16w=True)
    st = assert_close_bf16(u16(h), want_h, what="seg gate_up")
    assert st["bit_equal"] > 0.9, st
    # down on the GPU's h (isolates the down GEMM)
    r = ops.expert_down(h, dn, pk, seg=True)
    want_r = oracle.moe_down(u16(h), inds.view(np.uint32), opk, *stack_np(dn_h), bf16w=True)
    st = assert_close_bf16(u16(r), want_r, what="seg down")
    assert st["bit_equal"] > 0.9, st


def _pairs_of(inds_flat, order, pair_row, sel):
    """(expert ids, pack) for the sorted positions `sel` alone, in the oracle's calling form: the
    oracle computes pair j of the returned table as the pair at sorted position sel[j]."""
    ids = np.ascontiguousarray(inds_flat[order[sel]]).astype(np.uint32)
    return ids, {"order": np.arange(sel.size, dtype=np.int32), "pair_row": np.ascontiguousarray(pair_row[sel])}


def test_segment_gemm_config3_geometry():
    """BASELINE configs[3]'s MoE half at full size: 2,108 rows (four 512-token prefill chunks and 60
    decode rows) routed top-8 over 128 experts -- 16,864 pairs, ~132 per expert, 160-row token
    chunks, every expert's column blocks on the XCD of its expert -- through the segment GEMMs,
    against the oracle's bf16-weight restatement on every pair of 16 experts (the largest segment
    among them) with the seg tests' >= 90% bit-equal floor."""
    B, E = 2108, 128
    gu_d = random_quantized((E, 2 * I, D), 61, device=DEV)
    dn_d = random_quantized((E, D, I), 62, device=DEV)
    gu, dn = ops.prepack(gu_d), ops.prepack(dn_d)
    gu_h, dn_h = gu_d.to("cpu"), dn_d.to("cpu")
    del gu_d, dn_d
    x = normal_bf16((B, D), seed=63)
    inds, _, _ = oracle.router_topk(router_logits(0, B, E, seed=64), K_TOP, True)
    pk = ops.moe_pack(torch.from_numpy(inds.view(np.int32)).to(DEV), E)
    h = ops.expert_gate_up(bf16_tensor(x, DEV), gu, pk, seg=True)
    r = ops.expert_down(h, dn, pk, seg=True)
    torch.cuda.synchronize()
    cnt = pk.expert_cnt.cpu().numpy()
    order, pair_row = pk.order.cpu().numpy(), pk.pair_row.cpu().numpy()
    by_count = np.argsort(cnt, kind="stable")
    pick = set(by_count[np.linspace(0, E - 1, 15).astype(int)].tolist()) | {int(cnt.argmax())}
    while len(pick) < 16:
        pick.add(int(by_count[len(pick)]))
    flat = inds.reshape(-1)
    sel = np.flatnonzero(np.isin(flat[order], sorted(pick)))
    assert cnt.max() >= 150 and sel.size > 16 * 64, (cnt.max(), sel.size)  # a whole 160-row chunk; ~2,100 pairs
    ids, spk = _pairs_of(flat, order, pair_row, sel)
    want_h = oracle.moe_gate_up(x, ids, spk, *stack_np(gu_h), bf16w=True)
    st = assert_close_bf16(u16(h)[sel], want_h, what="config 3 seg gate_up")
    assert st["bit_equal"] > 0.9, st
    h_sel = np.ascontiguousarray(u16(h)[sel])
    want_r = oracle.moe_down(h_sel, ids, {"order": spk["order"]}, *stack_np(dn_h), bf16w=True)
    st = assert_close_bf16(u16(r)[sel], want_r, what="config 3 seg down")
    assert st["bit_equal"] > 0.9, st


def test_segment_gemm_rows_are_independent(seg_case):
    """A row's result does not depend on the other rows of its expert's segment (MMA rows are
    independent): a sub-batch gives the same bits as the full batch."""
    B, E, _, _, gu, dn, x, inds = seg_case
    xt = bf16_tensor(x, DEV)
    pk = ops.moe_pack(torch.from_numpy(inds).to(DEV), E)
    h = ops.expert_gate_up(xt, gu, pk, seg=True)
    r = ops.expert_down(h, dn, pk, seg=True)
    sub = np.arange(1, B, 3)
    pk2 = ops.moe_pack(torch.from_numpy(inds[sub]).to(DEV), E)
    h2 = ops.expert_gate_up(xt[torch.from_numpy(sub).to(DEV)].contiguous(), gu, pk2, seg=True)
    r2 = ops.expert_down(h2, dn, pk2, seg=True)
    # flat pair (row, slot) -> sorted position, in both batches
    inv, inv2 = pk.inv.cpu().numpy().reshape(B, K_TOP), pk2.inv.cpu().numpy().reshape(sub.size, K_TOP)
    hf, h2f, rf, r2f = u16(h), u16(h2), u16(r), u16(r2)
    for i, b in enumerate(sub):
        assert np.array_equal(hf[inv[b]], h2f[inv2[i]]), b
        assert np.array_equal(rf[inv[b]], r2f[inv2[i]]), b


def test_segment_gemm_close_to_decode_kernels(seg_case):
    """The segment GEMM (bf16 weights) and the decode kernels (exact weights) stay close on the
    same pairs.  Each is checked against its own oracle; here the bound is wider for h: rounding
    the weights moves g and u by ~0.2%, which can flip both of their bf16 roundings, and SwiGLU
    then moves h by about 2 |h| ulp(g, u) -- up to ~6 ulps of h -- so h gets 8 ulps and a relative
    norm bound of 1e-2 (expected ~4e-3: ~1e-3 from the weights and four independent bf16
    roundings per path), r (no SwiGLU) 4 ulps."""
    B, E, _, _, gu, dn, x, inds = seg_case
    xt = bf16_tensor(x, DEV)
    pk = ops.moe_pack(torch.from_numpy(inds).to(DEV), E)
    hs = ops.expert_gate_up(xt, gu, pk, seg=True)
    hd = ops.expert_gate_up(xt, gu, pk)
    assert_close_bf16(u16(hs), u16(hd), what="gate_up seg vs decode", ulps=8.0)
    a, b = hs.float(), hd.float()
    assert float((a - b).norm() / b.norm()) < 1e-2
    rs = ops.expert_down(hd, dn, pk, seg=True)
    rd = ops.expert_down(hd, dn, pk)
    assert_close_bf16(u16(rs), u16(rd), what="down seg vs decode", ulps=4.0)


def test_moe_block_prefill_switch():
    """MoEBlock takes the segment GEMM for a prefill batch with >= 4 pairs per expert and the
    decode kernels otherwise; both within tolerance of the oracle's whole expert chain."""
    E, B = 32, 128
    router = random_quantized((E, D), 41)
    gu_h, dn_h = _stack(E, 2 * I, D, 42), _stack(E, D, I, 43)
    blk = MoEBlock(router.to(DEV), gu_h.to(DEV), dn_h.to(DEV), top_k=8)
    assert blk.use_seg(B * 8, prefill=True) and not blk.use_seg(B * 8, prefill=False)
    assert not blk.use_seg(15 * 8, prefill=True)  # 3 pairs per expert (4 need P >= 128 here)
    assert blk.use_seg(16 * 8, prefill=True)
    x = normal_bf16((B, D), seed=44)
    xt = bf16_tensor(x, DEV)
    inds, scores = blk.route(xt)
    y = blk.experts(xt, inds, scores, prefill=True)
    wi = inds.cpu().numpy().view(np.uint32)
    ws = u16(scores)
    pk = oracle.moe_pack(wi, E)
    h = oracle.moe_gate_up(x, wi, pk, *stack_np(gu_h), bf16w=True)
    r = oracle.moe_down(h, wi, pk, *stack_np(dn_h), bf16w=True)
    want = oracle.moe_combine(r, pk["inv"], ws)
    assert_close_bf16(u16(y), want, what="prefill experts")


@pytest.mark.parametrize("T,N,K", [(512, 2048, 4096), (2108, 2048, 4096), (1200, 5120, 2048), (2108, 5120, 2048)])
def test_dense_segment_gemm_repeats_bit_for_bit(T, N, K):
    """A dense batch sized to each token chunk the launch picks on 256 CUs (4, 6, 8 and 10 tiles: the
    o_proj of a 512-row prompt chunk and of config 3's 2,108 rows, and qkv at 1,200 and 2,108 rows)
    gives the same bits on every call.
    A regression test: the kernel's waits for its direct global->LDS loads count the loads issued
    after the awaited ones, and with a count fixed for 10-tile chunks the shorter chunks read a
    weight stage before it had landed, now and then."""
    q = ops.prepack(random_quantized((N, K), T + N).to(DEV))
    x = bf16_tensor(normal_bf16((T, K), seed=T), DEV)
    first = ops.qmm(x, q, seg=True)
    for _ in range(12):
        assert torch.equal(ops.qmm(x, q, seg=True), first)
