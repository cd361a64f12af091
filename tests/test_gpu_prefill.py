"""Causal attention of prefill chunks over the paged pool vs the CPU oracle (MI355X only).

The oracle states the causal mask as what it is: chunk token t at position ctx + t attends the
first ctx + t + 1 keys of its sequence, i.e. the float64 decode attention of that token over
ctx + t + 1 keys (oracle.paged_prefill_attn).  The bar is the north-star float tolerance; the
invariants below are bit-exact.  The float bar is tests.helpers.assert_attention_parity without its
stock criterion (MLX's full-attention kernel is not restated): every element within one bf16 ulp +
2^-14 of its row of the float64 result and >= 98% of each row's outputs correctly rounded, which a
dropped or misplaced page fails (tests/test_attention_bar.py); plus the north star's tolerance."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from jitengine_amd import ops
from tests.helpers import assert_attention_parity, assert_close_bf16, bf16_tensor, bf16_to_f32, normal_bf16, u16

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCALE = 128 ** -0.5


def _pool(seq_keys, seed, Hkv=4, extra=7):
    """A pool holding each sequence's keys in permuted pages; table [S, max_pages]."""
    rng = np.random.default_rng(seed)
    npg = [-(-n // 16) for n in seq_keys]
    total = sum(npg) + extra
    perm = rng.permutation(total)
    table = np.zeros((len(seq_keys), max(npg)), np.int32)
    at = 0
    for i, n in enumerate(npg):
        table[i, :n] = perm[at:at + n]
        at += n
    pool = normal_bf16((total, Hkv, 2, 16 * 128), seed=seed + 1)
    return pool, table


def _run(q, pool, table, chunks, H=32, Hkv=4):
    plan = ops.prefill_plan(chunks, H, Hkv, DEV)
    out = ops.paged_prefill_attention(bf16_tensor(q, DEV), bf16_tensor(pool, DEV),
                                      torch.from_numpy(table).to(DEV), plan, SCALE)
    return u16(out)


@pytest.mark.parametrize("H,Hkv", [(32, 4), (16, 1), (8, 8)])
def test_prefill_attention_parity(H, Hkv):
    # chunks: from position 0, a context ending mid-page, one token, a long context, a chunk
    # whose keys end exactly on a 32-key step
    chunks = [(0, 0, 37), (1, 100, 64), (2, 1500, 1), (3, 4093, 70), (4, 16, 16)]
    keys = [ctx + n for _, ctx, n in chunks]
    pool, table = _pool(keys, seed=H + Hkv, Hkv=Hkv)
    T = sum(n for *_, n in chunks)
    q = normal_bf16((T, H, 128), seed=5)
    got = _run(q, pool, table, chunks, H, Hkv)
    want, exact = oracle.paged_prefill_attn(q, pool, table, chunks, SCALE, exact=True)
    assert_attention_parity(got, exact, what=f"prefill H={H} Hkv={Hkv}")
    assert_close_bf16(got, want, what=f"prefill H={H} Hkv={Hkv}")


def test_prefill_token_result_is_independent_of_the_chunking():
    """A token's bits depend only on its q row and its keys: the same 90 positions prefilled as
    one chunk, as two chunks, or decoded row by row through prefill chunks of one token agree."""
    pool, table = _pool([300], seed=11)
    q = normal_bf16((90, 32, 128), seed=12)
    whole = _run(q, pool, table, [(0, 210, 90)])
    split = _run(q, pool, table, [(0, 210, 41), (0, 251, 49)])
    assert np.array_equal(whole, split)
    single = _run(q[57:58], pool, table, [(0, 267, 1)])
    assert np.array_equal(single[0], whole[57])


def test_prefill_key_parts_keep_results_independent_of_the_chunking():
    """Keys are cut into parts at multiples of jit_prefill_part_keys (6,144): tokens past a cut are
    merged from per-part partials.  The cuts sit at key positions, so a token's bits still do not
    depend on the chunking: positions 6,100 .. 6,229 (around the first cut) as one chunk, as two
    chunks split at the cut and off it, and as one-token chunks agree; and the oracle agrees."""
    assert int(ops._lib.lib().jit_prefill_part_keys()) == 6144
    pool, table = _pool([6230], seed=81)
    q = normal_bf16((130, 32, 128), seed=82)
    whole = _run(q, pool, table, [(0, 6100, 130)])
    assert np.array_equal(whole, _run(q, pool, table, [(0, 6100, 44), (0, 6144, 86)]))
    assert np.array_equal(whole, _run(q, pool, table, [(0, 6100, 71), (0, 6171, 59)]))
    for i in (0, 43, 44, 45, 129):
        assert np.array_equal(_run(q[i:i + 1], pool, table, [(0, 6100 + i, 1)])[0], whole[i]), i
    sel = np.r_[40:48, 120:130]
    want, exact = oracle.paged_decode_attn(q[sel], pool, table[np.zeros(sel.size, int)], 6100 + sel + 1, SCALE,
                                           exact=True)
    assert_attention_parity(whole[sel], exact, what="prefill across the first key cut")
    assert_close_bf16(whole[sel], want, what="prefill across the first key cut")


def test_prefill_three_key_parts_and_a_mixed_plan():
    """Tokens of three key parts (past 12,288) beside a chunk of one part in the same launch."""
    chunks = [(0, 12270, 40), (1, 30, 50)]
    pool, table = _pool([12310, 80], seed=91)
    q = normal_bf16((90, 32, 128), seed=92)
    plan = ops.prefill_plan(chunks, 32, 4, DEV)
    assert plan.pmax == 3
    got = _run(q, pool, table, chunks)
    sel = np.r_[0:4, 16:22, 36:40, 40:44, 86:90]
    seqs = np.where(sel < 40, 0, 1)
    lens = np.where(sel < 40, 12270 + sel + 1, 30 + (sel - 40) + 1)
    want, exact = oracle.paged_decode_attn(q[sel], pool, table[seqs], lens.astype(np.int32), SCALE, exact=True)
    assert_attention_parity(got[sel], exact, what="prefill of three key parts")
    assert_close_bf16(got[sel], want, what="prefill of three key parts")


def test_prefill_one_token_matches_decode_attention():
    """A one-token chunk at position p is decode attention over p + 1 keys (both within the
    tolerance of the same oracle row, and close to each other)."""
    pool, table = _pool([2000], seed=21)
    q = normal_bf16((1, 32, 128), seed=22)
    pre = _run(q, pool, table, [(0, 1799, 1)])
    plan = ops.attn_plan([1800], DEV)
    dec = u16(ops.paged_decode_attention(bf16_tensor(q, DEV), bf16_tensor(pool, DEV),
                                         torch.from_numpy(table).to(DEV), plan, SCALE))
    want, exact = oracle.paged_decode_attn(q, pool, table, [1800], SCALE, exact=True)
    assert_attention_parity(pre, exact, what="prefill one token")
    assert_attention_parity(dec, exact, what="decode one token")
    assert_close_bf16(pre, want, what="prefill one token")
    assert np.mean(pre == dec) >= 0.98


def test_prefill_page_permutation_and_stale_slots():
    """Moving the pages leaves the bits unchanged, and NaN bits in slots past the last key (a
    page's unwritten tail) do not reach the output."""
    chunks = [(0, 5, 23), (1, 700, 9)]
    pool, table = _pool([28, 709], seed=31)
    q = normal_bf16((32, 32, 128), seed=32)
    base = _run(q, pool, table, chunks)
    poisoned = pool.copy()
    for seq, n in ((0, 28), (1, 709)):  # slots n % 16 .. 15 of the last page (K chunk-major, V dim-major)
        pg = table[seq, (n - 1) // 16]
        k = poisoned[pg, :, 0].reshape(4, 4, 16, 32)
        k[:, :, n % 16:, :] = 0x7FC0
        v = poisoned[pg, :, 1].reshape(4, 128, 16)
        v[:, :, n % 16:] = 0x7FC0
    assert np.array_equal(_run(q, poisoned, table, chunks), base)
    perm = np.random.default_rng(33).permutation(pool.shape[0])
    pool2 = np.empty_like(pool)
    pool2[perm] = pool
    assert np.array_equal(_run(q, pool2, perm[table].astype(np.int32), chunks), base)


def test_prefill_config3_chunks():
    """BASELINE config 3's prefill half: 4 chunks of 512 tokens after contexts up to 8,192."""
    rng = np.random.default_rng(0x4A450030)
    ctx = rng.integers(0, 8193, 4)
    chunks = [(i, int(c), 512) for i, c in enumerate(ctx)]
    pool, table = _pool([int(c) + 512 for c in ctx], seed=41)
    q = normal_bf16((2048, 32, 128), seed=42)
    got = _run(q, pool, table, chunks)
    sel = np.r_[0:40, 500:560, 1024:1030, 2000:2048]  # rows across every chunk (the oracle is O(T.L))
    lens = np.array([int(ctx[r // 512]) + r % 512 + 1 for r in sel], np.int32)
    want, exact = oracle.paged_decode_attn(q[sel], pool, table[sel // 512], lens, SCALE, exact=True)
    assert_attention_parity(got[sel], exact, what="config 3 prefill")
    assert_close_bf16(got[sel], want, what="config 3 prefill")


def test_mixed_prefill_decode_layer_stages():
    """One mixed chunked-prefill + decode step of a decoder layer (config 3's shape, small): the
    attention rows against the oracle on the step's own q and pool, and the MoE half (segment GEMM)
    against the oracle's expert chain on the step's own normed rows."""
    from jitengine_amd.model import DecoderLayer, MoEConfig, make_mixed_state, random_layer_weights

    cfg = MoEConfig(experts=32, layers=1)
    chunks = [(0, 30, 40), (1, 0, 21), (2, 511, 64)]
    dec_pos = [100, 7, 3000]
    seq_keys = [ctx + n for _, ctx, n in chunks] + [p + 1 for p in dec_pos]
    pool, table = _pool(seq_keys, seed=51)
    w = random_layer_weights(cfg, seed=52, device=DEV)
    layer = DecoderLayer(cfg, w)
    ms = make_mixed_state(cfg, chunks, table[:3], dec_pos, table[3:], DEV)
    T = ms.P + len(dec_pos)
    x = bf16_tensor(normal_bf16((T, cfg.hidden), seed=53), DEV)
    pt = bf16_tensor(pool, DEV)
    dbg = {}
    y = layer.mixed(x, pt, ms, debug=dbg)
    torch.cuda.synchronize()
    assert layer.moe.use_seg(T * cfg.top_k, prefill=True)
    q, attn, pool_after = u16(dbg["q"]), u16(dbg["attn"]), u16(pt)
    want_pre, ex_pre = oracle.paged_prefill_attn(q[:ms.P], pool_after, table[:3], chunks, SCALE, exact=True)
    assert_attention_parity(attn[:ms.P], ex_pre, what="mixed step prefill rows")
    assert_close_bf16(attn[:ms.P], want_pre, what="mixed step prefill rows")
    want_dec, ex_dec = oracle.paged_decode_attn(q[ms.P:], pool_after, table[3:], np.array(dec_pos) + 1, SCALE,
                                                exact=True)
    assert_attention_parity(attn[ms.P:], ex_dec, what="mixed step decode rows")
    assert_close_bf16(attn[ms.P:], want_dec, what="mixed step decode rows")

    def host_q(lin):
        return (lin.weight.cpu().numpy().view(np.uint32), u16(lin.scales), u16(lin.biases))

    hn = u16(dbg["hn"])
    wi = dbg["inds"].cpu().numpy().view(np.uint32)
    pk = oracle.moe_pack(wi, cfg.experts)
    h = oracle.moe_gate_up(hn, wi, pk, *host_q(w["gate_up"]), bf16w=True)
    r = oracle.moe_down(h, wi, pk, *host_q(w["down"]), bf16w=True)
    moe = oracle.moe_combine(r, pk["inv"], u16(dbg["scores"]))
    want_y = oracle.f32_to_bf16(bf16_to_f32(u16(dbg["h"])) + bf16_to_f32(moe))
    assert_close_bf16(u16(y), want_y, what="mixed step output")


def test_prefill_and_mixed_step_past_4096_pages():
    """Contexts beyond 65,536 keys (4,096 pages, the page ids a prefill work item stages in LDS): a
    prefill chunk after 70,000 tokens reads its later page ids from the table, and a mixed step carries
    a decode row of 70,001 keys beside a short chunk; both against the oracle."""
    from jitengine_amd.model import DecoderLayer, MoEConfig, make_mixed_state, random_layer_weights

    pool, table = _pool([70040], seed=71)
    q = normal_bf16((40, 32, 128), seed=72)
    got = _run(q, pool, table, [(0, 70000, 40)])
    sel = np.array([0, 13, 39])
    want, exact = oracle.paged_decode_attn(q[sel], pool, table[[0, 0, 0]], 70000 + sel + 1, SCALE, exact=True)
    assert_attention_parity(got[sel], exact, what="prefill past 4096 pages")
    assert_close_bf16(got[sel], want, what="prefill past 4096 pages")

    cfg = MoEConfig(experts=32, layers=1)
    chunks = [(0, 100, 30)]
    dec_pos = [70000]
    pool, table = _pool([130, 70001], seed=73)
    w = random_layer_weights(cfg, seed=74, device=DEV)
    layer = DecoderLayer(cfg, w)
    ms = make_mixed_state(cfg, chunks, table[:1], dec_pos, table[1:], DEV)
    x = bf16_tensor(normal_bf16((31, cfg.hidden), seed=75), DEV)
    pt = bf16_tensor(pool, DEV)
    dbg = {}
    layer.mixed(x, pt, ms, debug=dbg)
    torch.cuda.synchronize()
    qh, attn, pool_after = u16(dbg["q"]), u16(dbg["attn"]), u16(pt)
    _, ex_pre = oracle.paged_prefill_attn(qh[:30], pool_after, table[:1], chunks, SCALE, exact=True)
    assert_attention_parity(attn[:30], ex_pre, what="mixed prefill rows")
    _, ex_dec = oracle.paged_decode_attn(qh[30:], pool_after, table[1:], np.array(dec_pos) + 1, SCALE, exact=True)
    assert_attention_parity(attn[30:], ex_dec, what="mixed decode row of 70,001 keys")
