"""HIP path vs the CPU oracle on the same seeded inputs (MI355X only).

Integer outputs (expert ids, packing tables, KV bytes) must be bit-exact; bf16 outputs must meet
the north-star tolerance (max-abs <= 2e-2, cosine >= 0.9995) and, for the quantized projections,
the reference's own criterion (FN/kernels/selfcheck.py:313-331): the kernel's largest error against
the float64 result is at most 8x that of the reference's fp32 arithmetic (restated in
oracle.qmv_mlx_f32, rounded to bf16 as the reference returns it) plus 4 fp32 ulps of the scale."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from jitengine_amd import ops
from jitengine_amd.moe import MoEBlock
from jitengine_amd.quant import QLinear
from tests.helpers import (
    assert_attention_parity, assert_close_bf16, assert_fn_criterion, bf16_tensor, bf16_to_f32, f32_to_bf16, make_stack,
    normal_bf16, router_logits, stack_np, tie_gates, u16,
)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _i32(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(DEV)


def _dev(q: QLinear) -> QLinear:
    return q.to(DEV)


# ----------------------------------------------------------------------------- router
@pytest.mark.parametrize("N", [128, 256])
@pytest.mark.parametrize("norm", [True, False])
def test_router_topk_bit_exact(N, norm):
    for t in range(24):
        B = 1 + t % 8
        lg = router_logits(t % 4, B, N, seed=3000 + t)
        inds, scores, gates = ops.router_topk(bf16_tensor(lg, DEV), 8, norm, gates_out=True)
        wi, ws, wg = oracle.router_topk(lg, 8, norm)
        assert np.array_equal(u16(gates), wg), t
        assert np.array_equal(inds.cpu().numpy().view(np.uint32), wi), t
        assert np.array_equal(u16(scores), ws), t


@pytest.mark.parametrize("B", [64, 32, 2108, 1])
def test_router_topk_config_rows(B):
    lg = router_logits(2 if B == 1 else 0, B, 128, seed=B)
    inds, scores = ops.router_topk(bf16_tensor(lg, DEV), 8, True)
    wi, ws, _ = oracle.router_topk(lg, 8, True)
    assert np.array_equal(inds.cpu().numpy().view(np.uint32), wi)
    assert np.array_equal(u16(scores), ws)


@pytest.mark.parametrize("N,k", [(128, 64), (128, 65), (256, 100), (1024, 200)])
@pytest.mark.parametrize("norm", [True, False])
def test_router_topk_wide_k_bit_exact(N, k, norm):
    """Both slot paths of the top-k: k <= 64 keeps slot j in lane j, more slots go through LDS."""
    for t in range(6):
        lg = router_logits(t % 4, 1 + t % 3, N, seed=5000 + N + k + t)
        inds, scores = ops.router_topk(bf16_tensor(lg, DEV), k, norm)
        wi, ws, _ = oracle.router_topk(lg, k, norm)
        assert np.array_equal(inds.cpu().numpy().view(np.uint32), wi), t
        assert np.array_equal(u16(scores), ws), t


@pytest.mark.parametrize("N,k", [(256, 8), (128, 8), (1024, 16), (64, 64), (1024, 100)])
def test_topk_from_gates_bit_exact(N, k):
    for t in range(12):
        g = tie_gates(3, N, seed=400 + t) if t % 2 else oracle.softmax_bf16(router_logits(t % 4, 3, N, seed=400 + t))
        got = ops.topk(bf16_tensor(g, DEV), k).cpu().numpy().view(np.uint32)
        assert np.array_equal(got, oracle.topk_from_gates(g, k)), t


# ----------------------------------------------------------------------------- packing
@pytest.mark.parametrize("rows,N", [(1, 128), (2, 128), (3, 64), (4, 128), (4, 32), (1, 96)])
def test_route_pack_equals_two_launches(rows, N):
    """The one-launch top-k + packing of a small step gives the two launches' bits."""
    for t in range(6):
        lg = bf16_tensor(router_logits(t % 4, rows, N, seed=700 + 10 * rows + t), DEV)
        for norm in (True, False):
            i2, s2 = ops.router_topk(lg, 8, norm)
            p2 = ops.moe_pack(i2, N)
            i1, s1, p1 = ops.route_pack(lg, 8, norm)
            assert torch.equal(i1, i2) and torch.equal(s1.view(torch.int16), s2.view(torch.int16)), (t, norm)
            U = int(p2.meta[0])
            for name in ("order", "pair_row", "inv", "expert_cnt", "expert_off", "meta"):
                assert torch.equal(getattr(p1, name), getattr(p2, name)), (name, t)
            for name in ("seg_expert", "seg_start", "seg_cnt"):
                assert torch.equal(getattr(p1, name)[:U], getattr(p2, name)[:U]), (name, t)


@pytest.mark.parametrize("B,k,E", [(64, 8, 128), (32, 8, 128), (1, 8, 128), (2108, 8, 128), (300, 5, 7), (3, 8, 1024)])
def test_pack_bit_exact(B, k, E):
    rng = np.random.default_rng(B + E)
    if E < k:
        inds = rng.integers(0, E, (B, k)).astype(np.uint32)
    else:
        inds = np.stack([rng.permutation(E)[:k] for _ in range(B)]).astype(np.uint32)
    pk = ops.moe_pack(_i32(inds), E)
    want = oracle.moe_pack(inds, E)
    U = int(want["meta"][0])
    for name in ("order", "pair_row", "inv", "expert_cnt", "expert_off"):
        assert np.array_equal(getattr(pk, name).cpu().numpy(), want[name]), name
    for name in ("seg_expert", "seg_start", "seg_cnt"):
        assert np.array_equal(getattr(pk, name).cpu().numpy()[:U], want[name][:U]), name
    meta = pk.meta.cpu().numpy()
    assert meta[0] == U and meta[1] == want["meta"][1] and meta[2] == 0


@pytest.mark.parametrize("P,k,E,skew,bad", [(2056, 8, 128, False, 0), (16864, 8, 128, True, 0),
                                             (50000, 5, 1023, True, 37), (3072, 1, 64, False, 5)])
def test_pack_many_workgroups_equal_one(P, k, E, skew, bad):
    """A long batch's three-launch packing (jit_moe_pack_ws) gives the one-workgroup kernel's
    tables bit for bit: skewed routing (segments of thousands of pairs), ids past E (dropped,
    inv = -1, counted in meta[2]), tiles that do not divide P."""
    from jitengine_amd import _lib

    rng = np.random.default_rng(P + E)
    w = 1.0 / (1.0 + np.arange(E)) ** (1.2 if skew else 0.0)
    inds = rng.choice(E, P, p=w / w.sum()).astype(np.uint32)
    inds[rng.permutation(P)[:bad]] = E + rng.integers(0, 50, bad).astype(np.uint32)
    t = _i32(inds.reshape(-1, k))
    assert _lib.lib().jit_moe_pack_workspace_bytes(P, E) > 0
    multi = ops.moe_pack(t, E)
    one = ops._packing_buffers(P, k, E, DEV)
    _lib.check(_lib.lib().jit_moe_pack(ops._p(t), P, k, E, *[ops._p(getattr(one, n)) for n in (
        "order", "pair_row", "inv", "expert_cnt", "expert_off", "seg_expert", "seg_start", "seg_cnt", "meta")],
        ops._stream()), "moe_pack")
    U = int(one.meta[0])
    valid = int(one.expert_cnt.sum())
    assert valid == P - bad and int(one.meta[2]) == bad
    for name in ("pair_row", "order"):
        assert torch.equal(getattr(multi, name)[:valid], getattr(one, name)[:valid]), name
    for name in ("inv", "expert_cnt", "expert_off", "meta"):
        assert torch.equal(getattr(multi, name), getattr(one, name)), name
    for name in ("seg_expert", "seg_start", "seg_cnt"):
        assert torch.equal(getattr(multi, name)[:U], getattr(one, name)[:U]), name
    if bad == 0:  # (the oracle rejects ids past E)
        want = oracle.moe_pack(inds.reshape(-1, k), E)
        assert np.array_equal(multi.inv.cpu().numpy(), want["inv"])


# ----------------------------------------------------------------------------- projections
@pytest.mark.parametrize("T", [1, 3, 16, 17, 40])
@pytest.mark.parametrize("N,K", [(128, 2048), (512, 2048), (256, 4096), (2048, 768 + 256)])
def test_qmm_parity(T, N, K):
    q = make_stack((N, K), seed=N + K)
    w, s, b = stack_np(q)
    x = normal_bf16((T, K), seed=T)
    y = ops.qmm(bf16_tensor(x, DEV), _dev(q))
    f64, want = oracle.qmm(x, w, s, b)
    assert_close_bf16(u16(y), want, what="qmm")
    if K % 512 == 0:
        assert_fn_criterion(u16(y), x, w, s, b, f64)


def _moe_inputs(B, E, D, I, seed):
    gu = make_stack((E, 2 * I, D), seed=seed + 1)
    dn = make_stack((E, D, I), seed=seed + 2)
    x = normal_bf16((B, D), seed=seed + 3)
    inds, scores, _ = oracle.router_topk(router_logits(0, B, E, seed=seed + 4), 8, True)
    return gu, dn, x, inds, scores


def _swiglu_np(g, u):
    """The oracle's SwiGLU rounding chain, vectorised (checked bit-exact against it below): the
    oracle's SigmoidX steps, then bf16(g * sigmoid) and bf16(sl * u)."""
    sg = oracle.sigmoid_bf16(g)
    with np.errstate(over="ignore", invalid="ignore"):  # inf and NaN gates are part of the domain
        sl = oracle.f32_to_bf16(bf16_to_f32(g) * bf16_to_f32(sg))
        return oracle.f32_to_bf16(bf16_to_f32(sl) * bf16_to_f32(u))


def _bf16_neighbours(b):
    """The bf16 values one ulp either side of each bit pattern (sign-magnitude order)."""
    b = b.astype(np.int32)
    mag, neg = b & 0x7FFF, (b & 0x8000) != 0
    up = np.where(neg, np.where(mag > 0, b - 1, 0x0001), b + 1)      # towards +inf
    dn = np.where(neg, b + 1, np.where(mag > 0, b - 1, 0x8001))      # towards -inf
    return up.astype(np.uint16), dn.astype(np.uint16)


def test_swiglu_exhaustive_over_bf16_gates():
    """jit_swiglu -- the expert epilogue's SwiGLU on given operands -- gives the oracle's chain
    (SigmoidX's bf16 steps, Q36/kernels/expert_solo.py:56-62,106-115) bit for bit for every bf16
    gate value (65,536 patterns, inf and NaN included; NaN results compare as NaN) against several
    up values and a random up row."""
    g = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ups = [f32_to_bf16(np.full(65536, v, np.float32)) for v in (1.0, -3.5, 0.0078125, 100.0, 1e-30)]
    ups.append(normal_bf16((65536,), seed=99, scale=3.0))
    gt = bf16_tensor(g, DEV)
    for u in ups:
        got = u16(ops.swiglu(gt, bf16_tensor(u, DEV)))
        want = _swiglu_np(g, u)
        nan = np.isnan(bf16_to_f32(want))
        assert np.array_equal(np.isnan(bf16_to_f32(got)), nan)
        bad = np.flatnonzero((got != want) & ~nan)
        assert bad.size == 0, [(hex(g[i]), hex(u[i]), hex(got[i]), hex(want[i])) for i in bad[:8]]
    odd = normal_bf16((1001,), seed=5)  # a length that is not a multiple of 8: the scalar tail
    assert np.array_equal(u16(ops.swiglu(bf16_tensor(odd, DEV), bf16_tensor(odd[::-1].copy(), DEV))),
                          _swiglu_np(odd, odd[::-1].copy()))


@pytest.mark.parametrize("B,E", [(64, 16), (5, 16), (1, 128), (300, 8)])
def test_gate_up_swiglu_parity(B, E):
    """Every h is the reference's SwiGLU chain -- g, u (the float64 projections) rounded to
    bf16, SigmoidX's bf16 steps (Q36/kernels/expert_solo.py:56-62), bf16(g * sigmoid) * u
    rounded -- exactly, on the kernel's own g and u: those accumulate in fp32, so each may land
    one bf16 ulp from the float64 value's rounding, and nothing else may differ; (300, 8) gives
    experts more than 16 tokens (several token tiles per weight slice)."""
    gu, dn, x, inds, scores = _moe_inputs(B, E, 2048, 768, seed=50 + B)
    pk = ops.moe_pack(_i32(inds), E)
    h = u16(ops.expert_gate_up(bf16_tensor(x, DEV), _dev(gu), pk))
    opk = oracle.moe_pack(inds, E)
    want = oracle.moe_gate_up(x, inds, opk, *stack_np(gu))
    st = assert_close_bf16(h, want, what="gate_up", ulps=4.0)
    assert st["bit_equal"] > 0.95, st
    w, s, b = stack_np(gu)
    I = w.shape[1] // 2
    flat = inds.reshape(-1)
    g = np.empty_like(want)
    u = np.empty_like(want)
    for e in range(E):
        ps = np.nonzero(flat[opk["order"]] == e)[0]
        if ps.size == 0:
            continue
        rows = opk["pair_row"][ps]
        g[ps] = oracle.qmm(x[rows], w[e, :I], s[e, :I], b[e, :I])[1]
        u[ps] = oracle.qmm(x[rows], w[e, I:], s[e, I:], b[e, I:])[1]
    assert np.array_equal(_swiglu_np(g, u), want)
    ok = np.zeros(h.shape, bool)
    for gg in (g, *_bf16_neighbours(g)):
        for uu in (u, *_bf16_neighbours(u)):
            ok |= _swiglu_np(gg, uu) == h
    # near zero (|g| or |u| ~ 1e-5) the fp32 accumulation's absolute error (~1e-6) spans many
    # bf16 ulps: there the h values must agree to 2^-12 absolute instead
    ok |= np.abs(bf16_to_f32(h).astype(np.float64) - bf16_to_f32(want)) <= 2.0**-12
    bad = np.argwhere(~ok)[:6]
    detail = [(tuple(i), float(bf16_to_f32(g[tuple(i)])), float(bf16_to_f32(u[tuple(i)])),
               float(bf16_to_f32(h[tuple(i)])), float(bf16_to_f32(want[tuple(i)]))) for i in bad]
    assert ok.all(), (f"{(~ok).sum()} of {ok.size} h values are neither the chain on g, u within one ulp "
                      f"nor within 2^-12 (index, g, u, h_gpu, h_oracle): {detail}")
    assert st["bit_equal"] > 0.97, st


@pytest.mark.parametrize("B,E", [(64, 16), (7, 128)])
def test_down_parity(B, E):
    gu, dn, x, inds, scores = _moe_inputs(B, E, 2048, 768, seed=70 + B)
    opk = oracle.moe_pack(inds, E)
    h = oracle.moe_gate_up(x, inds, opk, *stack_np(gu))
    pk = ops.moe_pack(_i32(inds), E)
    r = ops.expert_down(bf16_tensor(h, DEV), _dev(dn), pk)
    want = oracle.moe_down(h, inds, opk, *stack_np(dn))
    st = assert_close_bf16(u16(r), want, what="down")
    assert st["bit_equal"] > 0.95, st


@pytest.mark.parametrize("resid", [False, True])
def test_combine_bit_exact(resid):
    B, k, D, E = 33, 8, 2048, 128
    rng = np.random.default_rng(5)
    inds = np.stack([rng.permutation(E)[:k] for _ in range(B)]).astype(np.uint32)
    scores = oracle.router_topk(router_logits(1, B, E, seed=6), k, True)[1]
    r = normal_bf16((B * k, D), seed=7)
    pk = ops.moe_pack(_i32(inds), E)
    rs = normal_bf16((B, D), seed=8)
    y = ops.moe_combine(bf16_tensor(r, DEV), pk, bf16_tensor(scores, DEV), bf16_tensor(rs, DEV) if resid else None)
    want = oracle.moe_combine(r, oracle.moe_pack(inds, E)["inv"], scores)
    if resid:
        want = oracle.f32_to_bf16(bf16_to_f32(rs) + bf16_to_f32(want))
    assert np.array_equal(u16(y), want)


def test_moe_block_chain():
    """Router logits -> top-k -> experts -> combine + residual, each stage checked against the
    oracle applied to the GPU's own input of that stage (routing is bit-exact given the logits)."""
    B, E, D, I = 48, 32, 2048, 768
    router = make_stack((E, D), seed=91)
    gu = make_stack((E, 2 * I, D), seed=92)
    dn = make_stack((E, D, I), seed=93)
    blk = MoEBlock(_dev(router), _dev(gu), _dev(dn), top_k=8)
    x = normal_bf16((B, D), seed=94)
    res = normal_bf16((B, D), seed=95)
    xt = bf16_tensor(x, DEV)
    logits = ops.qmm(xt, blk.router)
    _, want_logits = oracle.qmm(x, *stack_np(router))
    assert_close_bf16(u16(logits), want_logits, what="router logits")
    inds, scores = ops.router_topk(logits, 8, True)
    wi, ws, _ = oracle.router_topk(u16(logits), 8, True)
    assert np.array_equal(inds.cpu().numpy().view(np.uint32), wi)
    assert np.array_equal(u16(scores), ws)
    y = blk.experts(xt, inds, scores, bf16_tensor(res, DEV))
    out = oracle.moe_experts(x, wi, ws, stack_np(gu), stack_np(dn), E)
    want = oracle.f32_to_bf16(bf16_to_f32(res) + bf16_to_f32(out["y"]))
    assert_close_bf16(u16(y), want, what="moe block")
    y2 = blk(xt, bf16_tensor(res, DEV))
    assert torch.equal(y2, y)
    direct = MoEBlock(_dev(router), _dev(gu), _dev(dn), top_k=8, prepack=False)
    assert torch.equal(direct(xt, bf16_tensor(res, DEV)), y)


# ----------------------------------------------------------------------------- packed layout
@pytest.mark.parametrize("E,N,K", [(1, 128, 2048), (3, 1536, 2048), (2, 2048, 768), (1, 5120, 2048)])
def test_prepack_bytes_match_oracle(E, N, K):
    q = make_stack((E, N, K), seed=E + N)
    got = ops.prepack(_dev(q)).data.cpu().numpy()
    assert np.array_equal(got, oracle.q4_prepack(*stack_np(q)))


@pytest.mark.parametrize("T,N,K", [(1, 128, 2048), (32, 5120, 2048), (17, 2048, 4096), (5, 256, 768)])
def test_qmm_packed_equals_direct(T, N, K):
    q = _dev(make_stack((N, K), seed=T + N))
    x = bf16_tensor(normal_bf16((T, K), seed=T), DEV)
    assert torch.equal(ops.qmm(x, ops.prepack(q)), ops.qmm(x, q))


@pytest.mark.parametrize("T,N,K", [(192, 256, 2048), (300, 5120, 2048), (2108, 2048, 4096), (161, 512, 768),
                                   (200, 256, 384), (17, 256, 128), (1200, 5120, 2048), (1800, 5120, 2048),
                                   (2108, 5120, 2048)])
def test_qmm_prefill_tile_gemm(T, N, K):
    """A long batch on the prefill tile GEMM (jit_qmm_seg): the reference's prefill arithmetic,
    bf16-dequantized weights with fp32 sums, restated by the oracle's bf16-weight mode (a dense
    matrix is a one-expert stack whose pairs are the rows in order); 161 rows: a partial token
    chunk; K = 384 and 128: an odd number of K steps, and a single one; N = 5120 over 1,200, 1,800
    and 2,108 rows: chunks of 8 and 10 token tiles (the launch sizes them to the CUs)."""
    q = make_stack((N, K), seed=T + K)
    x = normal_bf16((T, K), seed=T)
    y = ops.qmm(bf16_tensor(x, DEV), ops.prepack(_dev(q)), seg=True)
    inds = np.zeros((T, 1), np.uint32)
    w, s_, b = stack_np(q)
    want = oracle.moe_down(x, inds, oracle.moe_pack(inds, 1), w[None], s_[None], b[None], bf16w=True)
    st = assert_close_bf16(u16(y), want, what=f"qmm_seg T={T} N={N} K={K}")
    assert st["bit_equal"] > 0.9, st
    if T >= ops.QMM_SEG_MIN_ROWS:  # the automatic switch takes it too
        assert torch.equal(ops.qmm(bf16_tensor(x, DEV), ops.prepack(_dev(q))), y)


@pytest.mark.parametrize("B,E", [(64, 128), (300, 8), (1, 16)])
def test_expert_paths_packed_equal_direct(B, E):
    gu, dn, x, inds, scores = _moe_inputs(B, E, 2048, 768, seed=60 + B)
    pk = ops.moe_pack(_i32(inds), E)
    xt = bf16_tensor(x, DEV)
    gud, dnd = _dev(gu), _dev(dn)
    h = ops.expert_gate_up(xt, gud, pk)
    assert torch.equal(ops.expert_gate_up(xt, ops.prepack(gud), pk), h)
    assert torch.equal(ops.expert_down(h, ops.prepack(dnd), pk), ops.expert_down(h, dnd, pk))


# ----------------------------------------------------------------------------- paged KV
def _pool(lens, seed, Hkv=4, H=32, extra=5):
    rng = np.random.default_rng(seed)
    npg = [-(-L // 16) for L in lens]
    total = sum(npg) + extra
    perm = rng.permutation(total)
    table = np.zeros((len(lens), max(npg)), np.int32)
    at = 0
    for i, n in enumerate(npg):
        table[i, :n] = perm[at:at + n]
        at += n
    pool = normal_bf16((total, Hkv, 2, 16 * 128), seed=seed + 1)
    q = normal_bf16((len(lens), H, 128), seed=seed + 2)
    return q, pool, table


def test_kv_append_bit_exact():
    lens = [5, 40, 17, 1]
    _, pool, table = _pool(lens, seed=11)
    k = normal_bf16((4, 4, 128), seed=12)
    v = normal_bf16((4, 4, 128), seed=13)
    pos = np.array([4, 39, 16, 0], np.int32)
    pt = bf16_tensor(pool, DEV)
    ops.kv_append_paged(pt, bf16_tensor(k, DEV), bf16_tensor(v, DEV), _i32(pos), _i32(table))
    want = pool.copy()
    oracle.kv_append_paged(want, k, v, pos, table)
    assert np.array_equal(u16(pt), want)


LENS = [1, 7, 16, 17, 31, 32, 33, 255, 256, 257, 300, 383, 384, 385, 769, 1023, 1024, 1152, 1500, 1535, 1536, 1537,
        3072, 3073, 4095, 4096, 6000, 9000, 16384, 16385, 20000]


def _attn(q, pool, table, lens, scale=128 ** -0.5):
    plan = ops.attn_plan(lens, DEV)
    out = ops.paged_decode_attention(bf16_tensor(q, DEV), bf16_tensor(pool, DEV), _i32(table), plan, scale)
    return u16(out)


def _attn_bar(got, q, pool, table, lens, what, scale=128 ** -0.5):
    """The attention bar (tests.helpers.assert_attention_parity): the reference's 8x-stock criterion
    against oracle.sdpa_mlx_f32, every element within one ulp + 2^-14 of its row of the float64
    result, and per sequence >= 98% of the outputs equal to the correctly rounded result; plus the
    north star's max-abs / cosine tolerance."""
    want, exact = oracle.paged_decode_attn(q, pool, table, lens, scale, exact=True)
    stock, _ = oracle.sdpa_mlx_f32(q, pool, table, lens, scale)
    st = assert_attention_parity(got, exact, stock, what=what)
    assert_close_bf16(got, want, what=what)
    print(f"{what}: {st}", flush=True)
    return st


def test_paged_attention_parity():
    q, pool, table = _pool(LENS, seed=21)
    got = _attn(q, pool, table, LENS)
    _attn_bar(got, q, pool, table, LENS, "attention, 31 ragged lengths")


@pytest.mark.parametrize("L", [262144, 200003])
def test_paged_attention_long_context(L):
    """BASELINE config 4's shape: one sequence of 262,144 keys in permuted 16-token pages
    (128 chunks of 2048 keys split over 4 waves per kv head, merged in chunk order); and a
    length just past the 1536-key rule (121 chunks of 1664, the last one partial)."""
    q, pool, table = _pool([L], seed=23)
    got = _attn(q, pool, table, [L])
    _attn_bar(got, q, pool, table, [L], f"attention L={L}")


def test_paged_attention_merge_paths_are_per_sequence():
    """A sequence's result does not depend on whether another sequence of the batch is long
    enough (> 32 chunks) to need the merge kernel: the merge path follows each sequence's own
    length."""
    lens = [5000, 60000, 300]  # 60,000 keys = 40 chunks of 1,536
    q, pool, table = _pool(lens, seed=43)
    batched = _attn(q, pool, table, lens)
    for b in (0, 2):
        solo = _attn(q[b:b + 1], pool, table[b:b + 1], lens[b:b + 1])
        assert np.array_equal(solo[0], batched[b]), b
    _attn_bar(batched, q, pool, table, lens, "mixed merge paths")


def test_paged_attention_one_key_is_its_value():
    q, pool, table = _pool([1, 1], seed=31)
    got = _attn(q, pool, table, [1, 1])
    for b in range(2):
        kc, vc = oracle.kv_gather(pool, table[b], 1, 4, 128)
        assert np.array_equal(got[b].reshape(4, 8, 128), np.repeat(vc[:, :1], 8, 1))


def test_paged_attention_batched_row_equals_solo_and_page_permutation():
    lens = [300, 5000, 17, 20000]
    q, pool, table = _pool(lens, seed=41)
    batched = _attn(q, pool, table, lens)
    for b in range(len(lens)):
        solo = _attn(q[b:b + 1], pool, table[b:b + 1], lens[b:b + 1])
        assert np.array_equal(solo[0], batched[b]), b
    perm = np.random.default_rng(42).permutation(pool.shape[0])
    pool2 = np.empty_like(pool)
    pool2[perm] = pool
    assert np.array_equal(_attn(q, pool2, perm[table].astype(np.int32), lens), batched)


def test_paged_attention_gqa_shapes():
    for H, Hkv in [(16, 2), (8, 8), (64, 4)]:
        q, pool, table = _pool([70, 3000], seed=H + Hkv, H=H, Hkv=Hkv)
        got = _attn(q, pool, table, [70, 3000])
        _attn_bar(got, q, pool, table, [70, 3000], f"H={H} Hkv={Hkv}")


def test_empty_batches():
    """Zero rows through every op of the step: empty outputs, no launch, no error."""
    from jitengine_amd.quant import random_quantized

    lg = torch.empty((0, 128), dtype=torch.bfloat16, device=DEV)
    inds, scores = ops.router_topk(lg, 8, True)
    assert inds.shape == (0, 8) and scores.shape == (0, 8)
    pk = ops.moe_pack(inds, 128)
    assert pk.P == 0 and int(pk.expert_cnt.sum()) == 0 and int(pk.meta[0]) == 0
    i1, s1, p1 = ops.route_pack(lg, 8, True)
    assert i1.shape == (0, 8) and int(p1.expert_cnt.sum()) == 0
    lin = ops.prepack(random_quantized((256, 2048), 5, device=DEV))
    assert ops.qmm(torch.empty((0, 2048), dtype=torch.bfloat16, device=DEV), lin).shape == (0, 256)
    assert ops.argmax_rows(torch.empty((0, 1000), dtype=torch.bfloat16, device=DEV)).shape == (0,)
    assert ops.embed_q4(torch.empty(0, dtype=torch.int32, device=DEV),
                        random_quantized((16, 128), 6, device=DEV)).shape == (0, 128)


def test_expert_and_combine_calls_reject_mismatched_packing():
    """Packing tables that do not match the rows they are used with are refused on the host, before a
    kernel could index x, inv or r out of range: x with fewer rows than the tables' tokens, scores of
    another slot count or row count, r of another row count."""
    E, D, I, B, k = 16, 512, 256, 6, 4
    rng = np.random.default_rng(90)
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(B)]).astype(np.int32)
    pk = ops.moe_pack(_i32(inds), E)
    gu = ops.prepack(make_stack((E, 2 * I, D), seed=91).to(DEV))
    x = bf16_tensor(normal_bf16((B, D), seed=92), DEV)
    with pytest.raises(ValueError):
        ops.expert_gate_up(x[:B - 1].contiguous(), gu, pk)
    r = bf16_tensor(normal_bf16((B * k, D), seed=93), DEV)
    scores = bf16_tensor(normal_bf16((B, k), seed=94), DEV)
    w = torch.ones(D, dtype=torch.bfloat16, device=DEV)
    for sc, rr in ((scores[:, :k - 1].contiguous(), r), (scores[:B - 1].contiguous(), r),
                   (torch.cat([scores, scores]), r), (scores, r[:B * k - 1].contiguous())):
        with pytest.raises(ValueError):
            ops.moe_combine(rr, pk, sc)
        with pytest.raises(ValueError):
            ops.moe_combine_rmsnorm(rr, pk, sc, None, w, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(ops.moe_combine(r, pk, scores), ops.moe_combine_rmsnorm(r, pk, scores, None, w, 1e-6)[0])
