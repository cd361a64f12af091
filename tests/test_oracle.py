"""Pins of the CPU oracle (oracle/jit_oracle.c) against what fixes each function independently:
closed forms, library routines (numpy / torch float64 and bf16 ops), known-answer vectors and
invariants.  The reference holds no golden vectors for this path (its tests recompute stock MLX
live, Q36T/metal/kernels/*), so these are the oracle's anchors; the recipes (tie-heavy router
draws, lengths either side of the split-K switch) follow the reference's tests."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import bf16_to_f32, f32_to_bf16, make_stack, normal_bf16, router_logits, stack_np, tie_gates


# ----------------------------------------------------------------------------- bf16 + exp
def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(50000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 50000),
                        np.array([0.0, -0.0, np.inf, -np.inf, 1.0 + 2**-8, 1.0 + 3 * 2**-8], np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(f32_to_bf16(x), want)
    lib = oracle.lib()
    for v in x[:2000]:
        assert lib.jo_f2bf(float(v)) == f32_to_bf16(np.array([v], np.float32))[0]


def test_exp_neg_close_to_exp():
    xs = np.concatenate([np.linspace(-63.99, 0.0, 20001), -np.geomspace(1e-8, 63.0, 2000), [0.0, -1e-30]])
    worst = 0.0
    for x in xs.astype(np.float32):
        got = oracle.exp_neg(float(x))
        want = math.exp(float(x))
        worst = max(worst, abs(got - want) / want)
    assert worst < 4 * 2.0**-24, worst  # within 2 ulp of e^x
    assert oracle.exp_neg(0.0) == 1.0
    assert oracle.exp_neg(-64.0) == 0.0 and oracle.exp_neg(-1e9) == 0.0


def test_exp_pos_close_to_exp():
    xs = np.concatenate([np.linspace(0.0, 88.72, 40001), np.geomspace(1e-8, 88.0, 4000)]).astype(np.float32)
    worst = max(abs(oracle.exp_pos(float(x)) - math.exp(float(x))) / math.exp(float(x)) for x in xs)
    assert worst < 4 * 2.0**-24, worst  # within 2 ulp of e^x
    assert oracle.exp_pos(0.0) == 1.0
    assert math.isinf(oracle.exp_pos(89.5)) and math.isinf(oracle.exp_pos(1e30))
    assert math.isnan(oracle.exp_pos(float("nan")))


def test_sigmoid_steps_exhaustive():
    """SigmoidX's bf16 steps (Q36/kernels/expert_solo.py:56-62) over every finite bf16 g, against an
    independent numpy restatement with float64 exp: e = bf16(exp|g|), d = bf16(1 + e),
    y = bf16(1 / d), g < 0 ? y : bf16(1 - y).  (The oracle's own exp and numpy's differ in the last
    fp32 bits; rounded to bf16 they give the same e on every input here.)  The steps matter: a
    single rounding of the float64 sigmoid differs on over a thousand inputs."""
    g = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    gf = bf16_to_f32(g)
    g, gf = g[np.isfinite(gf)], gf[np.isfinite(gf)]
    got = oracle.sigmoid_bf16(g)
    a = np.abs(gf).astype(np.float64)
    with np.errstate(over="ignore", divide="ignore"):
        e = f32_to_bf16(np.exp(a).astype(np.float32))
        d = f32_to_bf16(np.float32(1) + bf16_to_f32(e))
        y = f32_to_bf16(np.float32(1) / bf16_to_f32(d))
    want = np.where(gf < 0, y, f32_to_bf16(np.float32(1) - bf16_to_f32(y)))
    assert np.array_equal(got, want)
    with np.errstate(over="ignore"):
        yy = 1.0 / (1.0 + np.exp(a))
    single = f32_to_bf16(np.where(gf < 0, yy, 1.0 - yy).astype(np.float32))
    assert np.sum(single != got) > 1000
    # known answers: sigma(0) = 0.5, sigma(+-inf-like) saturates
    h = f32_to_bf16(np.array([0.0, 100.0, -100.0, 1.0], np.float32))
    assert list(bf16_to_f32(oracle.sigmoid_bf16(h))[:3]) == [0.5, 1.0, 0.0]


def test_bf16_reciprocals_are_far_from_bf16_ties():
    """Why the GPU's SigmoidX may take the 1-ulp hardware reciprocal of d = bf16(1 + e): for every
    bf16 significand m, 1 / (m / 128) lies at least 192 fp32 ulps from the nearest bf16 rounding tie,
    so any reciprocal within a few ulps rounds to the bf16 of the correctly rounded division."""
    from fractions import Fraction

    worst = min(
        abs(Fraction(128, m) * 1024 - (2 * round((Fraction(128, m) * 1024 - 1) / 2) + 1)) * 2**14
        for m in range(129, 256)
    )
    assert worst > 192, float(worst)


# ----------------------------------------------------------------------------- router
@pytest.mark.parametrize("N", [32, 128, 256, 1024])
def test_softmax_within_one_ulp_of_float64(N):
    for kind in range(4):
        lg = router_logits(kind, 8, N, seed=10 + kind)
        g = oracle.softmax_bf16(lg)
        x = bf16_to_f32(lg).astype(np.float64)
        p = np.exp(x - x.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        want = bf16_to_f32(f32_to_bf16(p.astype(np.float32))).astype(np.float64)
        got = bf16_to_f32(g).astype(np.float64)
        ulp = np.maximum(np.abs(want), 2.0**-126) * 2.0**-7
        assert np.all(np.abs(got - want) <= ulp + 1e-30), kind


def _argpartition_tail(g_u16: np.ndarray, k: int) -> np.ndarray:
    """The ids MLX's stable argpartition puts last, in its order: a stable ascending sort by value
    (ties keep index order), last k -- numpy's stable argsort is that sort."""
    v = bf16_to_f32(g_u16)
    return np.argsort(v, axis=-1, kind="stable")[..., -k:].astype(np.uint32)


@pytest.mark.parametrize("N,k", [(256, 8), (128, 8), (128, 4), (64, 64), (32, 1)])
def test_topk_rank_rule_equals_stable_sort_tail(N, k):
    for t in range(60):
        if t % 3 == 2:
            g = tie_gates(2, N, seed=1000 + t)
        else:
            g = oracle.softmax_bf16(router_logits(t % 4, 2, N, seed=1000 + t))
        assert np.array_equal(oracle.topk_from_gates(g, k), _argpartition_tail(g, k)), t


def test_topk_contract():
    with pytest.raises(ValueError):
        oracle.topk_from_gates(np.zeros((1, 8), np.uint16), 0)
    with pytest.raises(ValueError):
        oracle.topk_from_gates(np.zeros((1, 8), np.uint16), 9)


@pytest.mark.parametrize("norm", [True, False])
def test_router_is_softmax_topk_gather_and_bf16_renorm(norm):
    for t in range(24):
        lg = router_logits(t % 4, 1 + t % 8, 128, seed=2000 + t)
        inds, scores, gates = oracle.router_topk(lg, 8, norm)
        assert np.array_equal(gates, oracle.softmax_bf16(lg))
        assert np.array_equal(inds, _argpartition_tail(gates, 8))
        sc = torch.from_numpy(np.take_along_axis(gates, inds.astype(np.int64), -1).view(np.int16)).view(torch.bfloat16)
        if norm:
            tot = torch.zeros(sc.shape[0], dtype=torch.bfloat16)
            for j in range(8):  # sequential bf16 sum in slot order
                tot = tot + sc[:, j]
            sc = sc / tot[:, None]
        assert np.array_equal(scores, sc.view(torch.int16).numpy().view(np.uint16))


# ----------------------------------------------------------------------------- packing
@pytest.mark.parametrize("B,k,E", [(64, 8, 128), (32, 8, 128), (1, 8, 128), (200, 8, 16), (5, 3, 7), (0, 8, 128)])
def test_pack_equals_numpy_stable_argsort_and_unique(B, k, E):
    rng = np.random.default_rng(B * 31 + E)
    inds = np.stack([rng.permutation(E)[:k] for _ in range(B)]).astype(np.uint32) if B else np.zeros((0, k), np.uint32)
    if E < 10 and B:
        inds = rng.integers(0, E, (B, k)).astype(np.uint32)  # repeats inside a row too
    pk = oracle.moe_pack(inds, E)
    flat = inds.reshape(-1).astype(np.int64)
    order = np.argsort(flat, kind="stable")
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size)
    uniq, start, cnt = np.unique(flat[order], return_index=True, return_counts=True)
    assert np.array_equal(pk["order"], order)
    assert np.array_equal(pk["inv"], inv)
    assert np.array_equal(pk["pair_row"], order // k)
    U = int(pk["meta"][0])
    assert U == uniq.size and int(pk["meta"][1]) == (int(cnt.max()) if cnt.size else 0)
    assert np.array_equal(pk["seg_expert"][:U], uniq)
    assert np.array_equal(pk["seg_start"][:U], start)
    assert np.array_equal(pk["seg_cnt"][:U], cnt)
    full = np.bincount(flat, minlength=E)
    assert np.array_equal(pk["expert_cnt"], full)
    assert np.array_equal(pk["expert_off"], np.concatenate([[0], np.cumsum(full)[:-1]]))


def test_pack_rejects_bad_ids():
    with pytest.raises(ValueError):
        oracle.moe_pack(np.array([[0, 200]], np.uint32), 128)


# ----------------------------------------------------------------------------- dequant / qmm
def test_dequant_known_answer():
    # word 0x76543210 holds nibbles 0..7 low first; scale 2, bias -1 -> 2q - 1
    w = np.full((1, 8), 0x76543210, np.uint32)
    s = f32_to_bf16(np.array([[2.0]], np.float32))
    b = f32_to_bf16(np.array([[-1.0]], np.float32))
    got = oracle.dequant4(w, s, b)
    assert np.array_equal(got[0], np.tile(2.0 * np.arange(8) - 1.0, 8))
    w2 = np.array([[0xF0000000] + [0] * 7], np.uint32)  # only element 7 is 15
    got2 = oracle.dequant4(w2, f32_to_bf16(np.array([[1.0]], np.float32)), f32_to_bf16(np.array([[0.0]], np.float32)))
    assert got2[0, 7] == 15.0 and got2[0].sum() == 15.0


def test_dequant_matches_independent_unpack():
    q = make_stack((40, 256), seed=3)
    w, s, b = stack_np(q)
    nib = (w.view(np.uint8)[..., None] >> np.array([0, 4], np.uint8)) & 0xF  # bytes, low nibble first
    nib = nib.reshape(40, 256).astype(np.float64)
    want = nib * np.repeat(bf16_to_f32(s), 64, -1) + np.repeat(bf16_to_f32(b), 64, -1)
    assert np.array_equal(oracle.dequant4(w, s, b), want)


def _bf16_weights_numpy(w, s, b):
    """The segment GEMM's weights computed independently: s * q + b is exact in float64 (bf16 s, b
    and q <= 15), its float32 rounding is the fused multiply-add's result, then RNE to bf16."""
    N = w.shape[0]
    nib = ((w.view(np.uint8)[..., None] >> np.array([0, 4], np.uint8)) & 0xF).reshape(N, -1).astype(np.float64)
    exact = nib * np.repeat(bf16_to_f32(s), 64, -1) + np.repeat(bf16_to_f32(b), 64, -1)
    return bf16_to_f32(f32_to_bf16(exact.astype(np.float32))).astype(np.float64), exact


def test_bf16_weights_match_independent_rounding():
    q = make_stack((48, 512), seed=13)
    w, s, b = stack_np(q)
    want, exact = _bf16_weights_numpy(w, s, b)
    got = oracle.dequant4(w, s, b, bf16w=True)
    assert np.array_equal(got, want)
    assert np.any(got != exact)  # the rounding is real at these scales
    assert np.all(np.abs(got - exact) <= 2.0**-8 * np.abs(exact))  # within half a bf16 ulp
    # known answer: 2q - 1 is a bf16 value, so rounding changes nothing
    w1 = np.full((1, 8), 0x76543210, np.uint32)
    one = oracle.dequant4(w1, f32_to_bf16(np.array([[2.0]], np.float32)), f32_to_bf16(np.array([[-1.0]], np.float32)),
                          bf16w=True)
    assert np.array_equal(one[0], np.tile(2.0 * np.arange(8) - 1.0, 8))


def test_qmm_matches_torch_float64_matmul():
    q = make_stack((96, 512), seed=4)
    w, s, b = stack_np(q)
    x = normal_bf16((5, 512), seed=5)
    f, h = oracle.qmm(x, w, s, b)
    nib = ((w.view(np.uint8)[..., None] >> np.array([0, 4], np.uint8)) & 0xF).reshape(96, 512)
    dq = torch.from_numpy(nib.astype(np.float64) * np.repeat(bf16_to_f32(s), 64, -1) + np.repeat(bf16_to_f32(b), 64, -1))
    want = torch.from_numpy(bf16_to_f32(x).astype(np.float64)) @ dq.T
    assert np.allclose(f, want.numpy(), rtol=1e-12, atol=1e-12)
    assert np.array_equal(h, f32_to_bf16(f.astype(np.float32)))


def test_mlx_lane_order_is_fp32_accurate():
    q = make_stack((64, 1024), seed=6)
    w, s, b = stack_np(q)
    x = normal_bf16((3, 1024), seed=7)
    f, _ = oracle.qmm(x, w, s, b)
    m = oracle.qmv_mlx_f32(x, w, s, b).astype(np.float64)
    bound = 1024 * 2.0**-22 * (np.abs(bf16_to_f32(x)).astype(np.float64) @ np.abs(oracle.dequant4(w, s, b)).T)
    assert np.all(np.abs(m - f) <= bound)
    assert np.abs(m - f).max() > 0  # fp32, not float64


# ----------------------------------------------------------------------------- experts
def test_swiglu_within_bf16_rounding_of_exact():
    rng = np.random.default_rng(8)
    g = f32_to_bf16((rng.standard_normal(4000) * 3).astype(np.float32))
    u = f32_to_bf16((rng.standard_normal(4000) * 3).astype(np.float32))
    got = np.array([oracle.swiglu_bf16(a, c) for a, c in zip(g, u)], np.uint16)
    gf, uf = bf16_to_f32(g).astype(np.float64), bf16_to_f32(u).astype(np.float64)
    want = gf / (1 + np.exp(-gf)) * uf
    err = np.abs(bf16_to_f32(got) - want)
    assert np.all(err <= 4 * 2.0**-8 * np.abs(want) + 1e-30)  # three bf16 roundings


def _moe_case(B=24, E=16, D=512, I=256, seed=0):
    gu = make_stack((E, 2 * I, D), seed=seed + 1)
    dn = make_stack((E, D, I), seed=seed + 2)
    x = normal_bf16((B, D), seed=seed + 3)
    lg = router_logits(0, B, E, seed=seed + 4)
    inds, scores, _ = oracle.router_topk(lg, 8, True)
    return x, inds, scores, stack_np(gu), stack_np(dn)


def test_gate_up_equals_per_pair_qmm_and_swiglu():
    x, inds, scores, gu, dn = _moe_case()
    pk = oracle.moe_pack(inds, 16)
    h = oracle.moe_gate_up(x, inds, pk, *gu)
    I = h.shape[1]
    flat = inds.reshape(-1)
    for p in range(0, pk["order"].size, 7):
        e, r = int(flat[pk["order"][p]]), int(pk["pair_row"][p])
        _, g = oracle.qmm(x[r:r + 1], gu[0][e, :I], gu[1][e, :I], gu[2][e, :I])
        _, u = oracle.qmm(x[r:r + 1], gu[0][e, I:], gu[1][e, I:], gu[2][e, I:])
        want = np.array([oracle.swiglu_bf16(a, c) for a, c in zip(g[0], u[0])], np.uint16)
        assert np.array_equal(h[p], want), p


def test_down_and_combine_equal_torch_bf16_composition():
    x, inds, scores, gu, dn = _moe_case(seed=10)
    out = oracle.moe_experts(x, inds, scores, gu, dn, 16)
    pk, h, r = out["pack"], out["h"], out["r"]
    flat = inds.reshape(-1)
    for p in range(0, pk["order"].size, 11):
        e = int(flat[pk["order"][p]])
        _, want = oracle.qmm(h[p:p + 1], dn[0][e], dn[1][e], dn[2][e])
        assert np.array_equal(r[p], want[0])
    rt = torch.from_numpy(r.view(np.int16)).view(torch.bfloat16)
    st = torch.from_numpy(scores.view(np.int16)).view(torch.bfloat16)
    B, k = scores.shape
    y = torch.zeros((B, r.shape[1]), dtype=torch.bfloat16)
    for j in range(k):  # products rounded to bf16, sequential bf16 sum in slot order
        y = y + rt[pk["inv"].reshape(B, k)[:, j]] * st[:, j:j + 1]
    assert np.array_equal(out["y"], y.view(torch.int16).numpy().view(np.uint16))


# ----------------------------------------------------------------------------- paged KV / attention
def _pool_case(lens, Hkv=4, H=32, seed=0, extra_pages=3):
    rng = np.random.default_rng(seed)
    pages_per = [-(-L // 16) for L in lens]
    num_pages = sum(pages_per) + extra_pages
    perm = rng.permutation(num_pages)
    width = max(pages_per)
    table = np.zeros((len(lens), width), np.int32)
    at = 0
    for i, n in enumerate(pages_per):
        table[i, :n] = perm[at:at + n]
        at += n
    pool = normal_bf16((num_pages, Hkv, 2, 16 * 128), seed=seed + 1)
    q = normal_bf16((len(lens), H, 128), seed=seed + 2)
    return q, pool, table


def test_kv_append_gather_round_trip():
    lens = [5, 40, 17]
    _, pool, table = _pool_case(lens, seed=3)
    pool = np.ascontiguousarray(pool)
    k = normal_bf16((3, 4, 128), seed=4)
    v = normal_bf16((3, 4, 128), seed=5)
    pos = np.array([4, 39, 16], np.int32)
    oracle.kv_append_paged(pool, k, v, pos, table)
    for b in range(3):
        kc, vc = oracle.kv_gather(pool, table[b], lens[b], 4, 128)
        assert np.array_equal(kc[:, pos[b]], k[b]) and np.array_equal(vc[:, pos[b]], v[b])
        pg, sl = table[b, pos[b] // 16], pos[b] % 16
        assert np.array_equal(pool[pg, :, 0].reshape(4, 4, 16, 32)[:, :, sl].reshape(4, 128), k[b])  # K chunk-major
        assert np.array_equal(pool[pg, :, 1].reshape(4, 128, 16)[:, :, sl], v[b])  # V dim-major


def test_attention_matches_torch_sdpa_float64():
    lens = [1, 7, 16, 33, 300]
    q, pool, table = _pool_case(lens, seed=6)
    scale = 128 ** -0.5
    out = oracle.paged_decode_attn(q, pool, table, lens, scale)
    for b, L in enumerate(lens):
        kc, vc = oracle.kv_gather(pool, table[b], L, 4, 128)
        qt = torch.from_numpy(bf16_to_f32(q[b]).astype(np.float64)).reshape(1, 32, 1, 128)
        kt = torch.from_numpy(bf16_to_f32(kc).astype(np.float64)).repeat_interleave(8, 0)[None]
        vt = torch.from_numpy(bf16_to_f32(vc).astype(np.float64)).repeat_interleave(8, 0)[None]
        want = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, scale=scale).reshape(32, 128)
        wb = f32_to_bf16(want.numpy().astype(np.float32))
        got = bf16_to_f32(out[b]).astype(np.float64)
        ulp = np.maximum(np.abs(bf16_to_f32(wb)), 1e-30) * 2.0**-7  # one bf16 ulp (summation order)
        assert np.all(np.abs(got - bf16_to_f32(wb)) <= ulp), b
        assert np.mean(out[b] == wb) > 0.99
    # one key: the output is that key's value row, exactly
    kc, vc = oracle.kv_gather(pool, table[0], 1, 4, 128)
    assert np.array_equal(out[0].reshape(4, 8, 128), np.repeat(vc[:, :1], 8, 1))


def test_attention_page_permutation_invariance():
    lens = [50, 130]
    q, pool, table = _pool_case(lens, seed=9)
    a = oracle.paged_decode_attn(q, pool, table, lens, 0.088)
    perm = np.random.default_rng(10).permutation(pool.shape[0])
    pool2 = np.empty_like(pool)
    pool2[perm] = pool
    b = oracle.paged_decode_attn(q, pool2, perm[table].astype(np.int32), lens, 0.088)
    assert np.array_equal(a, b)


def test_attention_float64_output_rounds_to_the_bf16_output():
    lens = [3, 900]
    q, pool, table = _pool_case(lens, seed=12)
    out, out64 = oracle.paged_decode_attn(q, pool, table, lens, 0.088, exact=True)
    assert np.array_equal(f32_to_bf16(out64.astype(np.float32)), out)


def test_sdpa_mlx_f32_pins():
    """The reference's stock arithmetic (an error yardstick only): fp32-accurate in the one-pass
    form (n < 1024), bf16 partials visible in the two-pass form (n >= 1024 on the M4 Pro), one key
    gives its value, pages may move and rows may be batched without changing a bit."""
    lens = [1, 300, 1023, 1024, 5000, 40000]
    q, pool, table = _pool_case(lens, seed=13)
    st, f32 = oracle.sdpa_mlx_f32(q, pool, table, lens, 128 ** -0.5)
    assert np.array_equal(f32_to_bf16(f32), st)
    _, ex = oracle.paged_decode_attn(q, pool, table, lens, 128 ** -0.5, exact=True)
    rel = np.abs(f32 - ex).max(-1) / np.abs(ex).max(-1)  # [B, H]
    assert rel[:3].max() < 2.0**-19, rel[:3].max()       # one pass: fp32 error
    assert rel[3:].max() < 2.0**-8, rel[3:].max()        # two passes: bf16 partials...
    assert rel[3:].max(-1).min() > 2.0**-16              # ...visibly above fp32 error in every row
    kc, vc = oracle.kv_gather(pool, table[0], 1, 4, 128)
    assert np.array_equal(st[0].reshape(4, 8, 128), np.repeat(vc[:, :1], 8, 1))
    perm = np.random.default_rng(14).permutation(pool.shape[0])
    pool2 = np.empty_like(pool)
    pool2[perm] = pool
    st2, _ = oracle.sdpa_mlx_f32(q, pool2, perm[table].astype(np.int32), lens, 128 ** -0.5)
    assert np.array_equal(st2, st)
    solo, _ = oracle.sdpa_mlx_f32(q[4:5], pool, table[4:5], lens[4:5], 128 ** -0.5)
    assert np.array_equal(solo[0], st[4])


# ----------------------------------------------------------------------------- packed layout
def _nibbles(words: np.ndarray) -> np.ndarray:
    """[..., 8] nibbles q0..q7 of uint32 words (bits 4i..4i+3)."""
    return (words[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF


def test_prepack_is_a_permutation_of_words_and_scales():
    """The packed layout holds every MLX word once, with its nibbles reordered so that the
    unpack (shifts by 0, 4, 8, 12 of the 16-bit halves) yields q0..q7 in natural order, and
    every scale and bias once: per (expert, 16-row block) GP nibble tiles of 1 KB, then GP
    scale tiles of 128 B."""
    E, N, K = 2, 32, 256
    GP = K // 128
    rng = np.random.default_rng(11)
    w = rng.integers(0, 2**32, (E, N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = np.arange(E * N * K // 64, dtype=np.uint16).reshape(E, N, K // 64)
    b = (s + 40000).astype(np.uint16)
    out = oracle.q4_prepack(w, s, b)
    assert out.size == E * (N // 16) * GP * 1152
    blocks = out.reshape(-1, GP * 1152)
    words = blocks[:, :GP * 1024].copy().view(np.uint32).ravel()
    # the unpack order: output pair s (s = 0..3) takes bits 4s (low half) and 16 + 4s (high half)
    pk = _nibbles(words)
    unpacked = np.stack([pk[:, 0], pk[:, 4], pk[:, 1], pk[:, 5], pk[:, 2], pk[:, 6], pk[:, 3], pk[:, 7]], -1)
    back = (unpacked.astype(np.uint32) << (4 * np.arange(8, dtype=np.uint32))).sum(-1).astype(np.uint32)
    assert np.array_equal(np.sort(back), np.sort(w.ravel()))  # each word placed exactly once
    sb = blocks[:, GP * 1024:].copy().view(np.uint16).reshape(-1, 16, 4)
    assert np.array_equal(np.sort(sb[..., :2].ravel()), s.ravel())
    assert np.array_equal(np.sort(sb[..., 2:].ravel()), b.ravel())
    # block (e=1, rb=1), pair gp=1, lane 16*2 + 5: row 21, words 2*2, 2*2+1 of groups 2 and 3;
    # the unpacked halves of each are q0..q7 of the MLX word in order
    blk = blocks[1 * 2 + 1]
    lane = blk[1024 * 1 + 16 * (16 * 2 + 5):1024 * 1 + 16 * (16 * 2 + 6)].copy().view(np.uint32)
    want = [w[1, 21, 8 * 2 + 4], w[1, 21, 8 * 2 + 5], w[1, 21, 8 * 3 + 4], w[1, 21, 8 * 3 + 5]]
    for got_w, want_w in zip(lane, want):
        halves = [(int(got_w) >> (4 * i)) & 0xF for i in (0, 4, 1, 5, 2, 6, 3, 7)]
        assert halves == [(int(want_w) >> (4 * i)) & 0xF for i in range(8)]
    sc = blk[GP * 1024 + 128 * 1 + 8 * 5:GP * 1024 + 128 * 1 + 8 * 6].copy().view(np.uint16)
    assert list(sc) == [s[1, 21, 2], s[1, 21, 3], b[1, 21, 2], b[1, 21, 3]]


# ----------------------------------------------------------------------------- decoder block glue
def test_rmsnorm_matches_torch_rms_norm_float64():
    x = normal_bf16((6, 2048), seed=70, scale=3.0)
    w = f32_to_bf16((1 + 0.02 * np.random.default_rng(71).standard_normal(2048)).astype(np.float32))
    y, _ = oracle.rmsnorm(x, w, 1e-6)
    xt = torch.from_numpy(bf16_to_f32(x).astype(np.float64))
    want = torch.nn.functional.rms_norm(xt, (2048,), weight=torch.from_numpy(bf16_to_f32(w).astype(np.float64)), eps=1e-6)
    got = bf16_to_f32(y).astype(np.float64)
    assert np.all(np.abs(got - want.numpy()) <= np.abs(want.numpy()) * 2.0**-7 + 1e-30)  # two bf16 roundings
    # a power-of-two scale of x leaves the norm's output unchanged (closed form)
    y4, _ = oracle.rmsnorm(f32_to_bf16(bf16_to_f32(x) * 4.0), w, 0.0)
    y1, _ = oracle.rmsnorm(x, w, 0.0)
    assert np.array_equal(y4, y1)
    # the residual form normalises bf16(x + r) and returns that sum
    r = normal_bf16((6, 2048), seed=72)
    yr, h = oracle.rmsnorm(x, w, 1e-6, resid=r)
    assert np.array_equal(h, f32_to_bf16(bf16_to_f32(x) + bf16_to_f32(r)))
    assert np.array_equal(yr, oracle.rmsnorm(h, w, 1e-6)[0])


def _rope_case(pos, seed=80, H=2, Hkv=1):
    qkv = normal_bf16((len(pos), (H + 2 * Hkv) * 128), seed=seed)
    ones = f32_to_bf16(np.ones(128, np.float32))
    inv = (1e6 ** (-np.arange(0, 128, 2) / 128)).astype(np.float32)
    pages = max(p // 16 for p in pos) + 1
    table = np.tile(np.arange(pages, dtype=np.int32), (len(pos), 1))
    pool = np.zeros((pages, Hkv, 2, 2048), np.uint16)
    q = oracle.qk_norm_rope_append(qkv, H, Hkv, ones, ones, 1e-6, inv, np.array(pos, np.int32), pool, table)
    return qkv, q, pool, inv


def test_rope_position_zero_is_the_norm_alone_and_rotation_keeps_pair_norms():
    qkv, q, pool, inv = _rope_case([0, 5, 70000])
    ones = f32_to_bf16(np.ones(128, np.float32))
    normed, _ = oracle.rmsnorm(qkv[:, :256].reshape(-1, 128), ones, 1e-6)
    assert np.array_equal(q[0].reshape(-1, 128), normed.reshape(3, 2, 128)[0])  # angle 0: identity
    a = bf16_to_f32(normed.reshape(3, 2, 128)).astype(np.float64)
    b = bf16_to_f32(q).astype(np.float64)
    na = np.hypot(a[..., :64], a[..., 64:])
    nb = np.hypot(b[..., :64], b[..., 64:])
    assert np.all(np.abs(na - nb) <= na * 2.0**-6 + 1e-6)


def test_rope_matches_complex_rotation():
    qkv, q, pool, inv = _rope_case([12345], seed=81)
    ones = f32_to_bf16(np.ones(128, np.float32))
    xn = bf16_to_f32(oracle.rmsnorm(qkv[:, :128], ones, 1e-6)[0][0]).astype(np.float64)
    ang = (np.float32(12345) * inv).astype(np.float64)  # the fp32 angle MLX forms
    z = (xn[:64] + 1j * xn[64:]) * np.exp(1j * ang)
    want = f32_to_bf16(np.concatenate([z.real, z.imag]).astype(np.float32))
    assert np.array_equal(q[0, 0], want)


def test_qk_append_writes_k_and_v_at_the_position():
    qkv, q, pool, inv = _rope_case([3, 40], seed=82)
    kc, vc = oracle.kv_gather(pool, np.array([0, 1, 2], np.int32), 41, 1, 128)
    assert np.array_equal(vc[0, 40], qkv[1, 3 * 128:])  # v copied verbatim
    assert np.array_equal(vc[0, 3], qkv[0, 3 * 128:])
    assert not np.array_equal(kc[0, 40], qkv[1, 2 * 128:3 * 128])  # k normed + rotated


def test_segment_gemm_weights_in_gate_up_and_down():
    """bf16w gate||up and down equal float64 products over independently rounded weights, rounded
    to bf16 (and SwiGLU for gate||up) -- and differ from the exact-weight results only slightly."""
    x, inds, scores, gu, dn = _moe_case(seed=20)
    pk = oracle.moe_pack(inds, 16)
    h = oracle.moe_gate_up(x, inds, pk, *gu, bf16w=True)
    h_exact = oracle.moe_gate_up(x, inds, pk, *gu)
    r = oracle.moe_down(h, inds, pk, *dn, bf16w=True)
    I = h.shape[1]
    flat = inds.reshape(-1)
    xf = bf16_to_f32(x).astype(np.float64)
    for p in range(0, pk["order"].size, 13):
        e, row = int(flat[pk["order"][p]]), int(pk["pair_row"][p])
        wgu, _ = _bf16_weights_numpy(gu[0][e], gu[1][e], gu[2][e])
        acc = wgu @ xf[row]
        g, u = f32_to_bf16(acc[:I].astype(np.float32)), f32_to_bf16(acc[I:].astype(np.float32))
        assert np.array_equal(h[p], np.array([oracle.swiglu_bf16(a, c) for a, c in zip(g, u)], np.uint16)), p
        wd, _ = _bf16_weights_numpy(dn[0][e], dn[1][e], dn[2][e])
        assert np.array_equal(r[p], f32_to_bf16((wd @ bf16_to_f32(h[p]).astype(np.float64)).astype(np.float32))), p
    assert not np.array_equal(h, h_exact)
    d = np.abs(bf16_to_f32(h).astype(np.float64) - bf16_to_f32(h_exact))
    assert d.max() <= 2e-2


def test_embed_q4_pinned_by_torch_bf16_ops():
    """mx.dequantize in bf16 arithmetic: bf16(bf16(s * q) + b), against torch's own bf16 multiply
    and add (a library routine); q = 0 gives the bias exactly; an out-of-range id a zero row."""
    rng = np.random.default_rng(8)
    V, D = 40, 256
    w = rng.integers(0, 2**32, (V, D // 8), dtype=np.uint64).astype(np.uint32)
    w[5] = 0
    s = oracle.f32_to_bf16(rng.normal(0, 0.01, (V, D // 64)).astype(np.float32))
    b = oracle.f32_to_bf16(rng.normal(0, 0.05, (V, D // 64)).astype(np.float32))
    ids = np.array([3, 0, 39, 5, 40, -2])
    got = oracle.embed_q4(ids, w, s, b)
    q = ((torch.from_numpy(w.astype(np.int64))[:, :, None] >> (4 * torch.arange(8))) & 15).reshape(V, D)
    st = torch.from_numpy(s.view(np.int16)).view(torch.bfloat16).repeat_interleave(64, 1)
    bt = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).repeat_interleave(64, 1)
    ref = (st * q.to(torch.bfloat16) + bt).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got[:4], ref[[3, 0, 39, 5]])
    assert np.array_equal(got[3], np.repeat(b[5], 64))
    assert not got[4].any() and not got[5].any()


def test_argmax_rows_pinned_by_numpy():
    x = oracle.f32_to_bf16(np.random.default_rng(2).normal(0, 3, (7, 1001)).astype(np.float32))
    x[1, [4, 9]] = x[1].view(np.int16).max()  # positive bf16 patterns order like their values
    got = oracle.argmax_rows(x)
    assert np.array_equal(got, np.argmax(oracle.bf16_to_f32(x), axis=1))
    y = x.copy()
    y[0, :3] = 0x7FC0                     # NaN never wins
    y[2, :] = 0x7FC0                      # all NaN: 0
    assert oracle.argmax_rows(y)[0] == np.argmax(oracle.bf16_to_f32(x[0, 3:])) + 3
    assert oracle.argmax_rows(y)[2] == 0


def test_mlx_f32_layer_close_to_float64_layer():
    """decoder_layer_mlx_f32 (the reference's fp32 arithmetic, the CPU baseline's chain) agrees with
    the float64 decoder_layer within the composition tolerance, and its 768-wide down projection (a
    partial 512-block of qmv lanes) is fp32-accurate."""
    from jitengine_amd.model import MoEConfig, random_layer_weights, rope_inv_freq

    cfg = MoEConfig(layers=1, experts=16)
    w = random_layer_weights(cfg, 9, "cpu")
    qn = ("qkv", "o", "router", "gate_up", "down")
    lw = {k: (stack_np(v) if k in qn else v.view(torch.int16).numpy().view(np.uint16)) for k, v in w.items()}
    lens = [5, 300, 2000]
    npg = [-(-(L + 1) // 16) for L in lens]
    perm = np.random.default_rng(3).permutation(sum(npg))
    table = np.zeros((3, max(npg)), np.int32)
    at = 0
    for i, n in enumerate(npg):
        table[i, :n] = perm[at:at + n]
        at += n
    pool = normal_bf16((sum(npg), 4, 2, 2048), seed=4)
    x = normal_bf16((3, 2048), seed=5)
    ocfg = {"heads": 32, "kv_heads": 4, "experts": 16, "top_k": 8, "eps": 1e-6, "inv_freq": rope_inv_freq(1e6, 128)}
    pos = np.array(lens, np.int32)
    y = oracle.decoder_layer_mlx_f32(x, lw, pool.copy(), table, pos, ocfg)
    ref = oracle.decoder_layer(x, lw, pool.copy(), table, pos, ocfg)["y"]
    a, b = bf16_to_f32(y).astype(np.float64), bf16_to_f32(ref).astype(np.float64)
    assert a.ravel() @ b.ravel() / (np.linalg.norm(a) * np.linalg.norm(b)) > 0.9999
    assert np.abs(a - b).max() <= 4 * np.maximum(np.abs(b), 1) .max() * 2.0**-8
    dw, ds, db = lw["down"]
    hx = normal_bf16((4, 768), seed=6)
    f, _ = oracle.qmm(hx, dw[0], ds[0], db[0])
    m = oracle.qmv_mlx_f32(hx, dw[0], ds[0], db[0]).astype(np.float64)
    assert np.abs(m - f).max() <= 2.0**-16 * np.abs(f).max()
