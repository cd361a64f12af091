"""Decoder-block kernels and a whole decoder layer on the GPU vs the CPU oracle (MI355X only)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from jitengine_amd import ops
from jitengine_amd.model import DecoderLayer, MoEConfig, Model, make_step_state, random_layer_weights, rope_inv_freq
from tests.helpers import (
    assert_attention_parity, assert_close_bf16, assert_fn_criterion, bf16_tensor, bf16_to_f32, f32_to_bf16,
    normal_bf16, u16,
)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _i32(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(DEV)


@pytest.mark.parametrize("resid", [False, True])
@pytest.mark.parametrize("rows", [1, 32, 300])
def test_rmsnorm_parity(resid, rows):
    x = normal_bf16((rows, 2048), seed=rows, scale=2.0)
    r = normal_bf16((rows, 2048), seed=rows + 1)
    w = oracle.f32_to_bf16((1 + 0.02 * np.random.default_rng(3).standard_normal(2048)).astype(np.float32))
    y, h = ops.rmsnorm(bf16_tensor(x, DEV), bf16_tensor(w, DEV), 1e-6,
                       resid=bf16_tensor(r, DEV) if resid else None, return_sum=True)
    wy, wh = oracle.rmsnorm(x, w, 1e-6, resid=r if resid else None)
    assert np.array_equal(u16(h), wh)
    st = assert_close_bf16(u16(y), wy, what="rmsnorm")
    assert st["bit_equal"] > 0.97, st


@pytest.mark.parametrize("pos", [[0, 1, 15, 16, 17], [4096, 32767, 100000, 262143]])
def test_qk_norm_rope_append_parity(pos):
    H, Hkv, B = 32, 4, len(pos)
    qkv = normal_bf16((B, (H + 2 * Hkv) * 128), seed=sum(pos) % 1000, scale=1.5)
    rng = np.random.default_rng(7)
    qn = oracle.f32_to_bf16((1 + 0.02 * rng.standard_normal(128)).astype(np.float32))
    kn = oracle.f32_to_bf16((1 + 0.02 * rng.standard_normal(128)).astype(np.float32))
    inv = rope_inv_freq(1e6, 128)
    npg = max(p // 16 for p in pos) + 1
    num_pages = B + 3
    table = rng.integers(0, num_pages, (B, npg)).astype(np.int32)  # only the written page matters
    for b, p in enumerate(pos):
        table[b, p // 16] = b  # distinct pages for the written slots
    pool = normal_bf16((num_pages, Hkv, 2, 2048), seed=9)
    pt = bf16_tensor(pool, DEV)
    q = ops.qk_norm_rope_append(bf16_tensor(qkv, DEV), H, Hkv, bf16_tensor(qn, DEV), bf16_tensor(kn, DEV), 1e-6,
                                torch.from_numpy(inv).to(DEV), _i32(pos), _i32(table), pt)
    want_pool = pool.copy()
    wq = oracle.qk_norm_rope_append(qkv, H, Hkv, qn, kn, 1e-6, inv, np.array(pos, np.int32), want_pool, table)
    st = assert_close_bf16(u16(q), wq, what="q")
    assert st["bit_equal"] > 0.95, st
    got_pool = u16(pt)
    assert np.array_equal(got_pool[:, :, 1], want_pool[:, :, 1])  # V parts: copied verbatim, nothing else touched
    kg = got_pool[:, :, 0].reshape(num_pages, Hkv, 4, 16, 32).copy()  # K chunk-major [d/32][slot][d%32]
    kw = want_pool[:, :, 0].reshape(num_pages, Hkv, 4, 16, 32).copy()
    for b, p in enumerate(pos):
        assert_close_bf16(kg[b, :, :, p % 16], kw[b, :, :, p % 16], what="k")
        kg[b, :, :, p % 16] = kw[b, :, :, p % 16]
    assert np.array_equal(kg, kw)  # K parts: only the written slots changed


def _layer_numpy(w: dict) -> dict:
    def q(lin):
        return (lin.weight.cpu().numpy().view(np.uint32), u16(lin.scales), u16(lin.biases))

    return {"input_norm": u16(w["input_norm"]), "qkv": q(w["qkv"]), "q_norm": u16(w["q_norm"]),
            "k_norm": u16(w["k_norm"]), "o": q(w["o"]), "post_norm": u16(w["post_norm"]),
            "router": q(w["router"]), "gate_up": q(w["gate_up"]), "down": q(w["down"])}


def _small_cfg():
    return MoEConfig(experts=32, layers=2)


def _ctx(lens, cfg, seed):
    rng = np.random.default_rng(seed)
    npg = [-(-(L + 1) // 16) for L in lens]
    num_pages = sum(npg) + 3
    perm = rng.permutation(num_pages)
    table = np.zeros((len(lens), max(npg)), np.int32)
    at = 0
    for i, n in enumerate(npg):
        table[i, :n] = perm[at:at + n]
        at += n
    pools = [normal_bf16((num_pages, cfg.kv_heads, 2, 2048), seed=seed + 10 + l) for l in range(cfg.layers)]
    return table, pools


def _stages_on_gpu_inputs(cfg, lens, table, pool_after, w, dbg, what):
    """Each stage of the attention and MoE halves against the oracle on the GPU's own inputs to that
    stage (so a stage's error is not hidden under the drift of the stages before it):
    * attention: the attention bar (tests.helpers.assert_attention_parity: the reference's 8x-stock
      criterion, one ulp + 2^-14 of the row, >= 98% correctly rounded) on the GPU's q over the pool
      the GPU's append left, through the layer's plan, page table and pos + 1 lengths;
    * router logits: the reference's criterion for quantized projections and >= 95% bit-equal;
    * gate||up + SwiGLU (h) and down (r): the north-star tolerance (h at 4 ulps, as its SwiGLU
      may flip with one ulp of g or u) and >= 95% bit-equal, under the GPU's routing;
    * the closing combine: y = bf16(h + combine(r, scores)) bit for bit."""
    lens1 = np.asarray(lens, np.int64) + 1
    q = u16(dbg["q"])
    _, exact = oracle.paged_decode_attn(q, pool_after, table, lens1, 128 ** -0.5, exact=True)
    stock, _ = oracle.sdpa_mlx_f32(q, pool_after, table, lens1, 128 ** -0.5)
    assert_attention_parity(u16(dbg["attn"]), exact, stock, what=f"{what}: attention stage")
    hn = u16(dbg["hn"])
    wr, sr, br = _layer_numpy(w)["router"]
    f64, want_l = oracle.qmm(hn, wr, sr, br)
    got_l = u16(dbg["logits"])
    assert_fn_criterion(got_l, hn, wr, sr, br, f64)
    st = assert_close_bf16(got_l, want_l, what=f"{what}: router logits")
    assert st["bit_equal"] >= 0.95, (what, "logits", st)
    gi = dbg["inds"].cpu().numpy().view(np.uint32)
    opk = oracle.moe_pack(gi, cfg.experts)
    lw = _layer_numpy(w)
    want_h = oracle.moe_gate_up(hn, gi, opk, *lw["gate_up"])
    st = assert_close_bf16(u16(dbg["hh"]), want_h, what=f"{what}: gate_up", ulps=4.0)
    assert st["bit_equal"] >= 0.95, (what, "gate_up", st)
    want_r = oracle.moe_down(u16(dbg["hh"]), gi, opk, *lw["down"])
    st = assert_close_bf16(u16(dbg["r"]), want_r, what=f"{what}: down")
    assert st["bit_equal"] >= 0.95, (what, "down", st)
    moe = oracle.moe_combine(u16(dbg["r"]), opk["inv"], u16(dbg["scores"]))
    want_y = f32_to_bf16(bf16_to_f32(u16(dbg["h"])) + bf16_to_f32(moe))
    assert np.array_equal(u16(dbg["y"]), want_y), f"{what}: y != bf16(h + combine(r))"


def _layer_vs_oracle(cfg, lens, table, pool, x, w, what, max_flips):
    """One layer step on the GPU against oracle.decoder_layer on the same inputs, stage by stage
    (the MoE half under the GPU's routing, which is bit-exact given the logits); rows whose float64
    routing differs are counted.  The layer output composes ~6 bf16 rounding stages (attention,
    o_proj, residual, experts, combine, residual): up to 4 ulps where that exceeds the absolute 2e-2.
    Then each stage against the oracle on the GPU's own inputs (_stages_on_gpu_inputs)."""
    layer = DecoderLayer(cfg, w)
    pool_t = bf16_tensor(pool, DEV)
    st = make_step_state(cfg, np.array(lens), _i32(table))
    dbg = {}
    y = layer.step(bf16_tensor(x, DEV), pool_t, st, debug=dbg)
    ref_pool = pool.copy()
    ocfg = {"heads": cfg.heads, "kv_heads": cfg.kv_heads, "experts": cfg.experts, "top_k": cfg.top_k,
            "eps": cfg.eps, "inv_freq": rope_inv_freq(cfg.rope_theta, 128)}
    gi = dbg["inds"].cpu().numpy().view(np.uint32)
    gs = u16(dbg["scores"])
    ref = oracle.decoder_layer(x, _layer_numpy(w), ref_pool, table, np.array(lens, np.int32), ocfg, routing=(gi, gs))
    for name in ("xn", "qkv", "q", "attn", "o", "h", "hn"):
        assert_close_bf16(u16(dbg[name]).reshape(ref[name].shape), ref[name], what=f"{what}: {name}")
    own = oracle.router_topk(ref["logits"], cfg.top_k, True)[0]
    flips = int(np.sum(np.any(np.sort(own, -1) != np.sort(gi, -1), -1)))
    assert flips <= max_flips, f"{what}: {flips} rows routed differently from the float64 logits"
    assert_close_bf16(u16(y), ref["y"], what=f"{what}: layer output", ulps=4.0)
    _stages_on_gpu_inputs(cfg, lens, table, u16(pool_t), w, dbg, what)
    return dbg, ref


def test_decoder_layer_config0():
    """BASELINE configs[0] on the GPU: one Qwen3-MoE-style block (128 experts, top-8) at batch 1,
    decoding at position 4,096 over a 4,096-token context in pages 0..255 in order (the new key
    goes to page 256), against the oracle's block."""
    cfg = MoEConfig(layers=1)
    L = 4096
    table = np.arange(L // 16 + 1, dtype=np.int32)[None]
    pool = normal_bf16((L // 16 + 1, cfg.kv_heads, 2, 2048), seed=0x4A450000 + 1)
    x = normal_bf16((1, cfg.hidden), seed=0x4A450000 + 2)
    w = random_layer_weights(cfg, seed=0x4A450000 % 100000, device=DEV)
    dbg, ref = _layer_vs_oracle(cfg, [L], table, pool, x, w, "config 0", max_flips=1)
    assert int(torch.unique(dbg["inds"]).numel()) == 8


def test_decoder_layer_config2_rows():
    """BASELINE configs[2]'s step on one layer at full geometry: the bench's 32 ragged rows (lengths
    log-uniform in [128, 32768], pages a random permutation) through a 128-expert block -- the
    decode expert GEMVs in their real regime (~2 rows per distinct expert) -- against the oracle."""
    cfg = MoEConfig(layers=1)
    rng = np.random.default_rng(0x4A450000 + 16 * 2)
    lens = np.round(np.exp(rng.uniform(np.log(128), np.log(32768), 32))).astype(np.int32)
    npg = (lens + 1 + 15) // 16
    perm = rng.permutation(int(npg.sum()))
    table = np.zeros((32, int(npg.max())), np.int32)
    at = 0
    for b in range(32):
        table[b, :npg[b]] = perm[at:at + npg[b]]
        at += npg[b]
    pool = normal_bf16((int(npg.sum()), cfg.kv_heads, 2, 2048), seed=0x4A450000 + 33)
    x = normal_bf16((32, cfg.hidden), seed=0x4A450000 + 34)
    w = random_layer_weights(cfg, seed=0x4A450000 % 100000 + 2, device=DEV)
    dbg, ref = _layer_vs_oracle(cfg, list(lens), table, pool, x, w, "config 2 rows", max_flips=3)
    assert int(torch.unique(dbg["inds"]).numel()) > 90  # the regime: most experts hit by 1-3 rows


def test_decoder_layer_parity():
    """One layer, 12 ragged rows: every stage checked against the oracle's layer; the MoE half
    is compared under the GPU's routing (routing is bit-exact given the router logits, and the
    logits themselves are within tolerance), and rows whose float64 routing differs are counted."""
    cfg = _small_cfg()
    lens = [1, 15, 16, 100, 255, 256, 257, 1000, 3000, 4096, 5000, 20000]
    w = random_layer_weights(cfg, seed=5, device=DEV)
    layer = DecoderLayer(cfg, w)
    table, pools = _ctx(lens, cfg, seed=6)
    x = normal_bf16((len(lens), 2048), seed=7)
    pool_t = bf16_tensor(pools[0], DEV)
    st = make_step_state(cfg, np.array(lens), _i32(table))
    dbg = {}
    y = layer.step(bf16_tensor(x, DEV), pool_t, st, debug=dbg)
    ref_pool = pools[0].copy()
    ocfg = {"heads": cfg.heads, "kv_heads": cfg.kv_heads, "experts": cfg.experts, "top_k": cfg.top_k,
            "eps": cfg.eps, "inv_freq": rope_inv_freq(cfg.rope_theta, 128)}
    gi = dbg["inds"].cpu().numpy().view(np.uint32)
    gs = u16(dbg["scores"])
    ref = oracle.decoder_layer(x, _layer_numpy(w), ref_pool, table, np.array(lens, np.int32), ocfg, routing=(gi, gs))
    for name in ("xn", "qkv", "q", "attn", "o", "h", "hn"):
        assert_close_bf16(u16(dbg[name]).reshape(ref[name].shape), ref[name], what=name)
    own = oracle.router_topk(ref["logits"], cfg.top_k, True)[0]
    flips = int(np.sum(np.any(np.sort(own, -1) != np.sort(gi, -1), -1)))
    assert flips <= 2, f"{flips} rows routed differently from the float64 logits"
    # the layer output composes ~6 bf16 rounding stages (attention, o_proj, residual, experts,
    # combine, residual): up to 4 ulps where that exceeds the absolute 2e-2 (|y| in [2, 4) has
    # an ulp of 1.6e-2)
    assert_close_bf16(u16(y), ref["y"], what="layer output", ulps=4.0)
    _stages_on_gpu_inputs(cfg, lens, table, u16(pool_t), w, dbg, "12 ragged rows")


@pytest.mark.parametrize("B,resid", [(1, True), (32, True), (33, False)])
def test_combine_rmsnorm_equals_combine_then_rmsnorm(B, resid):
    """The fused layer-closing launch gives bit for bit moe_combine and then the next layer's
    input RMSNorm of its output."""
    k, D, P = 8, 2048, B * 8
    rng = np.random.default_rng(B)
    r = bf16_tensor(normal_bf16((P, D), seed=B + 1, scale=0.5), DEV)
    inds = np.stack([rng.permutation(128)[:k] for _ in range(B)]).astype(np.int32)
    pk = ops.moe_pack(_i32(inds), 128)
    scores = bf16_tensor(normal_bf16((B, k), seed=B + 2, scale=0.2), DEV)
    h = bf16_tensor(normal_bf16((B, D), seed=B + 3), DEV) if resid else None
    w = bf16_tensor(oracle.f32_to_bf16((1 + 0.02 * rng.standard_normal(D)).astype(np.float32)), DEV)
    y, xn = ops.moe_combine_rmsnorm(r, pk, scores, h, w, 1e-6)
    y2 = ops.moe_combine(r, pk, scores, h)
    assert torch.equal(y, y2)
    assert torch.equal(xn, ops.rmsnorm(y2, w, 1e-6))


def test_model_decode_step_equals_layer_chain():
    """Model.decode_step (each layer's combine also norms the next layer's input) gives bit for
    bit the chain of stand-alone layer steps."""
    cfg = MoEConfig(experts=32, layers=3)
    lens = [70, 1500, 9]
    model = Model(cfg, [random_layer_weights(cfg, seed=40 + l, device=DEV) for l in range(cfg.layers)])
    table, pools = _ctx(lens, cfg, seed=41)
    x = bf16_tensor(normal_bf16((len(lens), 2048), seed=42), DEV)
    st = model.make_state(np.array(lens), _i32(table))
    pa = [bf16_tensor(p, DEV) for p in pools]
    pb = [bf16_tensor(p, DEV) for p in pools]
    fused = model.decode_step(x, pa, st)
    y = x
    for layer, pool in zip(model.layers, pb):
        y = layer.step(y, pool, st)
    assert torch.equal(fused, y)
    for p, q in zip(pa, pb):
        assert torch.equal(p, q)  # the same KV appended


def test_model_decode_step_rows_are_independent():
    """A row's output does not depend on the other rows of the batch (the reference's
    batched-row = solo-row property, Q36T/metal/engine/test_engine_consistency.py:43)."""
    cfg = _small_cfg()
    lens = [50, 3000, 17, 9000]
    model = Model(cfg, [random_layer_weights(cfg, seed=20 + l, device=DEV) for l in range(cfg.layers)])
    table, pools = _ctx(lens, cfg, seed=30)
    x = normal_bf16((len(lens), 2048), seed=31)
    st = model.make_state(np.array(lens), _i32(table))
    batched = u16(model.decode_step(bf16_tensor(x, DEV), [bf16_tensor(p, DEV) for p in pools], st))
    for b in range(len(lens)):
        stb = model.make_state(np.array(lens[b:b + 1]), _i32(table[b:b + 1]))
        solo = u16(model.decode_step(bf16_tensor(x[b:b + 1], DEV), [bf16_tensor(p, DEV) for p in pools], stb))
        assert np.array_equal(solo[0], batched[b]), b


def test_layer_packed_equals_mlx_layout_layer():
    """A decoder layer on packed weights and the same layer on MLX-layout weights give the same
    intermediates and output and append the same KV bits."""
    cfg = MoEConfig(experts=64, layers=1)
    lens = [5, 700, 64, 4000, 1]
    rng = np.random.default_rng(5)
    npg = [-(-(L + 1) // 16) for L in lens]
    num_pages = sum(npg) + 2
    perm = rng.permutation(num_pages)
    table = np.zeros((len(lens), max(npg)), np.int32)
    at = 0
    for i, n in enumerate(npg):
        table[i, :n] = perm[at:at + n]
        at += n
    w = random_layer_weights(cfg, seed=77, device=DEV)
    fused, plain = DecoderLayer(cfg, w, prepack=True), DecoderLayer(cfg, w, prepack=False)
    pool = bf16_tensor(normal_bf16((num_pages, cfg.kv_heads, 2, 2048), seed=78), DEV)
    pa, pb = pool.clone(), pool.clone()
    st = make_step_state(cfg, np.array(lens), torch.from_numpy(table).to(DEV))
    x = bf16_tensor(normal_bf16((len(lens), 2048), seed=79), DEV)
    da, db = {}, {}
    ya = fused.step(x, pa, st, debug=da)
    yb = plain.step(x, pb, st, debug=db)
    torch.cuda.synchronize()
    for name in ("hn", "logits", "inds", "scores", "hh", "r"):
        assert torch.equal(da[name], db[name]), name
    assert torch.equal(ya, yb)
    assert torch.equal(pa, pb)
