"""The one-row projections that build their own normed input row (jit_qmm_packed_add_rmsnorm,
jit_qmm_packed_combine_rmsnorm) against the launches they replace: jit_rmsnorm with a residual
then jit_qmm_packed, and jit_moe_combine_rmsnorm then jit_qmm_packed -- the same bits for every
output, on the GPU; and the one-token decode step that chains them against the layer-by-layer
step."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from jitengine_amd import ops
from jitengine_amd.model import MoEConfig, Model, random_layer_weights
from jitengine_amd.quant import random_quantized
from tests.helpers import bf16_tensor, normal_bf16, u16

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _i32(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(DEV)


def _norm_w(D, seed):
    rng = np.random.default_rng(seed)
    return bf16_tensor(oracle.f32_to_bf16((1 + 0.05 * rng.standard_normal(D)).astype(np.float32)), DEV)


# D 256 runs on two waves (fewer than the row's 256 owner threads), 512 on four, 1536 on six, 2048
# on eight; N 5120 and 4112 take the 32-row workgroups, 4112 with a half-empty last one
SHAPES = [(2048, 128), (2048, 5120), (1536, 4096), (1024, 4112), (512, 48), (256, 16)]


@pytest.mark.parametrize("D,N", SHAPES)
def test_add_rmsnorm_projection_equals_rmsnorm_then_qmm(D, N):
    lin = ops.prepack(random_quantized((N, D), 7 + D + N, device=DEV))
    a = bf16_tensor(normal_bf16((1, D), seed=D, scale=3.0), DEV)
    resid = bf16_tensor(normal_bf16((1, D), seed=D + 1), DEV)
    w = _norm_w(D, D + 2)
    hn0, h0 = ops.rmsnorm(a, w, 1e-6, resid=resid, return_sum=True)
    y0 = ops.qmm(hn0, lin, seg=False)
    y1, h1, hn1 = ops.qmm_add_rmsnorm(a, resid, w, 1e-6, lin)
    torch.cuda.synchronize()
    assert np.array_equal(u16(h0), u16(h1))
    assert np.array_equal(u16(hn0), u16(hn1))
    assert np.array_equal(u16(y0), u16(y1))


@pytest.mark.parametrize("D,N,k,resid", [(2048, 5120, 8, True), (2048, 128, 8, False), (1536, 4096, 3, True),
                                         (256, 16, 1, True), (512, 48, 17, True)])
def test_combine_rmsnorm_projection_equals_combine_rmsnorm_then_qmm(D, N, k, resid):
    E = 64
    lin = ops.prepack(random_quantized((N, D), 11 + D + k, device=DEV))
    rng = np.random.default_rng(D + k)
    pk = ops.moe_pack(_i32(rng.permutation(E)[:k][None, :]), E)
    r = bf16_tensor(normal_bf16((k, D), seed=k + 3, scale=0.5), DEV)
    scores = bf16_tensor(normal_bf16((1, k), seed=k + 4, scale=0.3), DEV)
    h = bf16_tensor(normal_bf16((1, D), seed=k + 5), DEV) if resid else None
    w = _norm_w(D, k + 6)
    y0, xn0 = ops.moe_combine_rmsnorm(r, pk, scores, h, w, 1e-6)
    out0 = ops.qmm(xn0, lin, seg=False)
    y1, out1 = ops.qmm_combine_rmsnorm(r, pk, scores, h, w, 1e-6, lin)
    torch.cuda.synchronize()
    assert np.array_equal(u16(y0), u16(y1))
    assert np.array_equal(u16(out0), u16(out1))


def test_row_prologue_projections_reject_what_they_do_not_cover():
    D = 2048
    a = torch.zeros((2, D), dtype=torch.bfloat16, device=DEV)
    w = torch.ones(D, dtype=torch.bfloat16, device=DEV)
    lin = ops.prepack(random_quantized((32, D), 1, device=DEV))
    with pytest.raises(ValueError):  # two rows
        ops.qmm_add_rmsnorm(a, a, w, 1e-6, lin)
    wide = ops.prepack(random_quantized((32, 4096), 2, device=DEV))
    a1 = torch.zeros((1, 4096), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ops._lib.UnsupportedShape):  # D > 2048
        ops.qmm_add_rmsnorm(a1, a1, torch.ones(4096, dtype=torch.bfloat16, device=DEV), 1e-6, wide)
    assert not ops.row_prologue_fits(wide, 4096)
    assert ops.row_prologue_fits(lin, D)
    with pytest.raises(ops._lib.UnsupportedShape):  # an MLX-layout matrix
        ops.qmm_add_rmsnorm(a[:1], a[:1], w, 1e-6, random_quantized((32, D), 1, device=DEV))


def _pages(lens, cfg, seed):
    rng = np.random.default_rng(seed)
    npg = [-(-(L + 1) // 16) for L in lens]
    perm = rng.permutation(sum(npg) + 1)
    table = np.zeros((len(lens), max(npg)), np.int32)
    c = 0
    for b, n in enumerate(npg):
        table[b, :n] = perm[c:c + n]
        c += n
    pools = [normal_bf16((len(perm), cfg.kv_heads, 2, 2048), seed=seed + 1 + l, scale=0.5) for l in range(cfg.layers)]
    return table, pools


@pytest.mark.parametrize("experts,lens", [(128, [3000]), (32, [17])])
def test_one_token_decode_step_equals_layer_chain(experts, lens):
    """At B = 1 Model.decode_step carries each layer's combine into the next layer's qkv launch,
    norms the post-attention sum inside the router launch and routes inside the gate||up launch;
    its output and appended KV equal the chain of stand-alone layer steps (each closing with its own
    combine) bit for bit."""
    cfg = MoEConfig(experts=experts, layers=3)
    model = Model(cfg, [random_layer_weights(cfg, seed=60 + l, device=DEV) for l in range(cfg.layers)])
    table, pools = _pages(lens, cfg, seed=61)
    x = bf16_tensor(normal_bf16((1, cfg.hidden), seed=62), DEV)
    st = model.make_state(np.array(lens), _i32(table))
    pa = [bf16_tensor(p, DEV) for p in pools]
    pb = [bf16_tensor(p, DEV) for p in pools]
    fused = model.decode_step(x, pa, st)
    y = x
    for layer, pool in zip(model.layers, pb):
        y = layer.step(y, pool, st)
    torch.cuda.synchronize()
    assert np.array_equal(u16(fused), u16(y))
    for p, q in zip(pa, pb):
        assert torch.equal(p, q)
