"""torch.ops.jitengine.* on MI355X: every registered operator gives the bits of the
jitengine_amd.ops call it wraps, and torch.compile traces a decoder layer's MoE half through
them in one graph (fullgraph, no graph break) with the eager result."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from jitengine_amd import ops, torch_ops
from tests.helpers import bf16_tensor, make_stack, normal_bf16, router_logits, sampler_logits

pytestmark = pytest.mark.gpu
DEV = "cuda"
J = torch.ops.jitengine
B, E, K_TOP, D, I = 24, 32, 8, 512, 256


def _i32(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(DEV)


@pytest.fixture(scope="module")
def moe():
    gu = ops.prepack(make_stack((E, 2 * I, D), seed=71).to(DEV))
    dn = ops.prepack(make_stack((E, D, I), seed=72).to(DEV))
    x = bf16_tensor(normal_bf16((B, D), seed=73), DEV)
    logits = bf16_tensor(router_logits(0, B, E, seed=74), DEV)
    resid = bf16_tensor(normal_bf16((B, D), seed=75), DEV)
    return gu, dn, x, logits, resid


def _moe_half(gu, dn, x, logits, resid, seg):
    inds, scores = J.router_topk(logits, K_TOP, True)
    buf = J.moe_pack(inds, E)
    h = J.expert_gate_up(x, gu.data, gu.E, gu.N, gu.K, buf, K_TOP, seg)
    r = J.expert_down(h, dn.data, dn.E, dn.N, dn.K, buf, K_TOP, seg)
    return J.moe_combine(r, buf, K_TOP, E, scores, resid)


@pytest.mark.parametrize("seg", [False, True])
def test_moe_operators_equal_the_library_calls(moe, seg):
    gu, dn, x, logits, resid = moe
    inds, scores = ops.router_topk(logits, K_TOP, True)
    pk = ops.moe_pack(inds, E)
    h = ops.expert_gate_up(x, gu, pk, seg=seg)
    r = ops.expert_down(h, dn, pk, seg=seg)
    want = ops.moe_combine(r, pk, scores, resid)
    ji, js = J.router_topk(logits, K_TOP, True)
    assert torch.equal(ji, inds) and torch.equal(js, scores)
    jpk = torch_ops.packing_from_buffer(J.moe_pack(ji, E), K_TOP, E)
    for name in ("order", "pair_row", "inv", "expert_cnt", "expert_off"):
        assert torch.equal(getattr(jpk, name), getattr(pk, name)), name
    assert torch.equal(_moe_half(gu, dn, x, logits, resid, seg), want)


def test_moe_half_compiles_into_one_graph(moe):
    gu, dn, x, logits, resid = moe
    eager = _moe_half(gu, dn, x, logits, resid, False)
    torch._dynamo.reset()
    fn = torch.compile(lambda *a: _moe_half(*a, False), fullgraph=True, backend="aot_eager")
    for _ in range(2):
        assert torch.equal(fn(gu, dn, x, logits, resid), eager)


def test_dense_norm_attention_and_sampler_operators():
    q4 = ops.prepack(make_stack((256, 512), seed=81).to(DEV))
    xt = bf16_tensor(normal_bf16((5, 512), seed=82), DEV)
    assert torch.equal(J.qmm(xt, q4.data, q4.N, q4.K), ops.qmm(xt, q4))
    w = bf16_tensor(normal_bf16((512,), seed=83), DEV)
    assert torch.equal(J.rmsnorm(xt, w, 1e-6), ops.rmsnorm(xt, w, 1e-6))

    lens = [5, 300, 2000]
    rng = np.random.default_rng(84)
    npg = [-(-L // 16) for L in lens]
    perm = rng.permutation(sum(npg) + 3)
    table = np.zeros((3, max(npg)), np.int32)
    at = 0
    for i, n in enumerate(npg):
        table[i, :n] = perm[at:at + n]
        at += n
    pool = bf16_tensor(normal_bf16((sum(npg) + 3, 4, 2, 2048), seed=85), DEV)
    q = bf16_tensor(normal_bf16((3, 32, 128), seed=86), DEV)
    plan = ops.attn_plan(lens, DEV)
    ws = torch.empty(ops.attn_workspace_bytes(plan.total, 32), dtype=torch.uint8, device=DEV)
    want = ops.paged_decode_attention(q, pool, _i32(table), plan, 128 ** -0.5)
    got = J.paged_decode_attention(q, pool, _i32(table), *torch_ops.plan_args(plan), 128 ** -0.5, ws)
    assert torch.equal(got, want)

    pool2 = pool.clone()
    qkv = bf16_tensor(normal_bf16((3, 40 * 128), seed=87), DEV)
    qn, kn = bf16_tensor(normal_bf16((128,), seed=88), DEV), bf16_tensor(normal_bf16((128,), seed=89), DEV)
    inv = torch.from_numpy(_inv_freq()).to(DEV)
    pos = _i32(np.array(lens, np.int32) - 1)
    a = ops.qk_norm_rope_append(qkv, 32, 4, qn, kn, 1e-6, inv, pos, _i32(table), pool)
    b = J.qk_norm_rope_append(qkv, 32, 4, qn, kn, 1e-6, inv, pos, _i32(table), pool2)
    assert torch.equal(a, b) and torch.equal(pool, pool2)

    logits = bf16_tensor(sampler_logits(0, 4, 1001, 90, scale=3.0), DEV)
    u = torch.tensor([0.1, 0.4, 0.7, 0.95], dtype=torch.float32, device=DEV)
    assert torch.equal(J.logprobs_rows(logits), ops.logprobs_rows(logits))
    assert torch.equal(J.argmax_rows(logits), ops.argmax_rows(logits))
    assert torch.equal(J.sample_rows(logits, 0.7, 0.9, 20, u), ops.sample_rows(logits, 0.7, 0.9, 20, u))
    keys = _i32(np.arange(8, dtype=np.uint32).reshape(4, 2) * np.uint32(2654435761))
    assert torch.equal(J.threefry_uniform(keys), ops.threefry_uniform(keys))


def _inv_freq():
    from jitengine_amd.model import rope_inv_freq

    return rope_inv_freq(1e6, 128)
