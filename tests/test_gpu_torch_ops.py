"""torch.ops.jitengine.* on MI355X: every registered operator gives the bits of the
jitengine_amd.ops call it wraps, and torch.compile traces a decoder layer's MoE half -- the
batched launches and the one-token fused ones -- through them in one graph (fullgraph, no graph
break) with the eager result."""

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


def _norm_w(n, seed):
    return (1 + 0.05 * bf16_tensor(normal_bf16((n,), seed=seed), DEV).float()).to(torch.bfloat16)


def _one_token_moe_half(gu, dn, x, logits, h, w, qkv_lin):
    """A one-token layer's MoE half and the next layer's qkv projection: three launches."""
    inds, scores, buf, hh = J.route_gate_up(x, logits, gu.data, gu.E, gu.N, gu.K, K_TOP, True)
    r = J.expert_down(hh, dn.data, dn.E, dn.N, dn.K, buf, K_TOP, False)
    return J.qmm_combine_rmsnorm(r, buf, K_TOP, E, scores, h, w, 1e-6, qkv_lin.data, qkv_lin.N, qkv_lin.K)


def test_fused_moe_and_row_operators_equal_the_library_calls(moe):
    gu, dn, x, logits, resid = moe
    inds, scores, pk = ops.route_pack(logits[:4], K_TOP, True)
    ji, js, jb = J.route_pack(logits[:4], K_TOP, True)
    jpk = torch_ops.packing_from_buffer(jb, K_TOP, E)
    assert torch.equal(ji, inds) and torch.equal(js, scores)
    for name in ("order", "pair_row", "inv", "expert_cnt", "expert_off", "meta"):
        assert torch.equal(getattr(jpk, name), getattr(pk, name)), name
    nseg = int(pk.meta[0])  # the segment tables are defined up to the segment count
    for name in ("seg_expert", "seg_start", "seg_cnt"):
        assert torch.equal(getattr(jpk, name)[:nseg], getattr(pk, name)[:nseg]), name

    x1, l1 = x[:1].contiguous(), logits[:1].contiguous()
    inds, scores, pk, hh = ops.route_gate_up(x1, l1, gu, K_TOP, True)
    ji, js, jb, jh = J.route_gate_up(x1, l1, gu.data, gu.E, gu.N, gu.K, K_TOP, True)
    jpk = torch_ops.packing_from_buffer(jb, K_TOP, E)
    assert torch.equal(ji, inds) and torch.equal(js, scores) and torch.equal(jh, hh)
    assert torch.equal(jpk.inv, pk.inv) and torch.equal(jpk.order, pk.order)

    r = ops.expert_down(hh, dn, pk)
    w = _norm_w(D, 91)
    y, xn = ops.moe_combine_rmsnorm(r, pk, scores, resid[:1], w, 1e-6)
    jy, jxn = J.moe_combine_rmsnorm(r, jb, K_TOP, E, js, resid[:1], w, 1e-6)
    assert torch.equal(jy, y) and torch.equal(jxn, xn)
    lin = ops.prepack(make_stack((128, D), seed=92).to(DEV))
    y, out = ops.qmm_combine_rmsnorm(r, pk, scores, resid[:1], w, 1e-6, lin)
    jy, jout = J.qmm_combine_rmsnorm(r, jb, K_TOP, E, js, resid[:1], w, 1e-6, lin.data, lin.N, lin.K)
    assert torch.equal(jy, y) and torch.equal(jout, out)
    a = resid[1:2].contiguous()
    want = ops.qmm_add_rmsnorm(a, x1, w, 1e-6, lin)
    got = J.qmm_add_rmsnorm(a, x1, w, 1e-6, lin.data, lin.N, lin.K)
    assert all(torch.equal(g, e) for g, e in zip(got, want))
    want = ops.rmsnorm(x, w, 1e-6, resid, return_sum=True)
    got = J.rmsnorm_add(x, resid, w, 1e-6)
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])


def test_one_token_moe_half_compiles_into_one_graph(moe):
    gu, dn, x, logits, resid = moe
    args = (gu, dn, x[:1].contiguous(), logits[:1].contiguous(), resid[:1].contiguous(), _norm_w(D, 93),
            ops.prepack(make_stack((256, D), seed=94).to(DEV)))
    eager = _one_token_moe_half(*args)
    torch._dynamo.reset()
    fn = torch.compile(_one_token_moe_half, fullgraph=True, backend="aot_eager")
    for _ in range(2):
        got = fn(*args)
        assert torch.equal(got[0], eager[0]) and torch.equal(got[1], eager[1])


def _paged(lens, seed, Hkv=4, extra=5):
    rng = np.random.default_rng(seed)
    npg = [-(-L // 16) for L in lens]
    perm = rng.permutation(sum(npg) + extra)
    table = np.zeros((len(lens), max(npg)), np.int32)
    at = 0
    for i, n in enumerate(npg):
        table[i, :n] = perm[at:at + n]
        at += n
    return bf16_tensor(normal_bf16((sum(npg) + extra, Hkv, 2, 2048), seed=seed + 1), DEV), _i32(table)


def test_fused_attention_prefill_and_kv_operators():
    H, Hkv, scale = 32, 4, 128 ** -0.5
    lens = [1, 300, 2000]
    pool, table = _paged(lens, 95)
    plan = ops.attn_plan(lens, DEV)
    qkv = bf16_tensor(normal_bf16((3, (H + 2 * Hkv) * 128), seed=96, scale=1.5), DEV)
    qn, kn = _norm_w(128, 97), _norm_w(128, 98)
    inv = torch.from_numpy(_inv_freq()).to(DEV)
    ws = torch.empty(ops.attn_workspace_bytes(plan.total, H), dtype=torch.uint8, device=DEV)
    pool2 = pool.clone()
    want = ops.paged_decode_attention_qkv(qkv, H, Hkv, qn, kn, 1e-6, inv, pool, table, plan, scale)
    got = J.paged_decode_attention_qkv(qkv, H, Hkv, qn, kn, 1e-6, inv, pool2, table, *torch_ops.plan_args(plan),
                                       scale, ws)
    assert torch.equal(got, want) and torch.equal(pool2, pool)

    chunks = [(0, 0, 37), (1, 100, 64), (2, 1900, 100)]
    pp = ops.prefill_plan(chunks, H, Hkv, DEV)
    q = bf16_tensor(normal_bf16((pp.rows, H, 128), seed=99), DEV)
    pws = torch.empty(max(ops.prefill_workspace_bytes(pp, H), 4), dtype=torch.uint8, device=DEV)
    want = ops.paged_prefill_attention(q, pool, table, pp, scale)
    got = J.paged_prefill_attention(q, pool, table, *torch_ops.prefill_plan_args(pp), scale, pws)
    assert torch.equal(got, want)

    k = bf16_tensor(normal_bf16((3, Hkv, 128), seed=100), DEV)
    v = bf16_tensor(normal_bf16((3, Hkv, 128), seed=101), DEV)
    pos = _i32(np.array([0, 299, 1999], np.int32))
    ops.kv_append_paged(pool, k, v, pos, table)
    J.kv_append_paged(pool2, k, v, pos, table)
    assert torch.equal(pool2, pool)
    src, dst = _i32(np.array([0, 3], np.int32)), _i32(np.array([pool.shape[0] - 1, pool.shape[0] - 2], np.int32))
    ops.kv_copy_pages(pool, src, dst)
    J.kv_copy_pages(pool2, src, dst)
    assert torch.equal(pool2, pool)


def test_attention_half_compiles_into_one_graph():
    """The attention half of a decode layer -- attention with the q/k/v rows (which writes the tokens'
    K and V into the pool) and the o projection -- under torch.compile (fullgraph): the mutated pool
    and the output equal the eager calls', on two calls in a row."""
    H, Hkv, scale = 32, 4, 128 ** -0.5
    lens = [7, 300, 1600]
    pool0, table = _paged(lens, 120)
    plan = ops.attn_plan(lens, DEV)
    qkv = bf16_tensor(normal_bf16((3, (H + 2 * Hkv) * 128), seed=121, scale=1.5), DEV)
    qn, kn = _norm_w(128, 122), _norm_w(128, 123)
    inv = torch.from_numpy(_inv_freq()).to(DEV)
    o_lin = ops.prepack(make_stack((512, H * 128), seed=124).to(DEV))
    ws = torch.empty(ops.attn_workspace_bytes(plan.total, H), dtype=torch.uint8, device=DEV)
    args = torch_ops.plan_args(plan)

    def half(qkv, pool):
        attn = J.paged_decode_attention_qkv(qkv, H, Hkv, qn, kn, 1e-6, inv, pool, table, *args, scale, ws)
        return J.qmm(attn.view(attn.shape[0], -1), o_lin.data, o_lin.N, o_lin.K)

    pool_e = pool0.clone()
    want = half(qkv, pool_e)
    torch._dynamo.reset()
    fn = torch.compile(half, fullgraph=True, backend="aot_eager")
    for _ in range(2):
        pool_c = pool0.clone()
        got = fn(qkv, pool_c)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
        assert torch.equal(pool_c, pool_e)  # the tokens' K and V written through the compiled graph


def test_opcheck_schemas_fakes_and_mutations(moe):
    """torch.library.opcheck on every registered operator with real inputs: the schema (declared
    mutations match what the call writes), the fake kernel against the real outputs, and tracing
    with dynamic shapes."""
    gu, dn, x, logits, resid = moe
    inds, scores = ops.router_topk(logits, K_TOP, True)
    buf = J.moe_pack(inds, E)
    h = J.expert_gate_up(x, gu.data, gu.E, gu.N, gu.K, buf, K_TOP, False)
    w = _norm_w(D, 131)
    cases = [
        (J.router_topk, (logits, K_TOP, True)),
        (J.moe_pack, (inds, E)),
        (J.route_pack, (logits[:4].contiguous(), K_TOP, True)),
        (J.expert_gate_up, (x, gu.data, gu.E, gu.N, gu.K, buf, K_TOP, False)),
        (J.expert_down, (h, dn.data, dn.E, dn.N, dn.K, buf, K_TOP, True)),
        (J.moe_combine_rmsnorm, (J.expert_down(h, dn.data, dn.E, dn.N, dn.K, buf, K_TOP, False), buf, K_TOP, E,
                                 scores, resid, w, 1e-6)),
        (J.rmsnorm_add, (x, resid, w, 1e-6)),
    ]
    H, Hkv = 32, 4
    lens = [5, 300]
    pool, table = _paged(lens, 132)
    plan = ops.attn_plan(lens, DEV)
    qkv = bf16_tensor(normal_bf16((2, (H + 2 * Hkv) * 128), seed=133), DEV)
    ws = torch.empty(ops.attn_workspace_bytes(plan.total, H), dtype=torch.uint8, device=DEV)
    cases.append((J.paged_decode_attention_qkv, (qkv, H, Hkv, _norm_w(128, 134), _norm_w(128, 135), 1e-6,
                                                 torch.from_numpy(_inv_freq()).to(DEV), pool, table,
                                                 *torch_ops.plan_args(plan), 128 ** -0.5, ws)))
    kv = bf16_tensor(normal_bf16((2, Hkv, 128), seed=136), DEV)
    cases.append((J.kv_append_paged, (pool, kv, kv, _i32(np.array([4, 299], np.int32)), table)))
    q = bf16_tensor(normal_bf16((2, H, 128), seed=137), DEV)
    cases.append((J.paged_decode_attention, (q, pool, table, *torch_ops.plan_args(plan), 128 ** -0.5, ws)))
    inv = torch.from_numpy(_inv_freq()).to(DEV)
    cases.append((J.qk_norm_rope_append, (qkv, H, Hkv, _norm_w(128, 138), _norm_w(128, 139), 1e-6, inv,
                                          _i32(np.array([4, 299], np.int32)), table, pool)))
    pp = ops.prefill_plan([(0, 0, 5), (1, 200, 40)], H, Hkv, DEV)
    qp = bf16_tensor(normal_bf16((pp.rows, H, 128), seed=140), DEV)
    pws = torch.empty(max(ops.prefill_workspace_bytes(pp, H), 4), dtype=torch.uint8, device=DEV)
    cases.append((J.paged_prefill_attention, (qp, pool, table, *torch_ops.prefill_plan_args(pp), 128 ** -0.5, pws)))
    cases.append((J.kv_copy_pages, (pool, _i32(np.array([0], np.int32)), _i32(np.array([pool.shape[0] - 1],
                                                                                        np.int32)))))
    lin = ops.prepack(make_stack((128, D), seed=141).to(DEV))
    x1 = x[:1].contiguous()
    cases.append((J.qmm, (x, lin.data, lin.N, lin.K)))
    cases.append((J.rmsnorm, (x, w, 1e-6)))
    cases.append((J.qmm_add_rmsnorm, (x1, resid[:1].contiguous(), w, 1e-6, lin.data, lin.N, lin.K)))
    i1, s1, b1, h1 = J.route_gate_up(x1, logits[:1].contiguous(), gu.data, gu.E, gu.N, gu.K, K_TOP, True)
    cases.append((J.route_gate_up, (x1, logits[:1].contiguous(), gu.data, gu.E, gu.N, gu.K, K_TOP, True)))
    r1 = J.expert_down(h1, dn.data, dn.E, dn.N, dn.K, b1, K_TOP, False)
    cases.append((J.qmm_combine_rmsnorm, (r1, b1, K_TOP, E, s1, resid[:1].contiguous(), w, 1e-6, lin.data, lin.N,
                                          lin.K)))
    cases.append((J.moe_combine, (r1, b1, K_TOP, E, s1, None)))
    lg = bf16_tensor(sampler_logits(0, 3, 1001, 142, scale=3.0), DEV)
    u = torch.tensor([0.2, 0.5, 0.9], dtype=torch.float32, device=DEV)
    cases += [(J.logprobs_rows, (lg,)), (J.argmax_rows, (lg,)), (J.sample_rows, (lg, 0.7, 0.9, 20, u)),
              (J.threefry_uniform, (_i32(np.arange(6, dtype=np.int32).reshape(3, 2)),))]
    assert {op._qualified_op_name.split("::")[1] for op, _ in cases} == set(torch_ops.OPS)
    for op, args in cases:
        torch.library.opcheck(op, args)


def _inv_freq():
    from jitengine_amd.model import rope_inv_freq

    return rope_inv_freq(1e6, 128)
