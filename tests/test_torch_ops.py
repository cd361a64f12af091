"""torch.ops.jitengine.* registration (jitengine_amd/torch_ops.py) on the CPU: every operator is
registered, and its fake kernel propagates shapes and dtypes through meta tensors without the
HIP library (what torch.compile's tracing relies on)."""

from __future__ import annotations

import pytest
import torch

from jitengine_amd import torch_ops

J = None


def setup_module():
    global J
    J = torch.ops.jitengine


def _m(shape, dtype):
    return torch.empty(shape, dtype=dtype, device="meta")


def test_every_operator_is_registered():
    for name in torch_ops.OPS:
        assert hasattr(J, name), name


def test_router_pack_and_experts_propagate_shapes():
    B, E, k, D, I = 32, 128, 8, 2048, 768
    inds, scores = J.router_topk(_m((B, E), torch.bfloat16), k, True)
    assert inds.shape == (B, k) and inds.dtype == torch.int32 and scores.dtype == torch.bfloat16
    buf = J.moe_pack(inds, E)
    P = B * k
    assert buf.shape == (3 * P + 5 * E + 4,) and buf.dtype == torch.int32
    pk = torch_ops.packing_from_buffer(buf, k, E)
    assert pk.P == P and pk.order.shape == (P,) and pk.expert_cnt.shape == (E,) and pk.meta.shape == (4,)
    h = J.expert_gate_up(_m((B, D), torch.bfloat16), _m((1000,), torch.uint8), E, 2 * I, D, buf, k, False)
    assert h.shape == (P, I) and h.dtype == torch.bfloat16
    r = J.expert_down(h, _m((1000,), torch.uint8), E, D, I, buf, k, True)
    assert r.shape == (P, D)
    y = J.moe_combine(r, buf, k, E, scores, _m((B, D), torch.bfloat16))
    assert y.shape == (B, D) and y.dtype == torch.bfloat16


def test_dense_attention_and_sampler_propagate_shapes():
    B, H, Hkv, D, V = 4, 32, 4, 2048, 1000
    assert J.qmm(_m((B, D), torch.bfloat16), _m((10,), torch.uint8), 5120, D).shape == (B, 5120)
    assert J.rmsnorm(_m((B, D), torch.bfloat16), _m((D,), torch.bfloat16), 1e-6).shape == (B, D)
    pool = _m((64, Hkv, 2, 2048), torch.bfloat16)
    q = J.qk_norm_rope_append(_m((B, (H + 2 * Hkv) * 128), torch.bfloat16), H, Hkv, _m((128,), torch.bfloat16),
                              _m((128,), torch.bfloat16), 1e-6, _m((64,), torch.float32), _m((B,), torch.int32),
                              _m((B, 16), torch.int32), pool)
    assert q.shape == (B, H, 128)
    out = J.paged_decode_attention(q, pool, _m((B, 16), torch.int32), _m((B,), torch.int32),
                                   _m((B + 1,), torch.int32), _m((8,), torch.int32), 8, 200, 128 ** -0.5,
                                   _m((1 << 16,), torch.uint8))
    assert out.shape == (B, H, 128) and out.dtype == torch.bfloat16
    x = _m((B, V), torch.bfloat16)
    assert J.logprobs_rows(x).shape == (B, V)
    assert J.argmax_rows(x).dtype == torch.int32
    assert J.sample_rows(x, 0.7, 0.9, 40, _m((B,), torch.float32)).shape == (B,)
    assert J.threefry_uniform(_m((B, 2), torch.int32)).dtype == torch.float32


def test_packing_buffer_split_matches_the_library_layout():
    from jitengine_amd import ops

    buf = torch.arange(3 * 24 + 5 * 16 + 4, dtype=torch.int32)
    pk = torch_ops.packing_from_buffer(buf, 8, 16)
    ref = ops._packing_buffers(24, 8, 16, "cpu")
    for name in ("order", "pair_row", "inv", "expert_cnt", "expert_off", "seg_expert", "seg_start", "seg_cnt", "meta"):
        assert getattr(pk, name).shape == getattr(ref, name).shape, name
    assert int(pk.expert_cnt[0]) == 3 * 24 and int(pk.meta[0]) == 3 * 24 + 5 * 16


def test_fused_launches_propagate_shapes():
    E, k, D, I, N = 128, 8, 2048, 768, 5120
    bf, i32 = torch.bfloat16, torch.int32
    inds, scores, buf = J.route_pack(_m((4, E), bf), k, True)
    assert inds.shape == (4, k) and scores.dtype == bf and buf.shape == (3 * 4 * k + 5 * E + 4,)
    inds, scores, buf, h = J.route_gate_up(_m((1, D), bf), _m((1, E), bf), _m((10,), torch.uint8), E, 2 * I, D, k,
                                           True)
    assert inds.shape == (1, k) and buf.shape == (3 * k + 5 * E + 4,) and h.shape == (k, I) and h.dtype == bf
    r = _m((k, D), bf)
    y, xn = J.moe_combine_rmsnorm(r, buf, k, E, scores, _m((1, D), bf), _m((D,), bf), 1e-6)
    assert y.shape == xn.shape == (1, D)
    y, out = J.qmm_combine_rmsnorm(r, buf, k, E, scores, None, _m((D,), bf), 1e-6, _m((10,), torch.uint8), N, D)
    assert y.shape == (1, D) and out.shape == (1, N) and out.dtype == bf
    y, h, hn = J.qmm_add_rmsnorm(_m((1, D), bf), _m((1, D), bf), _m((D,), bf), 1e-6, _m((10,), torch.uint8), E, D)
    assert y.shape == (1, E) and h.shape == hn.shape == (1, D)
    xn, h = J.rmsnorm_add(_m((3, D), bf), _m((3, D), bf), _m((D,), bf), 1e-6)
    assert xn.shape == h.shape == (3, D)


def test_attention_and_kv_operators_propagate_shapes():
    B, H, Hkv = 3, 32, 4
    bf, i32 = torch.bfloat16, torch.int32
    pool = _m((64, Hkv, 2, 2048), bf)
    out = J.paged_decode_attention_qkv(_m((B, (H + 2 * Hkv) * 128), bf), H, Hkv, _m((128,), bf), _m((128,), bf), 1e-6,
                                       _m((64,), torch.float32), pool, _m((B, 16), i32), _m((B,), i32),
                                       _m((B + 1,), i32), _m((8,), i32), 8, 200, 128 ** -0.5,
                                       _m((1 << 16,), torch.uint8))
    assert out.shape == (B, H, 128) and out.dtype == bf
    q = _m((70, H, 128), bf)
    o = J.paged_prefill_attention(q, pool, _m((2, 16), i32), _m((4, 2), i32), _m((3, 5), i32), [0, 0, 50, 1, 30, 20],
                                  1, 50, 128 ** -0.5, _m((16,), torch.uint8))
    assert o.shape == q.shape
    assert J.kv_append_paged(pool, _m((B, Hkv, 128), bf), _m((B, Hkv, 128), bf), _m((B,), i32),
                             _m((B, 16), i32)) is None
    assert J.kv_copy_pages(pool, _m((2,), i32), _m((2,), i32)) is None


def test_packed_matrix_refuses_data_of_another_size():
    """A PackedQ4 (what the operators build from a byte tensor and (E, N, K)) checks the byte count
    against the layout before any kernel reads it."""
    from jitengine_amd import ops

    n = ops.packed_bytes(2, 32, 256)
    assert n > 0
    ops.PackedQ4(torch.zeros(n, dtype=torch.uint8), 2, 32, 256, True)
    with pytest.raises(ValueError):
        ops.PackedQ4(torch.zeros(n - 1, dtype=torch.uint8), 2, 32, 256, True)
    with pytest.raises(ValueError):
        ops.PackedQ4(torch.zeros(n // 4, dtype=torch.int32), 2, 32, 256, True)
    with pytest.raises(ops._lib.UnsupportedShape):
        ops.PackedQ4(torch.zeros(n, dtype=torch.uint8), 2, 33, 256, True)
