"""jit_moe_gate_up_swiglu_routed_packed (a one-token step's top-k and packing inside its gate||up
launch) against the launches it replaces, jit_route_pack then jit_moe_gate_up_swiglu_packed: the
same top-k, scores, packing tables and h bits, on the GPU."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from jitengine_amd import ops
from jitengine_amd.quant import random_quantized
from tests.helpers import bf16_tensor, normal_bf16, u16

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _logits(E, seed, ties):
    rng = np.random.default_rng(seed)
    v = rng.standard_normal(E).astype(np.float32) * 3
    if ties:  # repeated values and exact ties around the k-th place: the index breaks them
        v[::7] = v[1]
        v[3] = v[5] = v.max()
    return torch.from_numpy(v[None, :]).to(torch.bfloat16).to(DEV)


@pytest.mark.parametrize("E,k,norm,ties", [(128, 8, True, False), (128, 8, True, True), (64, 4, False, True),
                                          (32, 2, True, False), (96, 8, False, False)])
def test_routed_gate_up_equals_route_pack_then_gate_up(E, k, norm, ties):
    D, I = 2048, 768
    gu = ops.prepack(random_quantized((E, 2 * I, D), 100 + E + k, device=DEV))
    x = bf16_tensor(normal_bf16((1, D), seed=E + k), DEV)
    logits = _logits(E, E * 10 + k, ties)
    inds0, scores0, pk0 = ops.route_pack(logits, k, norm)
    h0 = ops.expert_gate_up(x, gu, pk0)
    inds1, scores1, pk1, h1 = ops.route_gate_up(x, logits, gu, k, norm)
    torch.cuda.synchronize()
    assert torch.equal(inds0, inds1)
    assert torch.equal(scores0.view(torch.int16), scores1.view(torch.int16))
    for name in ("order", "pair_row", "inv", "expert_cnt", "expert_off", "meta"):
        assert torch.equal(getattr(pk0, name), getattr(pk1, name)), name
    for name in ("seg_expert", "seg_start", "seg_cnt"):  # (entries past the k segments are unspecified)
        assert torch.equal(getattr(pk0, name)[:k], getattr(pk1, name)[:k]), name
    assert np.array_equal(u16(h0), u16(h1))


def test_routed_gate_up_rejects_what_it_does_not_cover():
    gu = ops.prepack(random_quantized((8, 2 * 64, 512), 3, device=DEV))
    x = torch.zeros((1, 512), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ops._lib.UnsupportedShape):  # E % 32 != 0
        ops.route_gate_up(x, torch.zeros((1, 8), dtype=torch.bfloat16, device=DEV), gu, 2, True)
    with pytest.raises(ops._lib.UnsupportedShape):  # two tokens
        ops.route_gate_up(torch.zeros((2, 512), dtype=torch.bfloat16, device=DEV),
                          torch.zeros((2, 8), dtype=torch.bfloat16, device=DEV), gu, 2, True)
