"""jit_paged_decode_attn_qkv (the step's q/k norm + RoPE + KV append inside the attention launch)
against the two launches it replaces, jit_qk_norm_rope_append then jit_paged_decode_attn: the same
output bits and the same pool bits, on the GPU."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from jitengine_amd import ops
from jitengine_amd.model import rope_inv_freq
from tests.helpers import bf16_tensor, normal_bf16, u16

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(lens, H, Hkv, seed):
    """Rows whose token sits at position lens[b] - 1, the keys before it in permuted pages."""
    rng = np.random.default_rng(seed)
    npg = [-(-L // 16) for L in lens]
    total = sum(npg) + 3
    perm = rng.permutation(total)
    table = np.zeros((len(lens), max(npg)), np.int32)
    at = 0
    for b, n in enumerate(npg):
        table[b, :n] = perm[at:at + n]
        at += n
    pool = normal_bf16((total, Hkv, 2, 2048), seed=seed + 1)
    qkv = normal_bf16((len(lens), (H + 2 * Hkv) * 128), seed=seed + 2, scale=1.5)
    qn = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
    kn = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
    return pool, table, qkv, qn, kn


@pytest.mark.parametrize("lens,H,Hkv", [
    ([1, 2, 17, 33, 1536, 1537, 3000, 4097, 30000], 32, 4),  # one key; step-0 tokens; chunk edges
    ([129, 1600, 5000], 16, 1),                              # G = 16, one kv head a workgroup
    ([40, 2000], 8, 8),                                      # G = 1
    ([200_001], 32, 4),                                      # past 128 chunks: the long-sequence rule
])
def test_fused_equals_norm_rope_append_then_attention(lens, H, Hkv):
    pool, table, qkv, qn, kn = _case(lens, H, Hkv, seed=len(lens) * 7 + H)
    lens_a = np.array(lens, np.int32)
    inv = torch.from_numpy(rope_inv_freq(1e6, 128)).to(DEV)
    qkv_t, tab = bf16_tensor(qkv, DEV), torch.from_numpy(table).to(DEV)
    qn_t = torch.from_numpy(qn).to(DEV).to(torch.bfloat16)
    kn_t = torch.from_numpy(kn).to(DEV).to(torch.bfloat16)
    plan = ops.attn_plan(lens_a, DEV)
    scale = 128 ** -0.5
    pool_a, pool_b = bf16_tensor(pool, DEV), bf16_tensor(pool, DEV)
    pos = torch.from_numpy(lens_a - 1).to(DEV)
    q = ops.qk_norm_rope_append(qkv_t, H, Hkv, qn_t, kn_t, 1e-6, inv, pos, tab, pool_b)
    want = ops.paged_decode_attention(q, pool_b, tab, plan, scale)
    got = ops.paged_decode_attention_qkv(qkv_t, H, Hkv, qn_t, kn_t, 1e-6, inv, pool_a, tab, plan, scale)
    torch.cuda.synchronize()
    assert np.array_equal(u16(got), u16(want))
    assert np.array_equal(u16(pool_a), u16(pool_b))  # the tokens' K and V, nothing else


def test_fused_rejects_what_attention_rejects():
    z = torch.zeros((2, (30 + 8) * 128), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        ops.paged_decode_attention_qkv(z, 30, 4, z[0, :128], z[0, :128], 1e-6,
                                       torch.zeros(64, device=DEV), torch.zeros((4, 4, 2, 2048), dtype=torch.bfloat16,
                                                                                 device=DEV),
                                       torch.zeros((2, 1), dtype=torch.int32, device=DEV),
                                       ops.attn_plan([3, 4], DEV), 0.1)
