"""The allocation-free decode attention (jit_paged_decode_attn_noalloc, partials in the library's
fixed device scratch) against the workspace entry point (jit_paged_decode_attn) through the C-ABI:
the same kernels, so the same bits.  Two calls in a row, the second on a smaller input (the scratch
keeps the first call's partials), then the size limit, which must fail before any launch."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from jitengine_amd import _lib, ops
from tests.helpers import bf16_tensor, normal_bf16

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(lens, seed, H=32, Hkv=4):
    rng = np.random.default_rng(seed)
    npg = [-(-L // 16) for L in lens]
    total = sum(npg) + 3
    perm = rng.permutation(total)
    table = np.zeros((len(lens), max(npg)), np.int32)
    at = 0
    for i, n in enumerate(npg):
        table[i, :n] = perm[at:at + n]
        at += n
    pool = bf16_tensor(normal_bf16((total, Hkv, 2, 16 * 128), seed=seed + 1), DEV)
    q = bf16_tensor(normal_bf16((len(lens), H, 128), seed=seed + 2), DEV)
    return q, pool, torch.from_numpy(table).to(DEV), ops.attn_plan(lens, DEV)


def _both(q, pool, table, plan):
    scale = 128 ** -0.5
    want = ops.paged_decode_attention(q, pool, table, plan, scale)
    out = torch.full_like(q, float("nan"))
    got = ops.paged_decode_attention_noalloc(q, pool, table, plan, scale, out)
    torch.cuda.synchronize()
    return got, want


def _full_case(seed):
    """The largest plan the scratch holds: 16 sequences of 126 chunks of 1,536 keys (2,016 chunks),
    16 q heads over one kv head (8,320 bytes of partials per chunk: 16.0 of the 16 MiB)."""
    H, Hkv, n_seq, L = 16, 1, 16, 126 * 1536
    npg = L // 16
    g = torch.Generator(device=DEV).manual_seed(seed)
    pool = torch.randn((n_seq * npg + 1, Hkv, 2, 16 * 128), generator=g, device=DEV).to(torch.bfloat16)
    table = torch.randperm(n_seq * npg + 1, generator=g, device=DEV)[:n_seq * npg].view(n_seq, npg).to(torch.int32)
    q = torch.randn((n_seq, H, 128), generator=g, device=DEV).to(torch.bfloat16)
    return q, pool, table.contiguous(), ops.attn_plan([L] * n_seq, DEV)


def test_noalloc_equals_workspace_entry_two_calls():
    # first call: the whole scratch in use
    q, pool, table, plan = _full_case(seed=90)
    assert ops.attn_workspace_bytes(plan.total, 16) <= _lib.JIT_ATTN_SCRATCH_BYTES
    print(f"noalloc call 1: 16 x 193,536 keys, {plan.total} chunks", flush=True)
    got, want = _both(q, pool, table, plan)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    del q, pool, table
    # second call, smaller: ragged lengths, multi-chunk sequences (merge path) among one-chunk ones
    lens1 = [262144, 60000, 5000, 1537, 300, 17, 1]
    q, pool, table, plan = _case(lens1, seed=91)
    print(f"noalloc call 2: lens {lens1}, {plan.total} chunks", flush=True)
    got, want = _both(q, pool, table, plan)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # third call, smaller still: most of the scratch keeps the earlier calls' partials
    lens2 = [4000, 3100, 40]
    q, pool, table, plan = _case(lens2, seed=92, H=16, Hkv=2)
    print(f"noalloc call 3: lens {lens2}, {plan.total} chunks", flush=True)
    got, want = _both(q, pool, table, plan)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # the same call again on the same stream gives the same bits
    got2, _ = _both(q, pool, table, plan)
    assert torch.equal(got2.view(torch.int16), want.view(torch.int16))


def test_noalloc_allocates_no_device_memory():
    """After one warm call, further calls (inputs and `out` allocated beforehand) change neither the
    device's free memory (an allocation inside the library would take at least a 2 MiB page of it)
    nor torch's count of allocations."""
    lens = [262144, 5000, 17]
    q, pool, table, plan = _case(lens, seed=93)
    out = torch.empty_like(q)
    scale = 128 ** -0.5
    ops.paged_decode_attention_noalloc(q, pool, table, plan, scale, out)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    allocs0 = torch.cuda.memory_stats().get("allocation.all.allocated", 0)
    for _ in range(5):
        ops.paged_decode_attention_noalloc(q, pool, table, plan, scale, out)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    allocs1 = torch.cuda.memory_stats().get("allocation.all.allocated", 0)
    assert abs(free1 - free0) < (2 << 20), (free0, free1)
    assert allocs1 == allocs0, (allocs0, allocs1)


def test_noalloc_rejects_partials_past_the_scratch():
    lib = _lib.lib()
    per_chunk = lib.jit_attn_workspace_bytes(1, 32)
    too_many = _lib.JIT_ATTN_SCRATCH_BYTES // per_chunk + 1
    rc = lib.jit_paged_decode_attn_noalloc(None, None, None, 16, None, None, None, 1, 32, 4, 0.1, too_many,
                                           None, None)
    assert rc == _lib.JIT_EUNSUPPORTED
    assert b"scratch" in lib.jit_last_error()
    ok = _lib.JIT_ATTN_SCRATCH_BYTES // per_chunk
    assert lib.jit_attn_workspace_bytes(ok, 32) <= _lib.JIT_ATTN_SCRATCH_BYTES
