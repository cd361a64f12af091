"""The C-ABI library loads, exports every entry point include/jit_moe.h declares, and checks its
scalar contract on the host (no GPU work: every call here returns before any launch)."""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest

from jitengine_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "jit_moe.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(jit_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    declared = _declared()
    assert len(declared) >= 14
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_lib.exported_symbols())
    assert lib.jit_version() >= 1


def test_contract_breaks_return_einval_before_launch():
    lib = _lib.lib()
    assert lib.jit_router_topk(None, 4, 128, 0, 1, None, None, None, None) == _lib.JIT_EINVAL
    assert lib.jit_router_topk(None, 4, 128, 129, 1, None, None, None, None) == _lib.JIT_EINVAL
    assert b"0 < k <= N" in lib.jit_last_error()
    assert lib.jit_router_topk(None, 4, 100, 8, 1, None, None, None, None) == _lib.JIT_EUNSUPPORTED
    assert lib.jit_router_topk(None, 4, 2048, 8, 1, None, None, None, None) == _lib.JIT_EUNSUPPORTED
    assert lib.jit_topk(None, 1, 8, 9, None, None) == _lib.JIT_EINVAL
    assert lib.jit_moe_pack(None, 10, 8, 128, *([None] * 9), None) == _lib.JIT_EINVAL  # P % k
    assert lib.jit_moe_pack(None, 16, 8, 2000, *([None] * 9), None) == _lib.JIT_EUNSUPPORTED
    assert lib.jit_route_pack(None, 1, 128, 0, 1, *([None] * 11), None) == _lib.JIT_EINVAL
    assert lib.jit_route_pack(None, 5, 128, 8, 1, *([None] * 11), None) == _lib.JIT_EUNSUPPORTED
    assert lib.jit_route_pack(None, 1, 256, 8, 1, *([None] * 11), None) == _lib.JIT_EUNSUPPORTED
    assert lib.jit_qmm(None, 4, 100, None, None, None, 64, None, None) == _lib.JIT_EUNSUPPORTED
    assert lib.jit_moe_down(None, 768 + 64, None, None, 8, None, None, None, 2048, 16, None, None) == _lib.JIT_EUNSUPPORTED
    assert lib.jit_paged_decode_attn(None, None, None, 4, None, None, None, 2, 30, 4, 0.1, 4, None, None, None) == _lib.JIT_EINVAL
    assert lib.jit_paged_decode_attn(None, None, None, 4, None, None, None, 2, 64, 2, 0.1, 4, None, None, None) == _lib.JIT_EUNSUPPORTED
    assert lib.jit_prefill_block_tokens(32, 4) == 32 and lib.jit_prefill_block_tokens(24, 8) == -1
    assert lib.jit_paged_prefill_attn(*([None] * 3), 16, *([None] * 4), 1, None, None, None, 1, 1, 1, 32, 3, 0.1,
                                      None, None, None) == _lib.JIT_EINVAL
    assert lib.jit_paged_prefill_attn(*([None] * 3), 16, *([None] * 4), 1, None, None, None, 1, 1, 1, 24, 8, 0.1,
                                      None, None, None) == _lib.JIT_EUNSUPPORTED
    # key parts: 48 steps of 128 keys; partials of 132 floats per (token, part, head); none for one part
    assert lib.jit_prefill_part_keys() == 6144
    assert lib.jit_prefill_workspace_bytes(10, 2, 32) == 10 * 2 * 32 * 132 * 4
    assert lib.jit_prefill_workspace_bytes(10, 1, 32) == 0 and lib.jit_prefill_workspace_bytes(10, 0, 32) == -1
    assert lib.jit_paged_prefill_attn(*([None] * 3), 16, *([None] * 4), 1, None, None, None, 1, 0, 1, 32, 4, 0.1,
                                      None, None, None) == _lib.JIT_EINVAL  # pmax < 1
    assert lib.jit_qmm_seg(None, 4, 2048, None, 128, None, None) == _lib.JIT_EUNSUPPORTED
    assert lib.jit_moe_combine_rmsnorm(None, None, None, 2, 8, 4096, None, None, None, 1e-6, None, None) == _lib.JIT_EUNSUPPORTED
    assert lib.jit_sample_rows(None, 2, 0, 1.0, 0.9, 5, None, None, None) == _lib.JIT_EINVAL
    assert lib.jit_sample_rows(None, 2, (1 << 19) + 1, 1.0, 0.9, 5, None, None, None) == _lib.JIT_EUNSUPPORTED
    dummy = ctypes.c_void_p(16)  # (never dereferenced: every call below returns before a launch)
    # tokens of two key parts need the partials' workspace
    assert lib.jit_paged_prefill_attn(dummy, dummy, dummy, 16, dummy, dummy, dummy, dummy, 1, dummy, dummy, dummy, 1,
                                      2, 1, 32, 4, 0.1, None, dummy, None) == _lib.JIT_EINVAL
    assert lib.jit_sample_rows(dummy, 2, 64, 1.0, 0.9, -1, dummy, dummy, None) == _lib.JIT_EINVAL
    assert lib.jit_sample_rows(dummy, 2, 64, float("nan"), 0.9, 5, dummy, dummy, None) == _lib.JIT_EINVAL
    assert lib.jit_sample_rows(dummy, 2, 64, 1.0, 0.9, 5, None, dummy, None) == _lib.JIT_EINVAL
    assert lib.jit_sample_rows(dummy, 2, 64, 1e-300, 0.9, 5, dummy, dummy, None) == _lib.JIT_EUNSUPPORTED
    assert lib.jit_logprobs_rows(None, -1, 64, None, None) == _lib.JIT_EINVAL
    need = lib.jit_sampler_workspace_bytes()
    assert need > 64 * 32768 * 4  # the per-row histograms of the split draws, and the partials
    ws = ctypes.c_void_p(256)
    assert lib.jit_logprobs_rows_ws(dummy, 2, 64, dummy, ws, need - 1, None) == _lib.JIT_EINVAL
    assert lib.jit_argmax_rows_ws(dummy, 2, 64, dummy, ctypes.c_void_p(264), need, None) == _lib.JIT_EINVAL
    assert b"16-byte aligned" in lib.jit_last_error()
    assert lib.jit_sample_rows_ws(dummy, 2, 64, 1.0, 0.9, 5, dummy, dummy, ws, 16, None) == _lib.JIT_EINVAL
    assert lib.jit_threefry_uniform(None, -1, None, None) == _lib.JIT_EINVAL
    # empty work is a no-op, not an error
    assert lib.jit_router_topk(None, 0, 128, 8, 1, None, None, None, None) == _lib.JIT_OK
    with pytest.raises(ValueError):
        _lib.check(_lib.JIT_EINVAL, "x")
    with pytest.raises(_lib.UnsupportedShape):
        _lib.check(_lib.JIT_EUNSUPPORTED, "x")


def test_attn_plan_is_a_function_of_each_length():
    lib = _lib.lib()
    lens = np.array([1, 255, 256, 1535, 1536, 1537, 16385, 196608, 196609, 200003, 262144, 1 << 20], np.int32)
    cs = np.zeros(lens.size + 1, np.int32)
    seq = np.zeros(2000, np.int32)
    total = lib.jit_attn_plan(lens.ctypes.data_as(ctypes.c_void_p), lens.size, cs.ctypes.data_as(ctypes.c_void_p),
                              seq.ctypes.data_as(ctypes.c_void_p), seq.size)
    ck = [lib.jit_attn_chunk_tokens(int(L)) for L in lens]
    n = [-(-int(L) // c) for L, c in zip(lens, ck)]
    # 1536-key chunks up to 128 of them; a longer sequence gets about 128 chunks, whole 128-key
    # steps (32 keys for each of 4 waves), at most 4096 keys (a wave's run of at most 64 pages)
    assert ck == [1536] * 8 + [1664, 1664, 2048, 4096]
    assert n[7:] == [128, 119, 121, 128, 256]
    assert total == sum(n)
    assert list(cs) == list(np.concatenate([[0], np.cumsum(n)]))
    for b in range(lens.size):
        assert np.all(seq[cs[b]:cs[b + 1]] == b)
    bad = np.array([5, 0], np.int32)
    assert lib.jit_attn_plan(bad.ctypes.data_as(ctypes.c_void_p), 2, cs.ctypes.data_as(ctypes.c_void_p), None, 0) == _lib.JIT_EINVAL


def test_workspace_bytes():
    lib = _lib.lib()
    assert lib.jit_attn_workspace_bytes(10, 32) == 10 * 32 * 130 * 4
    # packing: no workspace up to two tiles of 1024 pairs, then 4 (E + 1) bytes a tile
    assert lib.jit_moe_pack_workspace_bytes(2048, 128) == 0
    assert lib.jit_moe_pack_workspace_bytes(16864, 128) == 17 * 129 * 4
    assert lib.jit_moe_pack_workspace_bytes(16864, 1024) == 0
    assert lib.jit_moe_pack_ws(None, 16864, 8, 128, *([None] * 9), None, 17 * 129 * 4 - 1, None) == _lib.JIT_EINVAL
