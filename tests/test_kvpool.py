"""KV pool bookkeeping, the page-level prefix store and the engine's admission rule, on CPU
(no device memory: KVPool(allocate=False) keeps the page accounting only)."""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from jitengine_amd.engine import Engine
from jitengine_amd.kvpool import KVPool, PoolExhausted, PrefixStore, pages_for


def _pool(n=16, seed=None):
    return KVPool(2, n, 4, "cpu", seed=seed, allocate=False)


def test_alloc_refcount_and_free_list():
    p = _pool(8)
    a = p.alloc(3)
    assert a == [0, 1, 2] and p.free_pages == 5 and list(p.refs[a]) == [1, 1, 1]
    p.incref(a[:2])
    p.decref(a)
    assert p.free_pages == 6 and list(p.refs[:3]) == [1, 1, 0]
    p.decref(a[:2])
    assert p.free_pages == 8
    with pytest.raises(ValueError):
        p.decref([0])
    with pytest.raises(PoolExhausted):
        p.alloc(9)
    # seeded: pages come out in a fixed permutation
    q1, q2 = _pool(8, seed=3), _pool(8, seed=3)
    assert q1.alloc(8) == q2.alloc(8) and sorted(q1.refs.tolist()) == [1] * 8


def test_copy_on_write_of_a_shared_page():
    p = _pool(16)
    p.open("a")
    p.prepare_write("a", 0, 40)  # 3 pages, the last one partial
    pa = list(p.pages["a"])
    p.open("b", pa, 40)  # b shares all three
    assert list(p.refs[pa]) == [2, 2, 2]
    p.prepare_write("b", 40, 1)  # b writes position 40: page 2 is shared -> copied
    pb = p.pages["b"]
    assert pb[:2] == pa[:2] and pb[2] != pa[2] and p.copies == 1
    assert list(p.refs[pa]) == [2, 2, 1] and p.refs[pb[2]] == 1
    p.prepare_write("b", 41, 30)  # 41..70: page 2 is now b's own; pages 3, 4 are new
    assert p.copies == 1 and len(pb) == 5
    p.release("a")
    p.release("b")
    assert p.free_pages == 16 and not p.refs.any()


def test_prefix_store_lookup_insert_evict():
    p = _pool(32)
    s = PrefixStore(p, max_entries=2, min_tokens=4)
    p.open("a")
    p.prepare_write("a", 0, 20)
    assert s.insert(list(range(20)), p.pages["a"])
    assert not s.insert(list(range(3)), p.pages["a"])  # shorter than min_tokens
    p.release("a")
    assert p.free_pages == 32 - 2  # the store holds the two pages
    assert s.lookup(list(range(20))) == (0, [])  # a prefix must leave a token to compute
    n, pages = s.lookup(list(range(25)))
    assert n == 20 and len(pages) == 2
    assert s.lookup([1, 2, 3, 4, 5]) == (0, [])
    p.open("b")
    p.prepare_write("b", 0, 40)
    s.insert(list(range(100, 140)), p.pages["b"])
    p.open("c")
    p.prepare_write("c", 0, 8)
    s.insert(list(range(200, 208)), p.pages["c"])  # a third entry evicts the least recent
    assert len(s.entries) == 2 and tuple(range(20)) not in s.entries
    p.release("b")
    p.release("c")
    s.make_room(32)
    assert not s.entries and p.free_pages == 32


def _engine(num_pages, store=True, prefill_chunk=8):
    cfg = SimpleNamespace(kv_heads=4, heads=32)
    lm = SimpleNamespace(cfg=cfg, layers=[None, None], vocab=100, eos_ids=(99,),
                         final_norm=torch.zeros(1))
    return Engine(lm, num_pages, prefill_chunk=prefill_chunk, prefix_store=store, allocate=False)


def test_admission_is_fifo_and_charges_the_whole_generation():
    e = _engine(10)
    a = e.submit(list(range(40)), 40)   # 80 positions: 5 pages
    b = e.submit(list(range(50)), 46)   # 96 positions: 6 pages
    c = e.submit([1, 2, 3], 4)          # 1 page, but behind b
    e._admit()
    assert [r.rid for r in e.rows] == [a.rid] and e.outstanding == 5 and e.deferred == 1
    assert b.state == "queued" and c.state == "queued"  # strict FIFO: c waits behind b
    e._write(a, 0, 40)
    assert e.outstanding == 2 and a.reserved == 2 and e.pool.free_pages == 7
    e._retire(a, "length")  # the prompt's pages stay in the prefix store
    assert e.outstanding == 0 and e.pool.free_pages == 7
    e._admit()  # b restores a's 40-token prompt (2 full pages shared): 4 new pages; c 1
    assert [r.rid for r in e.rows] == [b.rid, c.rid] and b.cached == 40
    assert len(e.store.entries) == 1 and e.outstanding == 5 and e.pool.free_pages == 7
    with pytest.raises(ValueError):
        e.submit([], 3)
    with pytest.raises(ValueError):
        e.submit([100], 3)
    with pytest.raises(PoolExhausted):
        e.submit([1] * 150, 20)


def test_admission_restores_a_stored_prefix():
    e = _engine(20)
    a = e.submit(list(range(40)), 8)
    e._admit()
    e._write(a, 0, 40)
    a.done_prompt = 40
    e._retire(a, "length")
    assert len(e.store.entries) == 1 and e.pool.free_pages == 17
    b = e.submit(list(range(40)) + [7, 8, 9], 5)   # 48 positions: 3 pages, 2 of them shared full
    e._admit()
    assert b.cached == 40 and b.done_prompt == 40 and b.reserved == pages_for(48) - 2
    e._write(b, 40, 3)  # page 2 holds positions 32..39 of the stored prefix: copied, not written
    assert e.pool.copies == 1 and b.reserved == 0
    assert e.pool.pages[b.rid][:2] == e.store.entries[tuple(range(40))][:2]
    assert e.pool.pages[b.rid][2] != e.store.entries[tuple(range(40))][2]


def test_restore_is_cut_back_to_the_chunk_grid():
    """A stored prefix restores only up to a multiple of prefill_chunk (the reference's absolute chunk
    grid, Q36/scheduler/prefill.py:1-6), so the rest of the prompt is computed in the chunks of a cold
    run; a chunk never crosses a grid line and a chunk larger than a step is refused."""
    e = _engine(20, prefill_chunk=16)
    a = e.submit(list(range(40)), 8)
    e._admit()
    e._write(a, 0, 40)
    a.done_prompt = 40
    e._retire(a, "length")
    b = e.submit(list(range(40)) + [7, 8, 9], 5)
    e._admit()
    assert b.cached == 32 and b.done_prompt == 32 and len(e.pool.pages[b.rid]) == 2
    with pytest.raises(ValueError):
        Engine(SimpleNamespace(cfg=SimpleNamespace(kv_heads=4, heads=32), layers=[None], vocab=10, eos_ids=(),
                               final_norm=torch.zeros(1)), 4, prefill_chunk=64, max_step_tokens=32, allocate=False)
