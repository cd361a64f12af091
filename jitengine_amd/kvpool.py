"""Paged KV pool: page allocator with reference counts, per-sequence page lists, copy-on-write,
and the page-level prefix store.

The reference keeps one contiguous growable [1, Hkv, cap, Dh] buffer per request and layer
(KVSlot, Q36/kvcache/kv_cache.py:27-85), and its prefix cache stores snapshot COPIES of a
request's KV that a later request copies back (RequestState.snapshot / restore,
Q36/kvcache/state.py:58-149; PrefixStore, Q36/kvcache/prefix_cache.py).  Here the KV lives in a
pool of 16-token pages per layer, [num_pages, Hkv, 2, 16 * 128] bf16 (for each kv head, part 0
holds K chunk-major ([d / 32][slot][d % 32]) and part 1 holds V dim-major ([d][slot]) -- the
operand layouts the attention kernels read).  A sequence owns a list of pages, the same page ids
in every layer; token t sits in page pages[t // 16], slot t % 16.  Sharing a prefix is sharing its
pages: each page carries a reference count, and a sequence about to write into a page that someone
else also holds first copies it (jit_kv_copy_pages), so a shared page is never written.  The pool
is zero-initialised, so every slot of an allocated page always holds finite values.
"""

from __future__ import annotations

from collections import OrderedDict

import numpy as np
import torch

from . import ops
from .ops import HEAD_DIM, PAGE


class PoolExhausted(RuntimeError):
    pass


def pages_for(n_tokens: int) -> int:
    return -(-int(n_tokens) // PAGE)


class KVPool:
    """`n_layers` pools of `num_pages` pages for `n_kv_heads` heads of dim 128 on `device`.

    `seed` given: free pages are handed out in a seeded random permutation (the configs' page
    tables are "a random permutation of free pages"); otherwise in ascending order.  With
    allocate=False no device memory is made (bookkeeping only)."""

    def __init__(self, n_layers: int, num_pages: int, n_kv_heads: int, device, seed: int | None = None,
                 allocate: bool = True):
        if num_pages <= 0 or n_layers <= 0 or n_kv_heads <= 0:
            raise ValueError("KVPool needs positive layers, pages and heads")
        self.n_layers, self.num_pages, self.n_kv_heads = int(n_layers), int(num_pages), int(n_kv_heads)
        self.device = torch.device(device)
        order = np.arange(num_pages) if seed is None else np.random.default_rng(seed).permutation(num_pages)
        self._free = [int(p) for p in order[::-1]]  # pop() hands out order[0] first
        self.refs = np.zeros(num_pages, np.int32)
        self.pages: dict = {}
        self.lengths: dict = {}
        self.copies = 0  # pages copied on write so far
        self.pools = (
            [torch.zeros((num_pages, n_kv_heads, 2, PAGE * HEAD_DIM), dtype=torch.bfloat16, device=self.device)
             for _ in range(n_layers)]
            if allocate else []
        )

    # ------------------------------------------------------------------ pages
    @property
    def page_bytes(self) -> int:
        """Bytes of one page in one layer (K and V of every kv head)."""
        return 2 * self.n_kv_heads * PAGE * HEAD_DIM * 2

    @property
    def free_pages(self) -> int:
        return len(self._free)

    def alloc(self, n: int) -> list:
        """n fresh pages (reference count 1)."""
        if n > len(self._free):
            raise PoolExhausted(f"{n} pages needed, {len(self._free)} free")
        out = [self._free.pop() for _ in range(int(n))]
        self.refs[out] = 1
        return out

    def incref(self, pages) -> None:
        for p in pages:
            if self.refs[p] <= 0:
                raise ValueError(f"page {p} is free")
            self.refs[p] += 1

    def decref(self, pages) -> None:
        for p in reversed(list(pages)):
            if self.refs[p] <= 0:
                raise ValueError(f"page {p} is already free")
            self.refs[p] -= 1
            if self.refs[p] == 0:
                self._free.append(int(p))

    def copy_pages(self, src: list, dst: list) -> None:
        """Device copy of pages src[i] -> dst[i] in every layer."""
        if not src or not self.pools:
            return
        s = ops.upload(np.asarray(src, np.int32), self.device)
        d = ops.upload(np.asarray(dst, np.int32), self.device)
        for pool in self.pools:
            ops.kv_copy_pages(pool, s, d)

    # -------------------------------------------------------------- sequences
    def open(self, seq_id, pages=(), length: int = 0) -> None:
        """Start sequence `seq_id` holding `pages` (shared: each gains a reference) with the first
        `length` positions valid."""
        if seq_id in self.pages:
            raise ValueError(f"sequence {seq_id} is open")
        if pages_for(length) > len(pages):
            raise ValueError(f"{length} positions do not fit {len(pages)} pages")
        self.incref(pages)
        self.pages[seq_id] = list(pages)
        self.lengths[seq_id] = int(length)

    def reserve(self, seq_id, n_tokens: int) -> list:
        """Make sequence `seq_id` hold room for `n_tokens` tokens; returns its page list."""
        pages = self.pages.setdefault(seq_id, [])
        self.lengths.setdefault(seq_id, 0)
        need = pages_for(n_tokens) - len(pages)
        if need > 0:
            pages += self.alloc(need)
        return pages

    def prepare_write(self, seq_id, start: int, n: int) -> list:
        """Before positions [start, start + n) of `seq_id` are written: pages reserved, and every
        page in that range that another holder shares is replaced by a private copy.  Returns the
        page list."""
        pages = self.reserve(seq_id, start + n)
        src, dst = [], []
        for i in range(start // PAGE, pages_for(start + n)):
            p = pages[i]
            if self.refs[p] > 1:
                q = self.alloc(1)[0]
                src.append(p)
                dst.append(q)
                self.decref([p])
                pages[i] = q
        self.copy_pages(src, dst)
        self.copies += len(src)
        return pages

    def set_length(self, seq_id, n_tokens: int) -> None:
        """Record that the first n_tokens positions of `seq_id` are valid (reserving pages)."""
        self.reserve(seq_id, n_tokens)
        self.lengths[seq_id] = int(n_tokens)

    def release(self, seq_id) -> None:
        """Drop a sequence's hold on its pages (pages nobody else holds become free)."""
        self.decref(self.pages.pop(seq_id, []))
        self.lengths.pop(seq_id, None)

    def page_table(self, seq_ids, width: int | None = None) -> torch.Tensor:
        """int32 [B, width] page ids of the given sequences (unused entries 0, never read)."""
        return ops.upload(self.page_table_host(seq_ids, width), self.device)

    def page_table_host(self, seq_ids, width: int | None = None) -> np.ndarray:
        rows = [self.pages.get(s, []) for s in seq_ids]
        w = max([len(r) for r in rows] + [1]) if width is None else int(width)
        t = np.zeros((len(rows), w), np.int32)
        for i, r in enumerate(rows):
            if len(r) > w:
                raise ValueError(f"sequence {seq_ids[i]} has {len(r)} pages, the table is {w} wide")
            t[i, : len(r)] = r
        return t


class PrefixStore:
    """Stored prefixes keyed by their token ids, each holding references on the pages of its KV.

    In place of the reference's snapshot copies (Q36/kvcache/state.py:58-149): storing a prefix
    takes a reference on its pages, restoring it opens the new sequence on the same pages, and the
    first write into a shared page copies that one page (KVPool.prepare_write).  Entries are
    evicted least recently used first when the pool needs pages."""

    def __init__(self, pool: KVPool, max_entries: int = 64, min_tokens: int = PAGE):
        self.pool = pool
        self.max_entries = int(max_entries)
        self.min_tokens = int(min_tokens)
        self.entries: OrderedDict = OrderedDict()  # key tuple -> page list
        self.hits = 0

    def insert(self, tokens, pages) -> bool:
        """Store the prefix `tokens` whose KV sits in `pages` (its first pages_for(len) pages)."""
        key = tuple(int(t) for t in tokens)
        if len(key) < self.min_tokens or key in self.entries:
            if key in self.entries:
                self.entries.move_to_end(key)
            return False
        held = list(pages[: pages_for(len(key))])
        self.pool.incref(held)
        self.entries[key] = held
        while len(self.entries) > self.max_entries:
            self.evict_one()
        return True

    def lookup(self, prompt) -> tuple:
        """(n, pages): the longest stored prefix of `prompt` shorter than the prompt (at least one
        prompt token is left to compute), or (0, [])."""
        prompt = tuple(int(t) for t in prompt)
        best = None
        for key in self.entries:
            if len(key) < len(prompt) and (best is None or len(key) > len(best)) and prompt[: len(key)] == key:
                best = key
        if best is None:
            return 0, []
        self.entries.move_to_end(best)
        self.hits += 1
        return len(best), list(self.entries[best])

    def evict_one(self) -> bool:
        if not self.entries:
            return False
        _, pages = self.entries.popitem(last=False)
        self.pool.decref(pages)
        return True

    def make_room(self, n_pages: int) -> None:
        """Evict entries until n_pages are free or the store is empty."""
        while self.pool.free_pages < n_pages and self.evict_one():
            pass
