"""Paged KV pool: page allocator, per-sequence page lists and page tables.

The reference keeps one contiguous growable [1, Hkv, cap, Dh] buffer per request and layer
(KVSlot, Q36/kvcache/kv_cache.py:27-85).  The build replaces it with a pool of 16-token pages per
layer, [num_pages, Hkv, 2, 16 * 128] bf16: for each kv head, part 0 of a page holds K
chunk-major ([d / 32][slot][d % 32]) and part 1 holds V dim-major ([d][slot]) -- the operand
layouts the attention kernel reads, with one kv head's K and V one contiguous 8 KiB block.  A sequence owns a list of pages, the
same page ids in every layer; token t sits in page pages[t // 16], slot t % 16.  The pool is
zero-initialised, so every slot of an allocated page always holds finite values.
"""

from __future__ import annotations

import numpy as np
import torch

from .ops import HEAD_DIM, PAGE


class PoolExhausted(RuntimeError):
    pass


class KVPool:
    """`n_layers` pools of `num_pages` pages for `n_kv_heads` heads of dim 128 on `device`.

    `seed` given: free pages are handed out in a seeded random permutation (the configs' page
    tables are "a random permutation of free pages"); otherwise in ascending order."""

    def __init__(self, n_layers: int, num_pages: int, n_kv_heads: int, device, seed: int | None = None,
                 allocate: bool = True):
        if num_pages <= 0 or n_layers <= 0 or n_kv_heads <= 0:
            raise ValueError("KVPool needs positive layers, pages and heads")
        self.n_layers, self.num_pages, self.n_kv_heads = int(n_layers), int(num_pages), int(n_kv_heads)
        self.device = torch.device(device)
        order = np.arange(num_pages) if seed is None else np.random.default_rng(seed).permutation(num_pages)
        self._free = [int(p) for p in order[::-1]]  # pop() hands out order[0] first
        self.pages: dict = {}
        self.lengths: dict = {}
        self.pools = (
            [torch.zeros((num_pages, n_kv_heads, 2, PAGE * HEAD_DIM), dtype=torch.bfloat16, device=self.device)
             for _ in range(n_layers)]
            if allocate else []
        )

    @property
    def page_bytes(self) -> int:
        """Bytes of one page in one layer (K and V of every kv head)."""
        return 2 * self.n_kv_heads * PAGE * HEAD_DIM * 2

    @property
    def free_pages(self) -> int:
        return len(self._free)

    def reserve(self, seq_id, n_tokens: int) -> list:
        """Make sequence `seq_id` hold room for `n_tokens` tokens; returns its page list."""
        pages = self.pages.setdefault(seq_id, [])
        self.lengths.setdefault(seq_id, 0)
        need = -(-int(n_tokens) // PAGE) - len(pages)
        if need > len(self._free):
            raise PoolExhausted(f"{need} pages needed, {len(self._free)} free")
        for _ in range(max(0, need)):
            pages.append(self._free.pop())
        return pages

    def set_length(self, seq_id, n_tokens: int) -> None:
        """Record that the first n_tokens positions of `seq_id` are valid (reserving pages)."""
        self.reserve(seq_id, n_tokens)
        self.lengths[seq_id] = int(n_tokens)

    def release(self, seq_id) -> None:
        """Return a sequence's pages to the free list."""
        for p in reversed(self.pages.pop(seq_id, [])):
            self._free.append(p)
        self.lengths.pop(seq_id, None)

    def page_table(self, seq_ids, width: int | None = None) -> torch.Tensor:
        """int32 [B, width] page ids of the given sequences (unused entries 0, never read)."""
        rows = [self.pages.get(s, []) for s in seq_ids]
        w = max([len(r) for r in rows] + [1]) if width is None else int(width)
        t = np.zeros((len(rows), w), np.int32)
        for i, r in enumerate(rows):
            if len(r) > w:
                raise ValueError(f"sequence {seq_ids[i]} has {len(r)} pages, the table is {w} wide")
            t[i, : len(r)] = r
        return torch.from_numpy(t).to(self.device)
