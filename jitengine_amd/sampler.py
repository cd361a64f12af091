"""Token sampling on the GPU behind the reference's `Sampler` (Q36/sampler.py:320-383).

One `Sampler` per request, as in the reference: greedy when the temperature is 0, else
temperature / top-p / top-k draws in mlx_lm's order under the request's own key stream, so seeded
requests are reproducible and can share a batch (`sample_rows` draws the rows of one settings
group in one launch, Q36/sampler.py:479-543).  The draw itself is `jit_sample_rows` and the
uniform of a step key `jit_threefry_uniform`; this module derives the step keys on the host.

The key stream restates MLX's `mx.random.key` and `mx.random.split` (Threefry-2x32 counters (j,
j + num) for the 2 num words of `split(key, num)`) and the reference's block chain
(Sampler.key, Q36/sampler.py:351-365).  No known-answer vectors of MLX's split exist outside MLX,
so which key a step gets is not pinned against the reference (the Threefry function is, by its
published vectors); the draw given a key is.
"""

from __future__ import annotations

import os

import numpy as np
import torch

from . import ops

KEY_BLOCK = 256
_ROT = (13, 15, 26, 6, 17, 29, 16, 24)


def threefry2x32(key, c0, c1):
    """Threefry-2x32-20 (Salmon et al., SC'11) of counters (c0, c1) (uint32 arrays) under one key
    pair: the two output words."""
    k0, k1 = np.uint32(key[0]), np.uint32(key[1])
    ks = (k0, k1, np.uint32(k0 ^ k1 ^ np.uint32(0x1BD11BDA)))
    x0 = (np.asarray(c0, np.uint32) + ks[0]).astype(np.uint32)
    x1 = (np.asarray(c1, np.uint32) + ks[1]).astype(np.uint32)
    with np.errstate(over="ignore"):
        for i in range(5):
            for q in range(4):
                r = _ROT[(i & 1) * 4 + q]
                x0 = (x0 + x1).astype(np.uint32)
                x1 = ((x1 << np.uint32(r)) | (x1 >> np.uint32(32 - r))).astype(np.uint32)
                x1 = (x1 ^ x0).astype(np.uint32)
            x0 = (x0 + ks[(i + 1) % 3]).astype(np.uint32)
            x1 = (x1 + ks[(i + 2) % 3] + np.uint32(i + 1)).astype(np.uint32)
    return x0, x1


def key_from_seed(seed: int) -> np.ndarray:
    """mx.random.key(seed): the high and the low 32 bits of the 64-bit seed."""
    s = int(seed) & 0xFFFFFFFFFFFFFFFF
    return np.array([s >> 32, s & 0xFFFFFFFF], np.uint32)


def split(key, num: int) -> np.ndarray:
    """mx.random.split(key, num) -> [num, 2] uint32: the 2 num words of the key's random bits,
    word j and word j + num from counter (j, j + num)."""
    j = np.arange(num, dtype=np.uint32)
    x, y = threefry2x32(key, j, j + np.uint32(num))
    return np.concatenate([x, y]).reshape(num, 2)


class Sampler:
    """One per request (Q36/sampler.py:320-349): `__call__(logits [1, V], step)` -> token [1]."""

    def __init__(self, temperature: float, top_p: float | None, top_k: int | None, seed: int | None,
                 max_steps: int, vocab: int):
        self.temperature = float(temperature or 0.0)
        self.top_p = float(top_p if top_p is not None else 1.0)
        self.top_k = int(top_k or 0)
        self.max_steps = int(max_steps)
        self.greedy = self.temperature <= 0.0
        self._root = self._chain = None
        self._block = -1
        self._keys = None
        if not self.greedy:
            if self.top_k >= vocab:
                self.top_k = 0
            if seed is None:
                seed = int.from_bytes(os.urandom(8), "little")
            self._root = self._chain = key_from_seed(seed)

    def rows_key(self):
        """Samplers with equal rows keys draw as one batch (rows_key, Q36/sampler.py:479-483)."""
        return None if self.greedy else (self.temperature, self.top_p, self.top_k)

    def key(self, step: int) -> np.ndarray:
        """The key of `step`: block b = step // KEY_BLOCK has (block key, chain_{b+1}) =
        split(chain_b, 2) with chain_0 = the root, and its step keys split(block key,
        KEY_BLOCK) (Sampler.key, Q36/sampler.py:351-365)."""
        b = step // KEY_BLOCK
        if b != self._block:
            if b < self._block:
                self._chain, self._block = self._root, -1
            blk = None
            while self._block < b:
                blk, self._chain = split(self._chain, 2)
                self._block += 1
            self._keys = split(blk, KEY_BLOCK)
        return self._keys[step % KEY_BLOCK]

    def __call__(self, logits: torch.Tensor, step: int) -> torch.Tensor:
        return sample_rows(logits.reshape(1, -1), [self], [step])


def sample_rows(logits: torch.Tensor, samplers: list, steps: list) -> torch.Tensor:
    """int32 [B]: one draw per row of bf16 logits [B, V] for samplers that share a rows key (all
    greedy, or equal (temperature, top_p, top_k)); each row under its own step key."""
    s0 = samplers[0]
    if any(s.rows_key() != s0.rows_key() for s in samplers):
        raise ValueError("sample_rows takes samplers with one rows key")
    if s0.greedy:
        return ops.argmax_rows(logits)
    keys = np.stack([s.key(st) for s, st in zip(samplers, steps)]).view(np.int32)
    u = ops.threefry_uniform(ops.upload(keys, logits.device))
    return ops.sample_rows(logits, s0.temperature, s0.top_p, s0.top_k, u)
