"""Continuous-batching generation over the paged KV pool.

Mirrors the reference's scheduler loop (Q36/scheduler/scheduler.py, admission.py, prefill.py,
decode.py, retire.py) on this build's pieces:
  * admission (AdmissionMixin._admit, Q36/scheduler/admission.py:19-51): strict FIFO; a request is
    charged its whole generation (prompt + max_tokens positions, :82-88) in KV pages up front, and
    the first request that does not fit stops admission until pages come back;
  * a prefix already in the prefix store is restored instead of recomputed -- here by sharing its
    pages (PrefixStore), where the reference copies a snapshot (Q36/kvcache/state.py:121-149);
  * every step runs the decoding rows (one token each) as one batched decode step
    (Model.decode_step, on the decode kernels whatever the batch size) and prompt chunks of the
    requests still in prefill, each chunk a forward of its own (max_step_tokens rows in all);
  * a generation depends on its request alone, as in the reference (Q36/scheduler/prefill.py:1-6):
    prompt chunks end at absolute multiples of prefill_chunk and a stored prefix is restored only
    at such a multiple, so a prompt position is always computed in a chunk of the same rows, with
    the same kernels (a chunk of 192 or more rows takes the segment GEMMs), cold, warm or batched;
  * a request retires on an end-of-sequence token or after max_tokens tokens
    (Q36/scheduler/retire.py); its prompt's pages then go to the prefix store and the rest of its
    reservation back to the pool;
  * decode pipelining (DecodingMixin._pump, Q36/scheduler/decode.py:21-114): while only decoding
    rows are left, the next step is issued -- fed by this step's tokens on the device, its
    positions known on the host -- before this step's tokens are read, so the host's bookkeeping
    overlaps the GPU's step; a row that stops on an end-of-sequence token costs one discarded step,
    as in the reference.
Tokens are drawn on the GPU by each request's Sampler (DecodingMixin._draw, Q36/scheduler/decode.py:116-
176): greedy (jit_argmax_rows) or temperature / top-p / top-k under the request's own key stream
(jit_sample_rows), the rows of equal settings in one launch, each drawing token n with its step-n
key, so a request's tokens do not depend on the batch.
"""

from __future__ import annotations

import itertools
from collections import deque
from dataclasses import dataclass, field

import numpy as np
import torch

from . import ops
from . import selfcheck as _selfcheck
from .kvpool import KVPool, PoolExhausted, PrefixStore, pages_for
from .ops import PAGE
from .model import CausalLM, make_mixed_state, make_step_state
from .sampler import Sampler, sample_rows


@dataclass
class Request:
    rid: int
    prompt: list
    max_tokens: int
    eos: frozenset
    tokens: list = field(default_factory=list)  # generated so far
    done_prompt: int = 0   # prompt positions whose KV is written (restored ones included)
    cached: int = 0        # prompt positions restored from the prefix store
    state: str = "queued"  # queued -> prefill -> decode -> done
    finish_reason: str | None = None
    reserved: int = 0      # pages charged at admission and not yet allocated
    sampler: Sampler | None = None  # (None: greedy)

    @property
    def length(self) -> int:
        """KV positions written so far."""
        return self.done_prompt + max(0, len(self.tokens) - 1)


class Engine:
    """Requests in, tokens out, many sequences per step over one KV pool."""

    def __init__(self, lm: CausalLM, num_pages: int, prefill_chunk: int = 512, max_step_tokens: int = 2048,
                 prefix_store: bool = True, page_seed: int | None = None, device=None, allocate: bool = True,
                 pipeline: bool = True, selfcheck: bool = False):
        if prefill_chunk <= 0 or max_step_tokens <= 0:
            raise ValueError("prefill_chunk and max_step_tokens must be positive")
        if prefill_chunk > max_step_tokens:
            raise ValueError(f"a prompt chunk ({prefill_chunk} rows) must fit a step ({max_step_tokens} rows)")
        self.lm = lm
        cfg = lm.cfg
        dev = device if device is not None else lm.final_norm.device
        self.device = torch.device(dev)
        if selfcheck or _selfcheck.enabled_by_env():  # the kernels against torch, once per device
            _selfcheck.run(self.device)
        self.pool = KVPool(len(lm.layers), num_pages, cfg.kv_heads, self.device, seed=page_seed, allocate=allocate)
        self.store = PrefixStore(self.pool) if prefix_store else None
        self.prefill_chunk = int(prefill_chunk)
        self.max_step_tokens = int(max_step_tokens)
        self.queue: deque = deque()
        self.rows: list = []       # admitted requests, in admission order
        self.outstanding = 0       # pages charged to admitted requests, not yet allocated
        self.deferred = 0          # admission attempts stopped by the pool
        self.steps = 0
        self.pipeline = bool(pipeline)
        self.pipelined = 0          # steps issued before the previous step's tokens were read
        self._inflight = None       # (rows, device tokens, pinned host copy, its event) of an unread step
        self._ids = itertools.count()

    # ------------------------------------------------------------------ requests
    def submit(self, prompt, max_tokens: int, eos=None, temperature: float = 0.0, top_p: float | None = None,
               top_k: int | None = None, seed: int | None = None) -> Request:
        """Queue a request; temperature > 0 samples with top_p / top_k under `seed`'s key stream
        (Sampler, Q36/scheduler/admission.py:104-113), else its tokens are greedy."""
        prompt = [int(t) for t in prompt]
        if not prompt:
            raise ValueError("empty prompt")
        if max_tokens < 1:
            raise ValueError("max_tokens must be >= 1")
        if min(prompt) < 0 or max(prompt) >= self.lm.vocab:
            raise ValueError(f"prompt token ids must lie in [0, {self.lm.vocab})")
        need = pages_for(len(prompt) + max_tokens)
        if need > self.pool.num_pages:
            raise PoolExhausted(f"a generation of {len(prompt) + max_tokens} positions needs {need} pages, "
                                f"the pool has {self.pool.num_pages}")
        eos = frozenset(self.lm.eos_ids if eos is None else eos)
        r = Request(next(self._ids), prompt, int(max_tokens), eos,
                    sampler=Sampler(temperature, top_p, top_k, seed, int(max_tokens), self.lm.vocab))
        self.queue.append(r)
        return r

    @property
    def busy(self) -> bool:
        return bool(self.queue or self.rows or self._inflight)

    def _admit(self) -> None:
        while self.queue:
            r = self.queue[0]
            total = pages_for(len(r.prompt) + r.max_tokens)
            n, pages = self._lookup(r.prompt)
            need = total - n // PAGE  # a shared partial page is copied before it is written
            if self.pool.free_pages - self.outstanding < need and self.store is not None:
                self.store.make_room(need + self.outstanding)
                n, pages = self._lookup(r.prompt)  # (the entry may have been evicted)
                need = total - n // PAGE
            if self.pool.free_pages - self.outstanding < need:
                self.deferred += 1
                break  # strict FIFO
            self.queue.popleft()
            self.pool.open(r.rid, pages[: pages_for(n)], n)
            r.done_prompt = r.cached = n
            r.reserved = need
            self.outstanding += need
            r.state = "prefill"
            self.rows.append(r)

    def _lookup(self, prompt) -> tuple:
        """The longest stored prefix of the prompt, cut back to a multiple of prefill_chunk (the chunk
        grid), so the rest of the prompt is computed in the same chunks as a cold run's."""
        if self.store is None:
            return 0, []
        n, pages = self.store.lookup(prompt)
        n = n // self.prefill_chunk * self.prefill_chunk
        return n, pages[: pages_for(n)]

    def _write(self, r: Request, start: int, n: int) -> None:
        before = self.pool.free_pages
        self.pool.prepare_write(r.rid, start, n)
        used = before - self.pool.free_pages
        r.reserved -= used
        self.outstanding -= used

    def _retire(self, r: Request, reason: str) -> None:
        r.state, r.finish_reason = "done", reason
        if self.store is not None:
            self.store.insert(r.prompt, self.pool.pages[r.rid])
        self.pool.release(r.rid)
        self.outstanding -= r.reserved
        r.reserved = 0
        self.rows.remove(r)

    # ---------------------------------------------------------------------- step
    def _draw(self, rows: list, h: torch.Tensor, steps: list) -> torch.Tensor:
        """The token of each row from its last-layer row h[i], int32 [B] on the device: the rows of
        equal sampler settings drawn in one launch, row i with its step-steps[i] key
        (DecodingMixin._draw / _draw_groups, Q36/scheduler/decode.py:116-176)."""
        samplers = [r.sampler for r in rows]
        keys = [s.rows_key() for s in samplers]
        if all(k is None for k in keys):
            return self.lm.greedy(h)
        logits = self.lm.logits(h)
        out = torch.empty(len(rows), dtype=torch.int32, device=logits.device)
        groups: dict = {}
        for i, k in enumerate(keys):
            groups.setdefault(k, []).append(i)
        for members in groups.values():
            idx = ops.upload(members, logits.device, torch.int64)
            sel = logits if len(members) == len(rows) else logits.index_select(0, idx).contiguous()
            tok = sample_rows(sel, [samplers[i] for i in members], [steps[i] for i in members])
            out.index_copy_(0, idx, tok)
        return out

    def _issue_decode(self, rows: list, ids, pos: np.ndarray, ahead: int = 0) -> torch.Tensor:
        """Launch one batched decode step over `rows` (ids: host list or int32 device tensor), whose
        tokens are each row's token len(tokens) + ahead; returns them, int32 [B] on the device (not
        read)."""
        lm = self.lm
        st = make_step_state(lm.cfg, pos, self.pool.page_table([r.rid for r in rows]))
        ids_t = ids if torch.is_tensor(ids) else ops.upload(ids, self.device, torch.int32)
        h = lm.model.decode_step(lm.embed_tokens(ids_t), self.pool.pools, st)
        return self._draw(rows, h, [len(r.tokens) + ahead for r in rows])

    def _can_pipeline(self, rows: list, ahead: int) -> bool:
        """Whether a decode step over `rows` may be issued with `ahead` steps' tokens still unread:
        no request waits to join, every row is decoding and needs that many more tokens."""
        return (self.pipeline and not self.queue and len(rows) == len(self.rows)
                and all(r.state == "decode" and len(r.tokens) + ahead < r.max_tokens for r in rows))

    def _in_flight(self, rows: list, toks: torch.Tensor) -> tuple:
        """A decode step left unread: its tokens' copy into pinned host memory is queued right behind
        it (before any later step), so reading them waits for this step alone, not for the step
        issued after it."""
        host = torch.empty(toks.shape, dtype=toks.dtype, pin_memory=True)
        host.copy_(toks, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        return rows, toks, host, ev

    def _pump(self) -> list:
        """Consume the step in flight, having issued the next one first when the rows allow."""
        rows, toks, host, ev = self._inflight
        self._inflight = None
        if self._can_pipeline(rows, 1):
            pos = np.array([r.length + 1 for r in rows], np.int32)
            for r in rows:
                self._write(r, r.length + 1, 1)
            self._inflight = self._in_flight(rows, self._issue_decode(rows, toks, pos, ahead=1))
            self.steps += 1
            self.pipelined += 1
        ev.synchronize()  # this step's tokens have landed; the next step may still be running
        drawn = [(r, t) for r, t in zip(rows, host.tolist()) if r.state != "done"]
        self._consume(drawn)
        return drawn

    def _consume(self, drawn: list) -> None:
        for r, t in drawn:
            r.tokens.append(int(t))
            r.state = "decode"
        for r in list(self.rows):
            if r.state == "decode" and r.tokens:
                self.pool.lengths[r.rid] = r.length
                if r.tokens[-1] in r.eos:
                    self._retire(r, "stop")
                elif len(r.tokens) >= r.max_tokens:
                    self._retire(r, "length")
            elif r.state == "prefill":
                self.pool.lengths[r.rid] = r.done_prompt

    def step(self) -> list:
        """One scheduling round; returns the (request, token) pairs it drew (with pipelining, the
        tokens of the step issued one round earlier)."""
        if self._inflight is not None:
            return self._pump()
        self._admit()
        decode = [r for r in self.rows if r.state == "decode"]
        pending = [r for r in self.rows if r.state == "prefill"]
        if pending:
            # the oldest pending prompt's next chunk always runs: when the decode rows leave it no
            # room, the step serves only as many of them as fit beside it (the others decode in the
            # next step; a row's tokens do not depend on the step it runs in), so a prompt's first
            # token never waits on the decode load
            n0 = self._chunk_len(pending[0])
            if len(decode) + n0 > self.max_step_tokens:
                decode = decode[:self.max_step_tokens - n0]
        budget = self.max_step_tokens - len(decode)
        chunks = []
        for r in pending:
            # the chunk up to the next multiple of prefill_chunk (or the prompt's end); a chunk that
            # does not fit the step's budget waits (strict FIFO), it is never cut short
            n = self._chunk_len(r)
            if n > budget:
                break
            chunks.append((r, r.done_prompt, n))
            budget -= n
        if not decode and not chunks:
            return []
        for r, ctx, n in chunks:
            self._write(r, ctx, n)
        for r in decode:
            self._write(r, r.length, 1)
        drawn = []
        if decode:
            dec_pos = np.array([r.length for r in decode], np.int32)
            toks = self._issue_decode(decode, [r.tokens[-1] for r in decode], dec_pos)
            if not chunks and self._can_pipeline(decode, 0):
                self.steps += 1
                self._inflight = self._in_flight(decode, toks)
                return []  # read at the next round, after the following step is issued
            drawn += list(zip(decode, toks.tolist()))
        for r, c, n in chunks:
            tok = self._prefill_chunk(r, c, n)
            r.done_prompt = c + n
            if tok is not None:
                drawn.append((r, tok))
        self.steps += 1
        self._consume(drawn)
        return drawn

    def _chunk_len(self, r: Request) -> int:
        """Rows of r's next prompt chunk: up to the next multiple of prefill_chunk (an absolute grid)
        or the prompt's end."""
        return min(self.prefill_chunk - r.done_prompt % self.prefill_chunk, len(r.prompt) - r.done_prompt)

    def _prefill_chunk(self, r: Request, c: int, n: int):
        """Prompt positions c .. c + n - 1 of request r as a forward of their own (the chunked-prefill
        layer step over one chunk); returns the drawn token when the chunk ends the prompt."""
        lm, dev = self.lm, self.device
        seq_table = self.pool.page_table_host([r.rid])
        ms = make_mixed_state(lm.cfg, [(0, c, n)], seq_table, np.zeros(0, np.int32),
                              np.zeros((0, seq_table.shape[1]), np.int32), dev)
        x = lm.embed_tokens(ops.upload(np.asarray(r.prompt[c:c + n], np.int32), dev))
        for layer, pool in zip(lm.layers, self.pool.pools):
            x = layer.mixed(x, pool, ms)
        if c + n < len(r.prompt):
            return None
        return int(self._draw([r], x[n - 1:n].contiguous(), [len(r.tokens)]).item())

    def run(self, max_steps: int | None = None) -> None:
        """Step until every submitted request is done (or max_steps rounds)."""
        n = 0
        while self.busy and (max_steps is None or n < max_steps):
            if not self.step() and not self.rows and self._inflight is None:
                if self.queue:
                    raise PoolExhausted("the queue head cannot be admitted into an idle pool")
                break
            n += 1
