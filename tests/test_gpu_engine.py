"""The step's ends (embedding, lm_head + greedy draw), KV page copies, the continuous-batching
engine and the checkpoint loader on MI355X.

Kernel parity: embedding and argmax bit-exact against the oracle, page copies bit-exact, logits
within the north-star tolerance.  Engine: generation is a function of each request alone --
bit-identical tokens whether a request runs alone or batched with staggered others, whether its
prompt's KV is computed or restored from the prefix store (shared pages, one copied), and when a
small pool defers admission.  The engine tests keep every step under 64 rows, where every op takes
its row-independent decode kernels (larger batches switch to the segment GEMMs, as the reference
switches to its prefill kernels): the engine keeps a generation independent of the batch by
computing prompt chunks on an absolute grid, each in a forward of its own, and decode rows on the
decode kernels at any batch size (test_engine_long_prompts_cold_warm_batched covers chunks of 512
rows, which take the segment GEMMs)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from jitengine_amd import checkpoint, ops
from jitengine_amd.engine import Engine
from jitengine_amd.model import CausalLM, DecoderLayer, Model, MoEConfig, random_causal_lm
from jitengine_amd.quant import QLinear, random_quantized
from tests.ckpt_util import config_dict, write_checkpoint
from tests.helpers import assert_close_bf16, bf16_tensor, normal_bf16, u16

pytestmark = pytest.mark.gpu
DEV = "cuda"
CFG = MoEConfig(layers=2, experts=32)
VOCAB = 2048


@pytest.fixture(scope="module")
def lm():
    return random_causal_lm(CFG, VOCAB, seed=11, device=DEV)


def _np(lin: QLinear):
    return (lin.weight.cpu().numpy().view(np.uint32), u16(lin.scales), u16(lin.biases))


def test_embed_q4_matches_oracle():
    tab = random_quantized((1000, 2048), 3, std=0.05, device=DEV)
    ids = np.array([0, 999, 17, 512, 1000, -1, 17], np.int32)
    got = u16(ops.embed_q4(torch.from_numpy(ids).to(DEV), tab))
    want = oracle.embed_q4(ids, *_np(tab))
    assert np.array_equal(got, want)
    assert not got[4].any() and not got[5].any() and np.array_equal(got[2], got[6])


@pytest.mark.parametrize("V", [151936, 1001])
def test_argmax_rows_matches_oracle(V):
    x = normal_bf16((6, V), seed=V)
    x[1, [5, 77, V - 1]] = 0x4300  # 128.0 three times: the first index wins
    x[2, 10:20] = 0x7FC0           # NaNs never win
    x[2, 30] = 0x4400
    x[3, :] = 0xFF80               # all -inf: index 0
    x[4, :] = 0x7FC0               # all NaN: index 0
    got = ops.argmax_rows(bf16_tensor(x, DEV)).cpu().numpy()
    want = oracle.argmax_rows(x)
    assert np.array_equal(got, want)
    assert got[1] == 5 and got[2] == 30 and got[3] == 0 and got[4] == 0
    ok = np.argmax(oracle.bf16_to_f32(x[[0, 5]]), axis=1)
    assert np.array_equal(got[[0, 5]], ok)


def test_kv_copy_pages_exact():
    pool = normal_bf16((12, 4, 2, 16 * 128), seed=9)
    pt = bf16_tensor(pool, DEV)
    src, dst = np.array([3, 7, 0], np.int32), np.array([5, 1, 11], np.int32)
    ops.kv_copy_pages(pt, torch.from_numpy(src).to(DEV), torch.from_numpy(dst).to(DEV))
    want = pool.copy()
    want[dst] = pool[src]
    assert np.array_equal(u16(pt), want)


def test_lm_logits_and_greedy(lm):
    h = normal_bf16((5, CFG.hidden), seed=4)
    logits = u16(lm.logits(bf16_tensor(h, DEV)))
    hn, _ = oracle.rmsnorm(h, u16(lm.final_norm), CFG.eps)
    _, want = oracle.qmm(hn, *_np(random_quantized((VOCAB, CFG.hidden), 11 * 10 + 9, device=DEV)))
    assert_close_bf16(logits, want, what="logits")
    assert np.array_equal(lm.greedy(bf16_tensor(h, DEV)).cpu().numpy(), oracle.argmax_rows(logits))


def _prompts(seed, lens):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, VOCAB, n).tolist() for n in lens]


_SAMPLING = ("temperature", "top_p", "top_k", "seed")


def _solo(lm, prompt, max_tokens, **kw):
    smp = {k: kw.pop(k) for k in _SAMPLING if k in kw}
    kw.setdefault("pipeline", False)
    e = Engine(lm, 64, prefill_chunk=16, max_step_tokens=48, **kw)
    r = e.submit(prompt, max_tokens, eos=(), **smp)
    e.run()
    return r.tokens


def test_engine_batched_equals_solo(lm):
    prompts = _prompts(1, [5, 17, 33, 40, 9])
    e = Engine(lm, 128, prefill_chunk=16, max_step_tokens=48, page_seed=7, selfcheck=True)
    reqs = [e.submit(p, 6, eos=()) for p in prompts[:2]]
    e.step()
    e.step()
    reqs += [e.submit(p, 6, eos=()) for p in prompts[2:]]
    e.run()
    assert e.pool.free_pages + sum(len(v) for v in e.store.entries.values()) == 128
    for r, p in zip(reqs, prompts):
        assert r.finish_reason == "length" and len(r.tokens) == 6
        assert r.tokens == _solo(lm, p, 6, prefix_store=False), r.rid


def test_engine_prompt_progresses_under_full_decode_load(lm):
    """A prompt admitted while the decode rows fill most of the step budget still advances one chunk
    per step (the step defers the decode rows that do not fit beside the chunk), and every
    generation stays the solo one."""
    prompts = _prompts(21, [5] * 8)
    e = Engine(lm, 256, prefill_chunk=16, max_step_tokens=20, pipeline=False, prefix_store=False)
    busy = [e.submit(p, 24, eos=()) for p in prompts]
    while any(r.state != "decode" for r in busy):
        e.step()
    late = e.submit(_prompts(22, [40])[0], 3, eos=())
    steps = 0
    while not late.tokens:
        e.step()
        steps += 1
        assert steps <= 4, "the prompt's 3 chunks (16 + 16 + 8) must run in consecutive steps"
    e.run()
    assert late.tokens == _solo(lm, _prompts(22, [40])[0], 3, prefix_store=False)
    for r, p in zip(busy, prompts):
        assert r.tokens == _solo(lm, p, 24, prefix_store=False), r.rid


def test_engine_sampled_requests_are_batch_independent(lm):
    """Sampled requests (temperature / top-p / top-k, seeded) generate the same tokens alone and
    batched with greedy and differently-set requests, pipelined or not; the same seed repeats its
    tokens and another seed differs; each token equals the oracle's draw given its step key's
    uniform (the draw of a whole generation, checked on the first token of every request)."""
    from jitengine_amd.sampler import Sampler
    prompts = _prompts(9, [12, 20, 7, 30])
    settings = [dict(temperature=0.8, top_p=0.9, top_k=40, seed=5), dict(), dict(temperature=1.2, top_p=1.0,
                top_k=0, seed=6), dict(temperature=0.8, top_p=0.9, top_k=40, seed=11)]
    e = Engine(lm, 128, prefill_chunk=16, max_step_tokens=48, page_seed=3)
    reqs = [e.submit(p, 7, eos=(), **kw) for p, kw in zip(prompts, settings)]
    e.run()
    for r, p, kw in zip(reqs, prompts, settings):
        assert len(r.tokens) == 7
        assert r.tokens == _solo(lm, p, 7, prefix_store=False, **kw), r.rid
        assert r.tokens == _solo(lm, p, 7, prefix_store=False, pipeline=True, **kw), r.rid
    other = _solo(lm, prompts[0], 7, prefix_store=False, temperature=0.8, top_p=0.9, top_k=40, seed=99)
    assert other != reqs[0].tokens
    # every draw of a solo run: the oracle's draw from the row's logits and its step key
    class Recording(Engine):
        def _draw(self, rows, h, steps):
            tok = super()._draw(rows, h, steps)
            self.seen.append((u16(self.lm.logits(h)), list(steps), tok.cpu().numpy()))
            return tok

    for p, kw in zip(prompts, settings):
        if not kw:
            continue
        e = Recording(lm, 64, prefill_chunk=16, max_step_tokens=48, pipeline=False)
        e.seen = []
        e.submit(p, 7, eos=(), **kw)
        e.run()
        smp = Sampler(kw["temperature"], kw["top_p"], kw["top_k"], kw["seed"], 7, lm.vocab)
        assert [st[0] for _, st, _ in e.seen] == list(range(7))
        for logits, st, tok in e.seen:
            u = oracle.threefry_uniform(smp.key(st[0])[None, :])
            assert oracle.sample_rows(logits, kw["temperature"], kw["top_p"], kw["top_k"], u)[0] == tok[0]


def test_engine_prefix_sharing_is_exact(lm):
    """A 40-token prefix restores at the chunk grid (24 tokens with 24-token chunks): one page shared
    whole, the half-used second one copied before the request writes into it, the stored pages never
    written; every generation equals the cold solo run."""
    base, = _prompts(2, [40])
    ext = _prompts(3, [10, 7])
    e = Engine(lm, 128, prefill_chunk=24, max_step_tokens=48)
    a = e.submit(base, 4, eos=())
    e.run()
    stored = list(e.store.entries[tuple(base)])
    before = [u16(p[stored]) for p in e.pool.pools]
    b = e.submit(base + ext[0], 5, eos=())
    c = e.submit(base + ext[1], 5, eos=())
    e.run()
    assert b.cached == 24 and c.cached == 24 and e.pool.copies >= 2
    assert all(np.array_equal(u16(p[stored]), x) for p, x in zip(e.pool.pools, before))  # never written
    assert a.tokens == _solo(lm, base, 4, prefix_store=False)
    assert b.tokens == _solo(lm, base + ext[0], 5, prefix_store=False)
    assert c.tokens == _solo(lm, base + ext[1], 5, prefix_store=False)


def test_engine_small_pool_defers_and_stops_on_eos(lm):
    prompts = _prompts(4, [30, 20])
    e = Engine(lm, 5, prefill_chunk=16, max_step_tokens=48, prefix_store=False)
    r0 = e.submit(prompts[0], 8, eos=())   # 3 pages
    r1 = e.submit(prompts[1], 30, eos=())  # 4 pages: waits for r0
    e.run()
    assert e.deferred > 0 and e.pool.free_pages == 5
    assert r0.tokens == _solo(lm, prompts[0], 8, prefix_store=False)
    assert r1.tokens == _solo(lm, prompts[1], 30, prefix_store=False)
    stop = r1.tokens[3]
    e2 = Engine(lm, 16, prefill_chunk=16, max_step_tokens=48)
    r = e2.submit(prompts[1], 30, eos=(stop,))
    e2.run()
    first = r1.tokens.index(stop)
    assert r.finish_reason == "stop" and r.tokens == r1.tokens[:first + 1]


def test_checkpoint_model_generates_on_gpu(tmp_path):
    cfg = config_dict(D=2048, H=32, Hkv=4, E=32, k=8, I=768, V=512, L=2)
    src = write_checkpoint(str(tmp_path), cfg, device=DEV)
    lm = checkpoint.load(str(tmp_path), DEV)
    mcfg = lm.cfg
    # the same model assembled by hand from the written tensors
    def q(n):
        return QLinear(src[n + ".weight"], src[n + ".scales"], src[n + ".biases"])

    def cat(ns, dim):
        return QLinear(*(torch.cat([src[n + "." + part] for n in ns], dim).contiguous()
                         for part in ("weight", "scales", "biases")))
    layers = []
    for i in range(2):
        p = f"model.layers.{i}."
        layers.append({"input_norm": src[p + "input_layernorm.weight"],
                       "qkv": cat([p + f"self_attn.{m}_proj" for m in "qkv"], 0),
                       "q_norm": src[p + "self_attn.q_norm.weight"], "k_norm": src[p + "self_attn.k_norm.weight"],
                       "o": q(p + "self_attn.o_proj"), "post_norm": src[p + "post_attention_layernorm.weight"],
                       "router": q(p + "mlp.gate"),
                       "gate_up": cat([p + f"mlp.switch_mlp.{m}_proj" for m in ("gate", "up")], 1),
                       "down": q(p + "mlp.switch_mlp.down_proj")})
    ref = CausalLM(Model(mcfg, layers), q("model.embed_tokens"), src["model.norm.weight"], q("lm_head"), 512)
    prompts = [[1, 2, 3, 4, 5, 6, 7], [100, 200, 300]]
    out = []
    for m in (lm, ref):
        e = Engine(m, 32, prefill_chunk=16, max_step_tokens=48)
        rs = [e.submit(p, 5, eos=()) for p in prompts]
        e.run()
        out.append([r.tokens for r in rs])
    assert out[0] == out[1]


def test_engine_decode_pipelining_is_exact(lm):
    """Issuing step n + 1 before reading step n (fed by its tokens on the device) draws the same
    tokens; an end-of-sequence token seen one step late only costs a discarded step."""
    prompts = _prompts(6, [12, 25, 7])
    out = {}
    for pipe in (False, True):
        e = Engine(lm, 64, prefill_chunk=16, max_step_tokens=48, pipeline=pipe)
        reqs = [e.submit(p, 9, eos=()) for p in prompts]
        e.run()
        out[pipe] = [r.tokens for r in reqs]
        if pipe:
            assert e.pipelined > 0
        assert e.pool.free_pages + sum(len(v) for v in e.store.entries.values()) == 64
    assert out[True] == out[False]
    stop = out[False][1][4]
    e = Engine(lm, 64, prefill_chunk=16, max_step_tokens=48, pipeline=True)
    reqs = [e.submit(p, 9, eos=(stop,)) for p in prompts]
    e.run()
    for r, full in zip(reqs, out[False]):
        want = full[:full.index(stop) + 1] if stop in full else full
        assert r.tokens == want and r.finish_reason == ("stop" if stop in full else "length")


def test_engine_page_aligned_edges(lm):
    """Page-aligned prompts and prefixes: a 32-token prompt retires after one token; a request
    restoring its 32-token prefix shares both pages and copies none; a 16-token prefix behind a
    17-token prompt restores one page."""
    p32, tail, p16 = _prompts(8, [32, 5, 16])
    e = Engine(lm, 32, prefill_chunk=16, max_step_tokens=48)
    a = e.submit(p32, 1, eos=())
    e.run()
    assert a.finish_reason == "length" and len(a.tokens) == 1
    assert a.tokens == _solo(lm, p32, 1, prefix_store=False)
    b = e.submit(p32 + tail, 3, eos=())
    e.run()
    assert b.cached == 32 and e.pool.copies == 0
    assert b.tokens == _solo(lm, p32 + tail, 3, prefix_store=False)
    c = e.submit(p16, 2, eos=())
    e.run()
    d = e.submit(p16 + [7], 4, eos=())
    e.run()
    assert d.cached == 16 and d.tokens == _solo(lm, p16 + [7], 4, prefix_store=False)


def test_engine_long_prompts_cold_warm_batched(lm):
    """Prompts over 192 tokens at the default prefill_chunk (512): their chunks take the segment
    GEMMs (the reference's prefill kernels), yet every generation is bit-identical cold (solo, no
    prefix store), warm (a stored 600-token prefix restores at the 512-token grid) and batched with
    another long prompt and decoding rows."""
    base, = _prompts(9, [600])
    tails = _prompts(10, [120, 30])
    A, B, X = base + tails[0], base + tails[1], base

    def solo(p, n):
        e = Engine(lm, 256, pipeline=False, prefix_store=False)
        r = e.submit(p, n, eos=())
        e.run()
        return r.tokens

    cold_a, cold_b = solo(A, 4), solo(B, 4)
    e = Engine(lm, 256)
    x = e.submit(X, 2, eos=())
    e.run()
    a = e.submit(A, 4, eos=())
    b = e.submit(B, 4, eos=())
    e.run()
    assert a.cached == 512 and b.cached == 512
    assert a.tokens == cold_a and b.tokens == cold_b
    e2 = Engine(lm, 256, prefix_store=False)
    rs = [e2.submit(p, n, eos=()) for p, n in ((A, 4), (B, 4), (X, 2))]
    short = e2.submit(_prompts(11, [9])[0], 6, eos=())
    e2.run()
    assert rs[0].tokens == cold_a and rs[1].tokens == cold_b and rs[2].tokens == x.tokens
    assert short.tokens == solo(_prompts(11, [9])[0], 6)


def test_decode_rows_independent_of_a_large_batch():
    """A decode step of 200 rows (past the 192-row switch of the dense projections) keeps every row's
    bits equal to the row decoded alone: the decode step never takes the segment GEMMs."""
    cfg = MoEConfig(layers=1, experts=32)
    from jitengine_amd.model import random_layer_weights

    model = Model(cfg, [random_layer_weights(cfg, seed=61, device=DEV)])
    B = 200
    rng = np.random.default_rng(62)
    lens = rng.integers(1, 60, B)
    npg = (lens + 1 + 15) // 16
    perm = rng.permutation(int(npg.sum()))
    table = np.zeros((B, int(npg.max())), np.int32)
    at = 0
    for b in range(B):
        table[b, :npg[b]] = perm[at:at + npg[b]]
        at += npg[b]
    pool = normal_bf16((int(npg.sum()), cfg.kv_heads, 2, 2048), seed=63)
    x = normal_bf16((B, 2048), seed=64)
    st = model.make_state(lens, torch.from_numpy(table).to(DEV))
    batched = u16(model.decode_step(bf16_tensor(x, DEV), [bf16_tensor(pool, DEV)], st))
    for b in (0, 77, 199):
        stb = model.make_state(lens[b:b + 1], torch.from_numpy(table[b:b + 1]).to(DEV))
        solo = u16(model.decode_step(bf16_tensor(x[b:b + 1], DEV), [bf16_tensor(pool, DEV)], stb))
        assert np.array_equal(solo[0], batched[b]), b


def test_engine_pipelining_overlaps_the_host(lm):
    """With pipelining the host reads step n's tokens (a pinned copy queued right behind step n) while
    step n + 1 runs, greedy and sampled rows alike (a step's host inputs -- positions, page table,
    attention plan, the sampler's keys -- go up through pinned memory without a host wait).  The
    generations must equal the synchronous loop's; the wall-clock times are printed, not asserted
    (a shared box's timing noise is no bug)."""
    import time

    prompts = _prompts(12, [20, 9, 33, 14])
    t, out = {}, {}
    for mode in ("greedy", "sampled"):
        kw = {} if mode == "greedy" else {"temperature": 0.8, "top_p": 0.9, "top_k": 40}
        for pipe in (False, True, False, True):
            e = Engine(lm, 128, prefill_chunk=16, max_step_tokens=48, pipeline=pipe, prefix_store=False)
            rs = [e.submit(p, 40, eos=(), seed=100 + i, **kw) for i, p in enumerate(prompts)]
            while any(r.state in ("queued", "prefill") for r in rs):
                e.step()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            e.run()
            torch.cuda.synchronize()
            t[mode, pipe] = time.perf_counter() - t0
            toks = [list(r.tokens) for r in rs]
            assert out.setdefault((mode,), toks) == toks, (mode, pipe)
        print(f"decode-only run, {mode}: synchronous {1e3 * t[mode, False]:.1f} ms, pipelined "
              f"{1e3 * t[mode, True]:.1f} ms", flush=True)
