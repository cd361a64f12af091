"""Benchmark of the ragged MoE decode step on one MI355X (prints ONE JSON line).

python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2] [--layers 48] [--no-graph] [--no-bs1]

config 2 (the default; BASELINE.json configs[2], the workload the metric is quoted on): ragged
continuous-batch decode of 32 sequences over the paged KV pool through 48 layers of the 4-bit
Qwen3-MoE-style block; a step decodes one token per sequence (value = tokens/s).  The step is
captured once as a HIP graph and replayed (--no-graph times eager launches).  The metric's bs=1
half -- config 4 on the same model -- is measured after it and reported in the line's "bs1" object
(--no-bs1 leaves it out).
config 4: single-sequence decode at 262,144 KV tokens through the 48
layers (value = tokens/s).
config 3: one mixed chunked-prefill + decode step of one block -- 4 x 512
prefill tokens (causal attention over their contexts) + 60 decode rows, the MoE on the segment GEMM
(value = rows/s; MFMA roofline of the dominant kernel).
config 1: one standalone quantized-MoE call -- 64 tokens, top-8 of 128
experts drawn from softmax of N(0,1) logits, gate/up [768 x 2048] and down [2048 x 768] per expert
(4-bit g64, N(0, 0.02) weights); a step = packing + gate||up/SwiGLU + down + combine.
Inputs are resident in HBM before timing; K steps are timed with HIP events after W warmups.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
SEED_BASE = 0x4A450000


def seed_for(config: int, layer: int = 0) -> int:
    return SEED_BASE + 16 * config + layer


def gen_stack(shape, seed, device):
    """N(0, 0.02) bf16 weights quantized to 4-bit g64, generated on the GPU in expert slices."""
    from jitengine_amd.quant import QLinear, random_quantized

    E = shape[0]
    parts = [random_quantized((min(16, E - e0), *shape[1:]), seed * 1000 + e0, device=device)
             for e0 in range(0, E, 16)]
    return QLinear(torch.cat([p.weight for p in parts]), torch.cat([p.scales for p in parts]),
                   torch.cat([p.biases for p in parts]))


HOT_OPS = ("paged_attention", "gate_up_swiglu", "down")  # the ops that move the expert and KV bytes


def hot_path_hbm(step_us: dict, alg_bytes: int) -> dict:
    """A kernel-level diagnostic, not the north-star measure: a decode step's quantized-expert and
    KV-pool bytes (alg_bytes) over the summed live time of only the ops that move them (step_us:
    microseconds per step by op), leaving out the rest of the step."""
    us = sum(step_us[n] for n in HOT_OPS if n in step_us)
    gbs = alg_bytes / (us * 1e-6) / 1e9 if us > 0 else None
    return {"label": "diagnostic: hot ops' live time only (not the whole step)", "ops": list(HOT_OPS),
            "alg_bytes": alg_bytes, "us_per_step": us, "GB_s": gbs, "frac": gbs / HBM_PEAK_GBS if gbs else None}


NORTH_STAR_FRAC = 0.6  # >= 60% of HBM peak on the combined expert + KV-pool traffic


def north_star(alg_bytes: int, ms_per_step: float, rows: int) -> dict:
    """The north-star measure as BASELINE defines it: the step's quantized-expert and KV-pool bytes
    over the whole step's time (every launch of the step included), as a fraction of the 8 TB/s peak,
    and the tokens/s a step meeting the 60% target would give on these bytes."""
    gbs = alg_bytes / (ms_per_step * 1e-3) / 1e9
    target_ms = alg_bytes / (NORTH_STAR_FRAC * HBM_PEAK_GBS * 1e9) * 1e3
    return {"alg_bytes": alg_bytes, "ms_per_step": ms_per_step, "GB_s": gbs, "frac": gbs / HBM_PEAK_GBS,
            "target_frac": NORTH_STAR_FRAC, "met": gbs / HBM_PEAK_GBS >= NORTH_STAR_FRAC,
            "tokens_s": rows / (ms_per_step * 1e-3), "tokens_s_at_target": rows / (target_ms * 1e-3)}


def time_ops(launches: dict, reps: int = 5) -> dict:
    """Mean device time per launch of each op, in microseconds.  `launches[name]` is a list of
    zero-argument callables, one launch each (for example the op on every layer's own weights and
    inputs).  Each list is captured once as a HIP graph and replayed `reps` times between two HIP
    events on the stream the launches run on, so host overhead between launches is not counted."""
    out = {}
    stream = torch.cuda.current_stream()
    for name, fns in launches.items():
        fns = list(fns) * max(1, -(-16 // len(fns)))  # >= 16 launches: a graph's own launch is amortised
        for f in fns:  # eager warm-up: the library is loaded and every allocation is cached
            f()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for f in fns:
                f()
        g.replay()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record(stream)
        for _ in range(reps):
            g.replay()
        e.record(stream)
        torch.cuda.synchronize()
        out[name] = 1e3 * s.elapsed_time(e) / (reps * len(fns))
        del g
    return out


def profile_traffic(name: str):
    """HBM bytes per launch of a kernel from a committed rocprofv3 summary (FETCH_SIZE and
    WRITE_SIZE, already scaled by the copy calibration): the line `traffic_bytes_per_launch: N`
    of profiles/<name>.txt, or None when there is no such summary."""
    path = os.path.join(ROOT, "profiles", name + ".txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def cpu_threads() -> int:
    return len(os.sched_getaffinity(0))


def bench_config1(steps: int, warmup: int, dev: str) -> dict:
    import oracle
    from jitengine_amd import ops

    B, E, D, I, k = 64, 128, 2048, 768, 8
    seed = seed_for(1)
    rng = np.random.default_rng(seed)
    gu_mlx = gen_stack((E, 2 * I, D), seed + 1, dev)
    dn_mlx = gen_stack((E, D, I), seed + 2, dev)
    gu, dn = ops.prepack(gu_mlx), ops.prepack(dn_mlx)  # one-time load-side reorder, untimed
    logits = oracle.f32_to_bf16(rng.standard_normal((B, E)).astype(np.float32))
    x_np = oracle.f32_to_bf16(rng.standard_normal((B, D)).astype(np.float32))
    to_dev = lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(dev)  # noqa: E731
    x = to_dev(x_np)
    inds, scores = ops.router_topk(to_dev(logits), k, True)
    torch.cuda.synchronize()

    def step():
        pk = ops.moe_pack(inds, E)
        h = ops.expert_gate_up(x, gu, pk)
        r = ops.expert_down(h, dn, pk)
        return ops.moe_combine(r, pk, scores)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        y = step()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps

    # per-op device time, each op replayed alone on the same inputs
    pk = ops.moe_pack(inds, E)
    h = ops.expert_gate_up(x, gu, pk)
    r = ops.expert_down(h, dn, pk)
    kus = time_ops({"moe_pack": [lambda: ops.moe_pack(inds, E)],
                    "gate_up_swiglu": [lambda: ops.expert_gate_up(x, gu, pk)],
                    "down": [lambda: ops.expert_down(h, dn, pk)],
                    "combine": [lambda: ops.moe_combine(r, pk, scores)]}, reps=max(steps, 10))

    flat = inds.cpu().numpy().reshape(-1)
    U = int(np.unique(flat).size)
    P = B * k
    gu_bytes_e = 2 * I * D // 2 + 2 * (2 * I) * (D // 64) * 2
    dn_bytes_e = D * I // 2 + 2 * D * (I // 64) * 2
    alg_gate_up = U * gu_bytes_e + B * D * 2 + P * I * 2
    alg_down = U * dn_bytes_e + P * I * 2 + P * D * 2
    # the expert step's algorithmic bytes: each distinct expert's weights once, x read, h written and
    # read back, the combined rows written
    alg_step = U * (gu_bytes_e + dn_bytes_e) + B * D * 2 + 2 * P * I * 2 + B * D * 2
    dom = "gate_up_swiglu"
    achieved = alg_gate_up / (kus[dom] * 1e-6) / 1e9

    # CPU baseline: the oracle's expert chain over the same bytes, on a bounded token sample
    nb = 16
    ind_np = flat.reshape(B, k)[:nb].astype(np.uint32)
    sc_np = scores[:nb].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)

    def host(q):
        return (q.weight.cpu().numpy().view(np.uint32), q.scales.view(torch.int16).cpu().numpy().view(np.uint16),
                q.biases.view(torch.int16).cpu().numpy().view(np.uint16))

    gu_h, dn_h = host(gu_mlx), host(dn_mlx)
    oracle.set_num_threads(cpu_threads())
    oracle.moe_experts(x_np[:nb], ind_np, sc_np, gu_h, dn_h, E)  # warm-up
    times = []
    for _ in range(5):
        c0 = time.perf_counter()
        oracle.moe_experts(x_np[:nb], ind_np, sc_np, gu_h, dn_h, E)
        times.append(time.perf_counter() - c0)
    cpu_tps = nb / float(np.median(times))

    return {
        "metric": "decode tok/s (bs=1, ragged bs=32) + achieved HBM GB/s as % of MI355X peak",
        "value": B / (ms * 1e-3),
        "unit": "tokens/s",
        "ms_per_step": ms,
        "dtype": "bf16",
        "arithmetic": "bf16 activations, 4-bit g64 weights, fp32 accumulate",
        "config": {"workload": "config1: standalone quantized MoE call, 64 tokens x top-8 of 128 experts, "
                               "gate/up 768x2048, down 2048x768, 4-bit g64",
                   "tokens": B, "experts": E, "top_k": k, "distinct_experts": U},
        "step_hbm": {"alg_bytes": alg_step, "GB_s": alg_step / (ms * 1e-3) / 1e9,
                     "frac": alg_step / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS},
        "kernels_us": kus,
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "alg_bytes_per_launch": alg_gate_up, "traffic": None},
        "cpu_baseline": {"value": cpu_tps, "unit": "tokens/s", "cores": oracle.num_threads(), "kind": "port",
                         "sample": f"oracle expert chain (pack, gate_up, down, combine; float64 dots) on {nb} of "
                                   f"the {B} tokens, median of 5 after a warm-up"},
        "_y": y,
    }


def bench_config3(steps: int, warmup: int, dev: str) -> dict:
    """one mixed chunked-prefill + decode step of one decoder block -- 4
    prefill chunks of 512 tokens after prior contexts U{0..8192} plus 60 decode sequences with
    lengths log-uniform in [256, 16384], 2,108 rows in all (DecoderLayer.mixed: qkv, norms and
    RoPE with the KV append of every row, causal prefill attention and split-K decode attention,
    o_proj, router, top-k, packing, the segment GEMM experts (~132 pairs per expert), combine).
    value = rows / step time; the roofline is the MFMA one of the dominant kernel."""
    import oracle
    from jitengine_amd import ops
    from jitengine_amd.model import DecoderLayer, MoEConfig, make_mixed_state, random_layer_weights, rope_inv_freq

    cfg = MoEConfig(layers=1)
    seed = seed_for(3)
    rng = np.random.default_rng(seed)
    ctx = rng.integers(0, 8193, 4)
    dec_len = np.round(np.exp(rng.uniform(np.log(256), np.log(16384), 60))).astype(np.int32)
    chunks = [(i, int(c), 512) for i, c in enumerate(ctx)]
    keys = [int(c) + 512 for c in ctx] + [int(L) + 1 for L in dec_len]  # decode row b writes position L_b
    npg = [-(-n // 16) for n in keys]
    perm = rng.permutation(sum(npg))
    table = np.zeros((len(keys), max(npg)), np.int32)
    at = 0
    for i, n in enumerate(npg):
        table[i, :n] = perm[at:at + n]
        at += n
    w = random_layer_weights(cfg, seed * 100, dev)
    layer = DecoderLayer(cfg, w)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed + 7)
    pool = torch.randn((sum(npg), cfg.kv_heads, 2, 16 * 128), generator=gen, device=dev, dtype=torch.bfloat16)
    ms = make_mixed_state(cfg, chunks, table[:4], dec_len, table[4:], dev)
    T = ms.P + len(dec_len)
    x = torch.randn((T, cfg.hidden), generator=gen, device=dev, dtype=torch.bfloat16)
    dbg = {}
    layer.mixed(x, pool, ms, debug=dbg)
    torch.cuda.synchronize()

    def step():
        return layer.mixed(x, pool, ms)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = step()
    g.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    ms_step = t0.elapsed_time(t1) / steps
    del g

    # per-op device time on the step's own intermediates
    scale = cfg.head_dim ** -0.5
    moe, pk = layer.moe, dbg["pk"]
    q = dbg["q"]
    kus = time_ops({
        "rmsnorm": [lambda: ops.rmsnorm(x, layer.input_norm, cfg.eps)],
        "qkv_proj": [lambda: ops.qmm(dbg["xn"], layer.qkv)],
        "qk_norm_rope_append": [lambda: ops.qk_norm_rope_append(
            dbg["qkv"], cfg.heads, cfg.kv_heads, layer.q_norm, layer.k_norm, cfg.eps, layer.inv_freq, ms.pos_rows,
            ms.table_rows, pool)],
        "prefill_attention": [lambda: ops.paged_prefill_attention(q[:ms.P], pool, ms.seq_table, ms.prefill, scale)],
        "decode_attention": [lambda: ops.paged_decode_attention(q[ms.P:], pool, ms.dec_table, ms.decode, scale,
                                                                ms.workspace)],
        "o_proj": [lambda: ops.qmm(dbg["attn"].view(T, -1), layer.o)],
        "add_rmsnorm": [lambda: ops.rmsnorm(dbg["o"], layer.post_norm, cfg.eps, resid=x, return_sum=True)],
        "router_proj": [lambda: ops.qmm(dbg["hn"], moe.router)],
        "router_topk": [lambda: ops.router_topk(dbg["logits"], cfg.top_k, cfg.norm_topk)],
        "moe_pack": [lambda: ops.moe_pack(dbg["inds"], cfg.experts)],
        "gate_up_swiglu_seg": [lambda: ops.expert_gate_up(dbg["hn"], moe.gate_up, pk, seg=True)],
        "down_seg": [lambda: ops.expert_down(dbg["hh"], moe.down, pk, seg=True)],
        "combine": [lambda: ops.moe_combine(dbg["r"], pk, dbg["scores"], dbg["h"])],
    }, reps=max(steps, 5))
    D, I, E, H = cfg.hidden, cfg.inter, cfg.experts, cfg.heads
    P = T * cfg.top_k
    flops = {
        "gate_up_swiglu_seg": 2.0 * P * 2 * I * D,
        "down_seg": 2.0 * P * D * I,
        "prefill_attention": float(sum(4.0 * H * 128 * (c + t + 1) for _, c, n in chunks for t in range(n))),
        "qkv_proj": 2.0 * T * cfg.qkv_rows * D,
        "o_proj": 2.0 * T * D * H * 128,
    }
    dom = max((k for k in kus if k in flops), key=kus.get)
    achieved = flops[dom] / (kus[dom] * 1e-6) / 1e12
    step_flops = sum(flops.values()) + 2.0 * T * E * D + float(sum(4.0 * H * 128 * (L + 1) for L in dec_len))

    # CPU baseline: the oracle's block on a self-contained row sample -- the first 16 tokens of
    # chunk 0 (their keys: chunk 0's context and themselves) and 16 decode rows
    u16 = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)  # noqa: E731

    def host_q(lin):
        return (lin.weight.cpu().numpy().view(np.uint32), u16(lin.scales), u16(lin.biases))

    lw = {k: (host_q(v) if k in ("qkv", "o", "router", "gate_up", "down") else u16(v)) for k, v in w.items()}
    nb = 16
    sel = np.r_[0:nb, ms.P:ms.P + nb]
    xs = u16(x)[sel]
    pos_s = np.concatenate([np.arange(ctx[0], ctx[0] + nb), dec_len[:nb]]).astype(np.int32)
    rows_s = np.concatenate([np.repeat(table[:1], nb, 0), table[4:4 + nb]]).astype(np.int32)
    pool_h = u16(pool)
    inv_freq = rope_inv_freq(cfg.rope_theta, 128)
    oracle.set_num_threads(cpu_threads())

    def cpu_sample():
        ph = pool_h.copy()
        xn, _ = oracle.rmsnorm(xs, lw["input_norm"], cfg.eps)
        _, qkv = oracle.qmm(xn, *lw["qkv"])
        qh = oracle.qk_norm_rope_append(qkv, H, cfg.kv_heads, lw["q_norm"], lw["k_norm"], cfg.eps, inv_freq, pos_s,
                                        ph, rows_s)
        a_pre = oracle.paged_prefill_attn(qh[:nb], ph, table[:1], [(0, int(ctx[0]), nb)], scale)
        a_dec = oracle.paged_decode_attn(qh[nb:], ph, table[4:4 + nb], dec_len[:nb] + 1, scale)
        _, o = oracle.qmm(np.concatenate([a_pre, a_dec]).reshape(2 * nb, -1), *lw["o"])
        hn, h = oracle.rmsnorm(o, lw["post_norm"], cfg.eps, resid=xs)
        _, logits = oracle.qmm(hn, *lw["router"])
        wi, ws, _ = oracle.router_topk(logits, cfg.top_k, True)
        opk = oracle.moe_pack(wi, E)
        hh = oracle.moe_gate_up(hn, wi, opk, *lw["gate_up"], bf16w=True)
        rr = oracle.moe_down(hh, wi, opk, *lw["down"], bf16w=True)
        return oracle.moe_combine(rr, opk["inv"], ws)

    cpu_sample()
    times = []
    for _ in range(5):
        c0 = time.perf_counter()
        cpu_sample()
        times.append(time.perf_counter() - c0)
    cpu_tps = 2 * nb / float(np.median(times))
    U = int(torch.unique(dbg["inds"]).numel())
    return {
        "metric": "decode tok/s (bs=1, ragged bs=32) + achieved HBM GB/s as % of MI355X peak",
        "value": T / (ms_step * 1e-3),
        "unit": "tokens/s",
        "ms_per_step": ms_step,
        "dtype": "bf16",
        "arithmetic": "bf16 activations, 4-bit g64 weights (bf16-dequantized on the segment GEMM), fp32 accumulate",
        "config": {"workload": "config3: one mixed chunked-prefill + decode step of one block -- 4 x 512 prefill "
                               "tokens after contexts U{0..8192} + 60 decode rows (lengths log-uniform [256, 16384])",
                   "rows": T, "prefill_ctx": [int(c) for c in ctx], "decode_kv_tokens": int(dec_len.sum()) + 60,
                   "pairs": P, "experts": E, "distinct_experts": U, "max_pairs_per_expert": int(pk.meta[1]),
                   "hip_graph": True},
        "step_tflops": step_flops / (ms_step * 1e-3) / 1e12,
        "op_us": kus,
        "op_us_sum_per_step": sum(kus.values()),
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": achieved, "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": achieved / 2500.0, "flops_per_launch": flops[dom],
                     "traffic": profile_traffic(f"{dom}_config3")},
        "cpu_baseline": {"value": cpu_tps, "unit": "tokens/s", "cores": oracle.num_threads(), "kind": "port",
                         "sample": f"the oracle's block (dense, norms, RoPE + append, causal prefill and decode "
                                   f"attention, router, segment-GEMM experts) on {2 * nb} of the {T} rows: the first "
                                   f"{nb} tokens of chunk 0 and {nb} decode rows, median of 5 after a warm-up"},
        "_y": y,
    }


CONFIG4_KEYS = 262144  # one sequence decoding at 262,144 KV tokens
CONFIG0_KEYS = 4096    # one block, batch 1, 4,096 context tokens in one page run


def decode_model(cfg, seed: int, dev: str):
    """The 48-layer model of a decode config: layer l's weights seeded with seed * 100 + l.  Also
    returns layer 0's weights (the CPU baseline's layer)."""
    from jitengine_amd.model import DecoderLayer, Model, random_layer_weights

    layers, w0 = [], None
    for l in range(cfg.layers):
        w = random_layer_weights(cfg, seed * 100 + l, dev)
        layers.append(DecoderLayer(cfg, w))
        if l == 0:
            w0 = w
        del w
    model = Model.__new__(Model)
    model.cfg, model.layers = cfg, layers
    return model, w0


def bench_decode(config: int, steps: int, warmup: int, dev: str, graph: bool, n_layers: int = 48,
                 model=None, cpu: bool = True) -> dict:
    """A decode step of the 4-bit Qwen3-MoE-style model over the paged KV pool (16-token pages in a
    random permutation of the pool), one token per sequence through every layer (each row writes
    position L_b and attends to L_b + 1 keys).
    config 2: 32 sequences with lengths log-uniform in [128, 32768], 48 layers
    with independent seeded weights.
    config 4: one sequence at 262,144 KV tokens (the step's own token is the
    262,144th key), 48 layers; `model` may pass in config 2's weights, which are as random as its own."""
    import oracle
    from jitengine_amd import ops
    from jitengine_amd.model import MoEConfig, make_step_state, rope_inv_freq

    seed = seed_for(config)
    rng = np.random.default_rng(seed)
    if config == 2:
        B = 32
        lens = np.round(np.exp(rng.uniform(np.log(128), np.log(32768), B))).astype(np.int32)
    elif config == 0:
        B = 1
        lens = np.array([CONFIG0_KEYS], np.int32)
        n_layers = 1
    else:
        B = 1
        lens = np.array([CONFIG4_KEYS - 1], np.int32)
    npg = (lens + 1 + 15) // 16
    num_pages = int(npg.sum())
    # config 0's context is one contiguous page run (pages 0.. in order); the others are permuted
    perm = np.arange(num_pages) if config == 0 else rng.permutation(num_pages)
    table = np.zeros((B, int(npg.max())), np.int32)
    at = 0
    for b in range(B):
        table[b, :npg[b]] = perm[at:at + npg[b]]
        at += npg[b]
    w0 = None
    if model is None:
        model, w0 = decode_model(MoEConfig(layers=n_layers), seed, dev)
    cfg = model.cfg
    n_layers = cfg.layers
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed + 7)
    pools = [torch.randn((num_pages, cfg.kv_heads, 2, 16 * 128), generator=gen, device=dev, dtype=torch.bfloat16)
             for _ in range(n_layers)]
    x = torch.randn((B, cfg.hidden), generator=gen, device=dev, dtype=torch.bfloat16)
    table_d = torch.from_numpy(table).to(dev)
    st = make_step_state(cfg, lens, table_d)
    torch.cuda.synchronize()

    # one eager step keeps every layer's intermediates: the distinct experts per layer (for the
    # algorithmic byte count) and the inputs of the per-op timing below
    dbg = []
    xx = x
    for l, layer in enumerate(model.layers):
        d = {}
        xx = layer.step(xx, pools[l], st, debug=d)
        dbg.append(d)
    U = [int(torch.unique(d["inds"]).numel()) for d in dbg]
    torch.cuda.synchronize()

    def step():
        return model.decode_step(x, pools, st)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        y = step()
    t1.record()
    torch.cuda.synchronize()
    ms_eager = t0.elapsed_time(t1) / steps
    ms = ms_eager
    if graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            yg = step()
        for _ in range(max(warmup, 1)):
            g.replay()
        torch.cuda.synchronize()
        t0.record()
        for _ in range(steps):
            g.replay()
        t1.record()
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / steps
        y = yg
        del g

    # per-op device time: each op over the 48 layers (each layer's own weights, pool and
    # inputs from the eager step above), replayed alone
    L_ = model.layers

    # the launches of one step, op by op: layer l's closing combine also norms layer l + 1's input,
    # so the stand-alone input norm runs for layer 0 only and the plain combine for the last layer
    last = n_layers - 1
    step_layers = {"rmsnorm": [0], "combine_rmsnorm": list(range(last)), "combine": [last]}
    per_layer = {
        "rmsnorm": lambda l: ops.rmsnorm(dbg[l]["x"], L_[l].input_norm, cfg.eps),
        "qkv_proj": lambda l: ops.qmm(dbg[l]["xn"], L_[l].qkv),
        # (the step's attention launch norms, rotates and appends the token itself: the fused entry; its
        # append rewrites the same slot with the same bits)
        "paged_attention": lambda l: ops.paged_decode_attention_qkv(
            dbg[l]["qkv"], cfg.heads, cfg.kv_heads, L_[l].q_norm, L_[l].k_norm, cfg.eps, L_[l].inv_freq, pools[l],
            st.page_table, st.plan, cfg.head_dim ** -0.5, st.workspace),
        "o_proj": lambda l: ops.qmm(dbg[l]["attn"].view(B, -1), L_[l].o),
        "add_rmsnorm": lambda l: ops.rmsnorm(dbg[l]["o"], L_[l].post_norm, cfg.eps, resid=dbg[l]["x"],
                                             return_sum=True),
        "router_proj": lambda l: ops.qmm(dbg[l]["hn"], L_[l].moe.router),
        "router_topk": lambda l: ops.router_topk(dbg[l]["logits"], cfg.top_k, cfg.norm_topk),
        "moe_pack": lambda l: ops.moe_pack(dbg[l]["inds"], cfg.experts),
        "route_pack": lambda l: ops.route_pack(dbg[l]["logits"], cfg.top_k, cfg.norm_topk),
        "gate_up_swiglu": lambda l: ops.expert_gate_up(dbg[l]["hn"], L_[l].moe.gate_up, dbg[l]["pk"]),
        "down": lambda l: ops.expert_down(dbg[l]["hh"], L_[l].moe.down, dbg[l]["pk"]),
        "combine_rmsnorm": lambda l: ops.moe_combine_rmsnorm(dbg[l]["r"], dbg[l]["pk"], dbg[l]["scores"],
                                                             dbg[l]["h"], L_[l + 1].input_norm, cfg.eps),
        "combine": lambda l: ops.moe_combine(dbg[l]["r"], dbg[l]["pk"], dbg[l]["scores"], dbg[l]["h"]),
    }
    # a step of at most ROUTE_PACK_MAX_ROWS rows routes and packs in one launch, a larger one in two
    for name in (("router_topk", "moe_pack") if B <= ops.ROUTE_PACK_MAX_ROWS else ("route_pack",)):
        del per_layer[name]
    if B == 1:  # one token routes itself inside the gate||up launch (DecoderLayer.run's choice)
        del per_layer["route_pack"]
        per_layer["gate_up_swiglu"] = lambda l: ops.route_gate_up(dbg[l]["hn"], dbg[l]["logits"], L_[l].moe.gate_up,
                                                                  cfg.top_k, cfg.norm_topk)[3]
        # ... layer l's combine and layer l + 1's input norm run inside that layer's qkv launch, and the
        # post-attention add + norm inside the router launch (Model.decode_step, DecoderLayer.run)
        # (the geometry's layers all take the prologues or none does)
        if all(ops.row_prologue_fits(m, cfg.hidden) for lay in L_ for m in (lay.qkv, lay.moe.router)):
            step_layers.update(qkv_proj=[0], combine_qkv=list(range(last)), combine_rmsnorm=[])
            del per_layer["add_rmsnorm"]
            per_layer["router_proj"] = lambda l: ops.qmm_add_rmsnorm(dbg[l]["o"], dbg[l]["x"], L_[l].post_norm,
                                                                     cfg.eps, L_[l].moe.router)[0]
            per_layer["combine_qkv"] = lambda l: ops.qmm_combine_rmsnorm(dbg[l]["r"], dbg[l]["pk"], dbg[l]["scores"],
                                                                         dbg[l]["h"], L_[l + 1].input_norm, cfg.eps,
                                                                         L_[l + 1].qkv)[1]
    launches = {name: step_layers.get(name, list(range(n_layers))) for name in per_layer}
    launches = {name: ls for name, ls in launches.items() if ls}  # (a one-layer step has no combine_rmsnorm)
    per_layer = {name: f for name, f in per_layer.items() if name in launches}
    kus = time_ops({name: [(lambda f=f, l=l: f(l)) for l in launches[name]] for name, f in per_layer.items()},
                   reps=3)
    step_us = {name: kus[name] * len(launches[name]) for name in kus}

    dense = cfg.qkv_rows * cfg.hidden // 2 * 9 // 8 + cfg.hidden * cfg.heads * 128 // 2 * 9 // 8 \
        + cfg.experts * cfg.hidden // 2 * 9 // 8
    per_expert = 2654208  # gate||up 1,769,472 + down 884,736 (weights, scales, biases)
    kv = int((lens.astype(np.int64) + 1).sum()) * 2 * cfg.kv_heads * 128 * 2  # 2,048 B per key
    alg_step = n_layers * (dense + kv) + sum(U) * per_expert
    # the dominant op by device time, and its algorithmic bytes per launch (the same for every layer
    # for attention; the mean over layers for the experts)
    alg_op = {"paged_attention": kv, "gate_up_swiglu": float(np.mean(U)) * 1769472,
              "down": float(np.mean(U)) * 884736, "qkv_proj": cfg.qkv_rows * cfg.hidden // 2 * 9 // 8,
              "o_proj": cfg.hidden * cfg.heads * 128 // 2 * 9 // 8, "router_proj": cfg.experts * cfg.hidden // 2 * 9 // 8}
    dom = max(kus, key=kus.get)
    achieved = alg_op[dom] / (kus[dom] * 1e-6) / 1e9 if dom in alg_op else None

    traffic = profile_traffic(f"{dom}_config{config}")
    if config == 2:
        workload = (f"config2: ragged 32-sequence decode, {n_layers} layers of the Qwen3-MoE-style 4-bit block, "
                    "paged bf16 KV (16-token pages, permuted), lens log-uniform [128, 32768]")
    elif config == 0:
        workload = ("config0: one Qwen3-MoE-style 4-bit block, batch-1 decode at position 4096 over a 4,096-token "
                    "bf16 context in one contiguous page run (pages 0..256 in order)")
    else:
        workload = (f"config4: single-sequence decode at {CONFIG4_KEYS} KV tokens, {n_layers} layers of the "
                    "Qwen3-MoE-style 4-bit block, paged bf16 KV (16-token pages, permuted), split-K attention")
    res = {
        "metric": "decode tok/s (bs=1, ragged bs=32) + achieved HBM GB/s as % of MI355X peak",
        "value": B / (ms * 1e-3),
        "unit": "tokens/s",
        "ms_per_step": ms,
        "dtype": "bf16",
        "config": {"workload": workload,
                   "weights": "MLX 4-bit affine g64 (bf16 scale/bias), dequantized in registers; fp32 accumulate",
                   "sequences": B, "layers": n_layers, "kv_tokens": int(lens.sum()), "lens_min": int(lens.min()),
                   "lens_max": int(lens.max()), "distinct_experts_mean": float(np.mean(U)),
                   "hip_graph": bool(graph), "ms_per_step_eager": ms_eager},
        "step_hbm": {"alg_bytes": alg_step, "GB_s": alg_step / (ms * 1e-3) / 1e9,
                     "frac": alg_step / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                     "split": {"experts": sum(U) * per_expert, "kv": n_layers * kv, "dense": n_layers * dense}},
        # the target's own measure: the quantized-expert and KV-pool bytes of a step over the time of
        # the ops that move them (attention with its merge, gate||up, down), each timed live
        "north_star": north_star(sum(U) * per_expert + n_layers * kv, ms, B),
        "hot_path_hbm": hot_path_hbm(step_us, sum(U) * per_expert + n_layers * kv),
        "op_us": kus,
        "op_us_per_step": step_us,
        "op_us_sum_per_step": sum(step_us.values()),
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": (achieved / HBM_PEAK_GBS) if achieved else None, "traffic": traffic,
                     "alg_bytes_per_launch": alg_op.get(dom), "launch_us": kus[dom]},
        "_y": y,
        "_model": model,
        "_pools": pools,
    }
    if not cpu or w0 is None:
        return res

    # CPU baseline: the oracle's decoder layer (layer 0's weights and pool) on all rows, median of
    # 5 after a warm-up, scaled to the 48 layers of a step
    def host_q(lin):
        return (lin.weight.cpu().numpy().view(np.uint32), lin.scales.view(torch.int16).cpu().numpy().view(np.uint16),
                lin.biases.view(torch.int16).cpu().numpy().view(np.uint16))
    u16 = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)  # noqa: E731
    lw = {"input_norm": u16(w0["input_norm"]), "qkv": host_q(w0["qkv"]), "q_norm": u16(w0["q_norm"]),
          "k_norm": u16(w0["k_norm"]), "o": host_q(w0["o"]), "post_norm": u16(w0["post_norm"]),
          "router": host_q(w0["router"]), "gate_up": host_q(w0["gate_up"]), "down": host_q(w0["down"])}
    pool_h = u16(pools[0])
    ocfg = {"heads": cfg.heads, "kv_heads": cfg.kv_heads, "experts": cfg.experts, "top_k": cfg.top_k,
            "eps": cfg.eps, "inv_freq": rope_inv_freq(cfg.rope_theta, 128)}
    xs = u16(x)
    oracle.set_num_threads(cpu_threads())
    times = []
    for i in range(6):
        ph = pool_h.copy()
        c0 = time.perf_counter()
        oracle.decoder_layer_mlx_f32(xs, lw, ph, table, lens, ocfg)
        if i:
            times.append(time.perf_counter() - c0)
    cpu_tps = B / (float(np.median(times)) * n_layers)

    res["cpu_baseline"] = {
        "value": cpu_tps, "unit": "tokens/s", "cores": cpu_threads(), "kind": "port", "label": "restatement",
        "sample": f"the reference's MLX op chain restated in its own fp32 arithmetic (oracle.decoder_layer_mlx_f32: "
                  f"qmv per-lane order, sdpa_vector / two-pass attention, C + OpenMP) on all {B} rows with layer 0's "
                  f"weights and KV ({int(lens.sum())} keys), median of 5 after a warm-up, x {n_layers} layers"}
    return res


def bench_sampler(dev: str) -> int:
    """The sampler's kernels (csrc/sampler.hip) on the reference's vocabulary (248,320) for 1 and
    32 rows of N(0, 3) logits: log-probabilities, the greedy draw, and draws under the settings of
    the reference's sampler checks (Q36/sampler.py:575).  Log-probabilities and greedy split each
    row over slices, one workgroup a slice, and read it three times; a draw's workgroup reads its
    row about six times from L2 (max, log-sum-exp, histogram, weights, the draw's walk).  The
    algorithmic bytes are the row's 2 V once."""
    from jitengine_amd import ops

    V = 248320
    out = {"vocab": V, "us": {}, "row_GB_s": {}}
    for B in (1, 32):
        gen = torch.Generator(device=dev)
        gen.manual_seed(1000 + B)
        x = (torch.randn((B, V), generator=gen, device=dev) * 3).to(torch.bfloat16)
        u = torch.rand(B, generator=gen, device=dev)
        launches = {"logprobs": [lambda: ops.logprobs_rows(x)], "greedy": [lambda: ops.argmax_rows(x)]}
        for T, p, k in ((0.7, 0.95, 40), (1.0, 0.9, 20), (1.0, 0.95, 0), (1.0, 1.0, 0)):
            launches[f"T{T}_p{p}_k{k}"] = [lambda T=T, p=p, k=k: ops.sample_rows(x, T, p, k, u)]
        us = time_ops(launches, reps=20)
        out["us"][f"B{B}"] = {k: round(v, 2) for k, v in us.items()}
        out["row_GB_s"][f"B{B}"] = {k: round(B * V * 2 / (v * 1e-6) / 1e9, 1) for k, v in us.items()}
    print(json.dumps({"sampler": out}), flush=True)
    return 0


def copy_calibration(dev: str) -> int:
    """A plain device copy of 256 MiB (torch's copy kernel), run 5 times: the known-size transfer
    the FETCH_SIZE / WRITE_SIZE counters are scaled by."""
    n = 64 * 1024 * 1024
    src = torch.empty(n, dtype=torch.float32, device=dev).uniform_()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(5):
        dst.copy_(src)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / 5
    print(json.dumps({"copy_bytes_read": n * 4, "copy_bytes_written": n * 4, "ms": ms,
                      "GB_s_read_plus_write": 2 * n * 4 / (ms * 1e-3) / 1e9}), flush=True)
    return 0


def probe(dev: str, parts=("read", "launch", "barrier")) -> int:
    """The yardsticks the kernels are rated against, measured on this GPU (csrc/probe.hip):
    the HBM streaming-read ceiling (4 GiB read whole, grid-stride or one contiguous run per
    workgroup, plain or nontemporal loads; and 196 MB reads, one launch each, rotating through 48
    distinct windows as the expert kernels' layers do), the device time of an empty launch inside
    a HIP graph, and the cost of a grid-wide barrier inside one cooperative launch."""
    import ctypes

    from jitengine_amd import build as hip_build

    lib = ctypes.CDLL(hip_build.PROBE_LIB)
    P, I, LL = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong
    lib.probe_read.argtypes = [P, LL, I, I, P, P]
    lib.probe_lds_ring.argtypes = [P, LL, I, I, P, P]
    lib.probe_empty.argtypes = [P]
    lib.probe_paged.argtypes = [P, P, I, I, I, P, P]
    lib.probe_barrier.argtypes = [I, I, I, P, P, I, P, P]
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)

    def timed(fn, reps):
        fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record(stream)
        for _ in range(reps):
            fn()
        e.record(stream)
        torch.cuda.synchronize()
        return s.elapsed_time(e) / reps  # ms

    out = {"read": {}, "launch": {}, "barrier": {}, "lds_ring": {}, "gemv": {}}
    if "lds" in parts:
        # streaming through an LDS ring by direct loads, one persistent workgroup per CU, over 48
        # rotating 196 MB windows (the expert weights' volume)
        win, n_win = 196 << 20, 8
        buf = torch.empty(win * n_win // 4, dtype=torch.int32, device=dev).random_()
        sink = torch.empty(1 << 16, dtype=torch.int32, device=dev)
        cus = torch.cuda.get_device_properties(0).multi_processor_count
        shapes = {0: "4x9KB_4stages", 1: "3x9KB_5stages", 2: "8x4KB_4stages", 3: "4x4KB_8stages", 4: "4x2KB_16stages"}
        for shape, name in shapes.items():
            def rot(shape=shape):
                for w in range(n_win):
                    lib.probe_lds_ring(ctypes.c_void_p(buf.data_ptr() + w * win), win, shape, cus,
                                       ctypes.c_void_p(sink.data_ptr()), sp)
            ms = timed(rot, 5)
            out["lds_ring"][f"{name}_{cus}wg"] = round(n_win * win / (ms * 1e-3) / 1e9, 1)
        del buf
    if "read" in parts:
        big = 4 << 30
        buf = torch.empty(big // 4, dtype=torch.int32, device=dev).random_()
        sink = torch.empty(1 << 16, dtype=torch.int32, device=dev)
        names = {0: "grid_stride", 1: "grid_stride_nt", 2: "contiguous_runs", 3: "contiguous_runs_nt"}
        for mode in range(4):
            for blocks in (1024, 4096, 16384):
                ms = timed(lambda: lib.probe_read(ctypes.c_void_p(buf.data_ptr()), big, mode, blocks,
                                                  ctypes.c_void_p(sink.data_ptr()), sp), 5)
                out["read"][f"{names[mode]}_{blocks}wg_4GiB"] = round(big / (ms * 1e-3) / 1e9, 1)
        win = 196 * 1000 * 1000 // 16 * 16
        n_win = min(48, big // win)
        for mode in (2, 3):
            def rot(mode=mode):
                for w in range(n_win):
                    lib.probe_read(ctypes.c_void_p(buf.data_ptr() + w * win), win, mode, 5376,
                                   ctypes.c_void_p(sink.data_ptr()), sp)
            ms = timed(rot, 3)
            out["read"][f"{names[mode]}_5376wg_196MB_per_launch"] = round(n_win * win / (ms * 1e-3) / 1e9, 1)
        # the attention access shape: 8 KB blocks at random pages, 2048 waves of 64-block runs
        nblk = big // 8192
        waves, run = 2048, 64
        perm = torch.randperm(nblk, device=dev)[:waves * run].to(torch.int32).contiguous()
        for mode, name in ((0, "paged_8KB_blocks_16B_loads"), (1, "paged_8KB_blocks_attention_loads")):
            ms = timed(lambda: lib.probe_paged(ctypes.c_void_p(buf.data_ptr()), ctypes.c_void_p(perm.data_ptr()),
                                               waves, run, mode, ctypes.c_void_p(sink.data_ptr()), sp), 5)
            out["read"][f"{name}_2048waves"] = round(waves * run * 8192 / (ms * 1e-3) / 1e9, 1)
        del buf, perm
        torch.cuda.empty_cache()

    if "gemv" in parts:
        # the gate||up expert GEMV's load shape without its arithmetic, against the kernel itself, on
        # config 2's routing regime (32 tokens x top-8 over 128 experts), rotating over 4 layers'
        # stacks so that HBM serves the weights
        from jitengine_amd import ops
        from jitengine_amd.quant import random_quantized

        lib.probe_gemv.argtypes = [P, P, LL, I, I, I, P, I, P, P]
        E, N, K, B, k = 128, 768, 2048, 32, 8
        stacks = [ops.prepack(random_quantized((E, 2 * N, K), 900 + i, device=dev)) for i in range(4)]
        estride = stacks[0].nbytes // E
        gen = torch.Generator(device=dev)
        gen.manual_seed(7)
        inds = torch.randn((B, E), generator=gen, device=dev).topk(k, dim=1).indices.to(torch.int32).contiguous()
        pk = ops.moe_pack(inds, E)
        cnt = pk.expert_cnt
        active = int((cnt > 0).sum())
        x = (torch.randn((B, K), generator=gen, device=dev) * 0.5).to(torch.bfloat16)
        sink = torch.empty(1 << 16, dtype=torch.int32, device=dev)
        alg = active * estride
        res = {"active_experts": active, "MB_per_launch": round(alg / 1e6, 1)}
        for mode, name in ((0, "weights_only"), (1, "weights_and_x")):
            def rot(mode=mode):
                for st_ in stacks:
                    lib.probe_gemv(ctypes.c_void_p(st_.data.data_ptr()), ctypes.c_void_p(cnt.data_ptr()), estride, E,
                                   N, K, ctypes.c_void_p(x.data_ptr()), mode, ctypes.c_void_p(sink.data_ptr()), sp)
            ms = timed(rot, 20) / len(stacks)
            res[f"{name}_us"] = round(ms * 1e3, 2)
            res[f"{name}_GB_s"] = round(alg / (ms * 1e-3) / 1e9, 1)
        ms = timed(lambda: [ops.expert_gate_up(x, st_, pk) for st_ in stacks], 20) / len(stacks)
        res["kernel_us"] = round(ms * 1e3, 2)
        res["kernel_GB_s"] = round(alg / (ms * 1e-3) / 1e9, 1)
        out["gemv"] = res
        del stacks

    if "launch" in parts:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(48):
                lib.probe_empty(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        ms = timed(g.replay, 20)
        out["launch"]["empty_in_graph_us"] = round(ms * 1e3 / 48, 3)
        del g

    if "barrier" in parts:
        cnt = torch.zeros(1, dtype=torch.int32, device=dev)
        status = torch.zeros(2, dtype=torch.int32, device=dev)
        max_blocks = int(lib.probe_barrier_max_blocks())
        for blocks in sorted({256, min(512, max_blocks)}):
            data = torch.zeros(blocks * 1024, dtype=torch.int32, device=dev)
            for words in (0, 1024):
                res = {}
                for phases in (0, 64):
                    def run(phases=phases, words=words, blocks=blocks, data=data):
                        cnt.zero_()
                        lib.probe_barrier(blocks, phases, words, ctypes.c_void_p(cnt.data_ptr()),
                                          ctypes.c_void_p(data.data_ptr()), 1 << 22,
                                          ctypes.c_void_p(status.data_ptr()), sp)
                    res[phases] = timed(run, 10)
                out["barrier"][f"{blocks}wg_{words * 4}B_per_wg_us"] = round((res[64] - res[0]) * 1e3 / 64, 3)
        out["barrier"]["timeouts"] = int(status[0])

    if "handoff" in parts:
        # cross-XCD handoff without cache-wide operations (device-coherent stores, a completion wait,
        # a device-scope counter; the last workgroup of a group reads its group's words back
        # device-coherent and checks each against this launch's values), against the same launch
        # without the handoff and against a second launch doing the read-back; 48 launches with
        # distinct values per HIP graph
        lib.probe_handoff.argtypes = [I, I, I, I, I, P, P, P, P]
        lib.probe_barrier2.argtypes = [I, I, I, P, P, I, P, P]
        res = {}
        status = torch.zeros(2, dtype=torch.int32, device=dev)
        handoff_shapes = ((32, 16, 2048), (256, 2, 2048), (128, 4, 4096), (1, 256, 1024), (1, 32, 4096))
        for groups, per, words in handoff_shapes:
            counters = torch.zeros(groups, dtype=torch.int32, device=dev)
            data = torch.zeros(groups * per * words, dtype=torch.int32, device=dev)
            ms = {}
            for mode in range(4):
                def launches(mode=mode, s=None):
                    for i in range(48):
                        rc = lib.probe_handoff(groups, per, words, 1000 * mode + i, mode,
                                               ctypes.c_void_p(counters.data_ptr()), ctypes.c_void_p(data.data_ptr()),
                                               ctypes.c_void_p(status.data_ptr()),
                                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
                        assert rc == 0, rc
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    launches()
                ms[mode] = timed(g.replay, 10) / 48
                del g
            key = f"{groups}x{per}wg_{words * 4 // 1024}KB"
            res[key] = {"write_only_us": round(ms[0] * 1e3, 3),
                        "handoff_device_scope_us": round(ms[1] * 1e3, 3),
                        "handoff_system_scope_us": round(ms[2] * 1e3, 3),
                        "write_then_readback_launch_us": round(ms[3] * 1e3, 3)}
        torch.cuda.synchronize()
        res["mismatched_words"] = int(status[0])
        # every handoff launch must have found exactly one last member per group
        res["readbacks"] = int(status[1])
        res["readbacks_expected"] = sum(g * 48 * 11 * 2 for g, _, _ in handoff_shapes)
        status.zero_()
        cnt = torch.zeros(1, dtype=torch.int32, device=dev)
        max_blocks = int(lib.probe_barrier2_max_blocks())
        for blocks in sorted({256, min(512, max_blocks)}):
            data = torch.zeros(2 * blocks * 1024, dtype=torch.int32, device=dev)
            for words in (0, 1024):
                t_ = {}
                for phases in (0, 64):
                    def run(phases=phases, words=words, blocks=blocks, data=data):
                        cnt.zero_()
                        rc = lib.probe_barrier2(blocks, phases, words, ctypes.c_void_p(cnt.data_ptr()),
                                                ctypes.c_void_p(data.data_ptr()), 1 << 22,
                                                ctypes.c_void_p(status.data_ptr()), sp)
                        assert rc == 0, rc
                    t_[phases] = timed(run, 10)
                res[f"grid_barrier_{blocks}wg_{words * 4}B_per_wg_us"] = round((t_[64] - t_[0]) * 1e3 / 64, 3)
        torch.cuda.synchronize()
        res["grid_barrier_mismatched_words"] = int(status[0])
        res["grid_barrier_timeouts"] = int(status[1])
        out["handoff"] = res
    print(json.dumps({"probe": out}), flush=True)
    return 0


def gemv_phases(dev: str) -> int:
    """Where the expert GEMVs' time goes: the gate||up and down kernels of the stamps build
    (libjit_stamps.so, JIT_QMM_STAMPS=1) on config 2's routing regime (32 tokens x top-8 over 128
    experts), rotating over 4 layers' stacks so that HBM serves the weights; per workgroup with work,
    s_memrealtime stamps at entry, once its expert's count is known, once its first pass's loads have
    landed, after the arithmetic, after the LDS reduction and at its end (csrc/qmm.hip)."""
    import ctypes

    from jitengine_amd import _lib
    from jitengine_amd import build as hip_build
    from jitengine_amd import ops
    from jitengine_amd.quant import random_quantized

    lib = ctypes.CDLL(hip_build.STAMPS_LIB)
    for name in ("jit_moe_gate_up_swiglu_packed", "jit_moe_down_packed"):
        getattr(lib, name).argtypes = _lib._SIGNATURES[name]
    lib.jit_qmm_stamps_clear.argtypes = [ctypes.c_void_p]
    lib.jit_qmm_stamps_read.argtypes = [ctypes.c_void_p, ctypes.c_int]
    E, I, D, B, k = 128, 768, 2048, 32, 8
    gus = [ops.prepack(random_quantized((E, 2 * I, D), 900 + i, device=dev)) for i in range(4)]
    dns = [ops.prepack(random_quantized((E, D, I), 950 + i, device=dev)) for i in range(4)]
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    inds = torch.randn((B, E), generator=gen, device=dev).topk(k, dim=1).indices.to(torch.int32).contiguous()
    pk = ops.moe_pack(inds, E)
    P = B * k
    x = (torch.randn((B, D), generator=gen, device=dev) * 0.5).to(torch.bfloat16)
    h = (torch.randn((P, I), generator=gen, device=dev) * 0.5).to(torch.bfloat16)
    hout = torch.empty((P, I), dtype=torch.bfloat16, device=dev)
    rout = torch.empty((P, D), dtype=torch.bfloat16, device=dev)
    active = int((pk.expert_cnt > 0).sum())
    sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731

    def gate_up(i):
        return lib.jit_moe_gate_up_swiglu_packed(p(x), D, p(pk.pair_row), p(pk.expert_cnt), p(pk.expert_off), E,
                                                 p(gus[i].data), I, P, p(hout), sp)

    def down(i):
        return lib.jit_moe_down_packed(p(h), I, p(pk.expert_cnt), p(pk.expert_off), E, p(dns[i].data), D, P,
                                       p(rout), sp)

    out = {"active_experts": active}
    names = ("count_known", "loads_landed", "arithmetic", "lds_reduction", "epilogue")
    for kname, fn, per_expert in (("gate_up_swiglu", gate_up, 1769472), ("down", down, 884736)):
        for rep in range(8):
            assert fn(rep % 4) == 0
        torch.cuda.synchronize()
        assert lib.jit_qmm_stamps_clear(sp) == 0
        s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s_ev.record()
        assert fn(0) == 0
        e_ev.record()
        torch.cuda.synchronize()
        buf = np.zeros((1 << 16, 8), np.uint64)
        assert lib.jit_qmm_stamps_read(buf.ctypes.data_as(ctypes.c_void_p), 1 << 16) == 0
        st = buf[buf[:, 6] == 1][:, :6].astype(np.int64)
        t0 = st[:, 0].min()
        span = int(st[:, 5].max() - t0)
        tick_us = 0.01  # s_memrealtime counts at 100 MHz
        d = np.diff(st, axis=1) * tick_us
        life = (st[:, 5] - st[:, 0]) * tick_us
        res = {"workgroups_with_work": int(st.shape[0]), "event_us": round(s_ev.elapsed_time(e_ev) * 1e3, 2),
               "stamp_span_us": round(span * tick_us, 2), "wg_life_mean_us": round(float(life.mean()), 3),
               "mean_resident_wgs": round(float(life.sum()) / (span * tick_us), 1),
               "alg_MB": round(active * per_expert / 1e6, 1)}
        for j, n in enumerate(names):
            res[f"{n}_mean_us"] = round(float(d[:, j].mean()), 3)
            res[f"{n}_p90_us"] = round(float(np.percentile(d[:, j], 90)), 3)
        # when the workgroups start, in tenths of the span: how the grid drains
        res["starts_by_tenth_of_span"] = np.histogram((st[:, 0] - t0) / max(span, 1), bins=10, range=(0, 1))[0].tolist()
        out[kname] = res
    print(json.dumps({"gemv_phases": out}), flush=True)
    return 0


def attn_phases(dev: str) -> int:
    """Where decode attention's time goes (the stamps build, libjit_stamps.so with JIT_ATTN_STAMPS=1):
    config 2's 32 ragged sequences and config 4's 262,144 keys, each over 3 pools in turn (so HBM
    serves the pages); per workgroup, s_memrealtime stamps at entry, once its first K has landed,
    at the end of its key loop, after its splits' states met in LDS and at its end."""
    import ctypes

    from jitengine_amd import _lib
    from jitengine_amd import build as hip_build
    from jitengine_amd import ops

    lib = ctypes.CDLL(hip_build.STAMPS_LIB)
    lib.jit_paged_decode_attn.argtypes = _lib._SIGNATURES["jit_paged_decode_attn"]
    lib.jit_attn_stamps_clear.argtypes = [ctypes.c_void_p]
    lib.jit_attn_stamps_read.argtypes = [ctypes.c_void_p, ctypes.c_int]
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = {}
    for config in (2, 4):
        rng = np.random.default_rng(seed_for(config))
        if config == 2:
            lens = np.round(np.exp(rng.uniform(np.log(128), np.log(32768), 32))).astype(np.int32) + 1
        else:
            lens = np.array([CONFIG4_KEYS], np.int32)
        B, H, Hkv = lens.size, 32, 4
        npg = (lens + 15) // 16
        num_pages = int(npg.sum())
        perm = rng.permutation(num_pages)
        table = np.zeros((B, int(npg.max())), np.int32)
        at = 0
        for b in range(B):
            table[b, :npg[b]] = perm[at:at + npg[b]]
            at += npg[b]
        gen = torch.Generator(device=dev)
        gen.manual_seed(5)
        pools = [torch.randn((num_pages, Hkv, 2, 2048), generator=gen, device=dev, dtype=torch.bfloat16)
                 for _ in range(3)]
        q = torch.randn((B, H, 128), generator=gen, device=dev, dtype=torch.bfloat16)
        tt = torch.from_numpy(table).to(dev)
        plan = ops.attn_plan(lens, dev)
        ws = torch.empty(ops.attn_workspace_bytes(plan.total, H), dtype=torch.uint8, device=dev)
        o = torch.empty_like(q)

        def run(i):
            return lib.jit_paged_decode_attn(p(q), p(pools[i]), p(tt), table.shape[1], p(plan.lens),
                                             p(plan.chunk_start), p(plan.chunk_seq), B, H, Hkv, 128 ** -0.5,
                                             plan.total, p(ws), p(o), sp)
        for rep in range(6):
            assert run(rep % 3) == 0
        torch.cuda.synchronize()
        assert lib.jit_attn_stamps_clear(sp) == 0
        s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s_ev.record()
        assert run(0) == 0
        e_ev.record()
        torch.cuda.synchronize()
        buf = np.zeros((1 << 14, 8), np.uint64)
        assert lib.jit_attn_stamps_read(buf.ctypes.data_as(ctypes.c_void_p), 1 << 14) == 0
        slots = np.flatnonzero(buf[:, 7] == 1)
        st = buf[slots][:, :5].astype(np.int64)
        t0 = st[:, 0].min()
        rel = (st - t0) * 0.01  # microseconds (s_memrealtime counts at 100 MHz)
        xcd = slots % 8  # workgroups are dealt to the 8 XCDs round-robin in launch order
        d = np.diff(st, axis=1) * 0.01
        kv = int(lens.astype(np.int64).sum()) * 2048

        def q_(v):
            return [round(float(np.percentile(v, x)), 2) for x in (0, 10, 50, 90, 100)]
        out[f"config{config}"] = {
            "workgroups": int(st.shape[0]), "event_us_kernel_plus_merge": round(s_ev.elapsed_time(e_ev) * 1e3, 2),
            "span_us": round(float(rel[:, 4].max()), 2), "kv_MB": round(kv / 1e6, 1),
            "start_us_pctl_0_10_50_90_100": q_(rel[:, 0]), "end_us_pctl_0_10_50_90_100": q_(rel[:, 4]),
            "first_k_landed_us_mean": round(float(d[:, 0].mean()), 2), "key_loop_us_pctl": q_(d[:, 1]),
            "split_merge_wait_us_mean": round(float(d[:, 2].mean()), 3), "tail_us_mean": round(float(d[:, 3].mean()), 3),
            "end_us_mean_by_xcd": [round(float(rel[xcd == x, 4].mean()), 2) for x in range(8)],
            "end_us_max_by_xcd": [round(float(rel[xcd == x, 4].max()), 2) for x in range(8)],
            # every workgroup of config 4 streams an equal share at once: the bytes over the median key loop
            "steady_rate_GB_s": round(kv / (float(np.median(d[:, 1])) * 1e-6) / 1e9, 1) if config == 4 else None}
    print(json.dumps({"attn_phases": out}), flush=True)
    return 0


OP_KERNELS = {  # the kernels one op launches (rocprofv3 kernel names contain these)
    "paged_attention": ["paged_attn_kernel", "attn_merge_kernel"],
    "gate_up_swiglu": ["qmm_kernel<1, 8, true, true"],
    "down": ["qmm_kernel<4, 4, false, true"],
    "gate_up_swiglu_seg": ["seg_kernel<true, false,"],  # (any token-chunk length)
    "down_seg": ["seg_kernel<false, false,"],
    "qkv_proj_seg": ["seg_kernel<false, true, 10>"],  # (config 3's 2,108 rows: the 10-tile chunk; o_proj takes 5)
    "prefill_attention": ["prefill_attn_kernel", "prefill_merge_kernel"],
}


def rocprof_summary(args) -> int:
    """Text summary of rocprofv3 CSV output for one op: per-kernel launch statistics (from
    --kernel-trace --stats) and HBM traffic per launch (FETCH_SIZE and WRITE_SIZE from two --pmc
    runs of the same command, each scaled by what the counter reads for a plain copy of known size
    in a --copy-calibration run)."""
    import csv
    import collections

    def per_kernel(path):
        d = collections.defaultdict(list)
        for r in csv.DictReader(open(path)):
            d[r["Kernel_Name"]].append(float(r["Counter_Value"]))
        return d

    def match(d, frag):
        hits = [k for k in d if frag in k]
        if len(hits) != 1:
            raise SystemExit(f"kernel fragment {frag!r} matches {len(hits)} names")
        return hits[0]

    d_dir = args.rocprof_summary
    stats = {r["Name"]: r for r in csv.DictReader(open(os.path.join(d_dir, "kt", "kt_kernel_stats.csv")))}
    cfg = " --no-bs1" if args.config == 2 else f" --config {args.config}"
    print(f"# rocprofv3 summary of bench.py's config-{args.config} workload, op {args.op}")
    print("# made on one MI355X from the repository root by:")
    print(f"#   rocprofv3 --kernel-trace --stats -f csv -d prof/kt -o kt -- python3 bench.py{cfg} --steps 10 --warmup 2")
    if args.op == "step":
        print(f"#   python3 bench.py --rocprof-summary prof --op step{cfg}")
        print("# this library's kernels over the whole run (warm-up + timed steps + per-op replays);")
        print("# launches, average / min / max duration in us, share of this library's kernel time")
        ours = [r for r in stats.values() if "(anonymous namespace)::" in r["Name"] and "at::" not in r["Name"]
                and "prepack" not in r["Name"]]
        ours.sort(key=lambda r: -float(r["TotalDurationNs"]))
        tot = sum(float(r["TotalDurationNs"]) for r in ours)
        for r in ours:
            name = r["Name"].replace("(anonymous namespace)::", "").split("(")[0]
            print(f"{int(r['Calls']):7d} {float(r['AverageNs']) / 1e3:9.2f} {float(r['MinNs']) / 1e3:9.2f} "
                  f"{float(r['MaxNs']) / 1e3:9.2f} {100 * float(r['TotalDurationNs']) / tot:6.1f}%  {name}")
        return 0
    ng = " --no-graph" if args.config in (0, 2, 4) else ""  # (config 3 always replays a graph)
    for c in (f"FETCH_SIZE -f csv -d prof/fetch -o fetch -- python3 bench.py{cfg} --steps 1 --warmup 1{ng}",
              f"WRITE_SIZE -f csv -d prof/write -o write -- python3 bench.py{cfg} --steps 1 --warmup 1{ng}",
              "FETCH_SIZE -f csv -d prof/cfetch -o cfetch -- python3 bench.py --copy-calibration",
              "WRITE_SIZE -f csv -d prof/cwrite -o cwrite -- python3 bench.py --copy-calibration"):
        print(f"#   rocprofv3 --pmc {c}")
    print(f"#   python3 bench.py --rocprof-summary prof --op {args.op}{cfg}")
    fetch = per_kernel(os.path.join(d_dir, "fetch", "fetch_counter_collection.csv"))
    write = per_kernel(os.path.join(d_dir, "write", "write_counter_collection.csv"))
    cfetch = per_kernel(os.path.join(d_dir, "cfetch", "cfetch_counter_collection.csv"))
    cwrite = per_kernel(os.path.join(d_dir, "cwrite", "cwrite_counter_collection.csv"))
    copy_kib = 256 * 1024  # the calibration copy reads and writes 256 MiB
    ck = match(cfetch, "copyBuffer")
    f_scale = copy_kib / float(np.mean(cfetch[ck]))
    w_scale = copy_kib / float(np.mean(cwrite[match(cwrite, "copyBuffer")]))
    print(f"op: {args.op}")
    print(f"calibration: FETCH_SIZE x {f_scale:.4f}, WRITE_SIZE x {w_scale:.4f} "
          f"(copy of 256 MiB reads {np.mean(cfetch[ck]):.1f} KiB by FETCH_SIZE)")
    tot_us, tot_bytes = 0.0, 0.0
    for frag in OP_KERNELS[args.op]:
        name = match(stats, frag)
        st = stats[name]
        avg_us = float(st["AverageNs"]) / 1e3
        fk, wk = match(fetch, frag), match(write, frag)
        fb = float(np.mean(fetch[fk])) * 1024 * f_scale
        wb = float(np.mean(write[wk])) * 1024 * w_scale
        tot_us += avg_us
        tot_bytes += fb + wb
        print(f"kernel: {name[:120]}")
        print(f"  launches {st['Calls']}, average {avg_us:.2f} us, min {float(st['MinNs']) / 1e3:.2f} us, "
              f"max {float(st['MaxNs']) / 1e3:.2f} us")
        print(f"  HBM read {fb / 1e6:.2f} MB, written {wb / 1e6:.2f} MB per launch "
              f"({len(fetch[fk])} / {len(write[wk])} dispatches counted)")
    print(f"op_average_us: {tot_us:.2f}")
    print(f"traffic_bytes_per_launch: {tot_bytes:.0f}")
    return 0


def rocprof_mfma(args) -> int:
    """Per-kernel MFMA and LDS evidence from one rocprofv3 --pmc pass (SQ_VALU_MFMA_BUSY_CYCLES,
    SQ_INSTS_VALU_MFMA_MOPS_BF16, SQ_BUSY_CU_CYCLES, SQ_LDS_BANK_CONFLICT, SQ_LDS_IDX_ACTIVE,
    GRBM_GUI_ACTIVE): the MFMA pipes' busy share of the
    kernel's active cycles over all 1,024 SIMDs (GRBM_GUI_ACTIVE adds up the 8 XCDs' active cycles, so
    the kernel's own cycles are an eighth of it), and the bf16 MFMA FLOPs actually issued (one MOP is
    512 FLOPs; padding rows and tokens included) per launch, and the LDS bank-conflict cycles per LDS
    active cycle."""
    import csv
    import collections

    d_dir = args.rocprof_mfma
    vals = collections.defaultdict(lambda: collections.defaultdict(list))
    for r in csv.DictReader(open(os.path.join(d_dir, "mfma", "mfma_counter_collection.csv"))):
        vals[r["Kernel_Name"]][r["Counter_Name"]].append(float(r["Counter_Value"]))
    cfg = " --no-bs1" if args.config == 2 else f" --config {args.config}"
    ng = " --no-graph" if args.config in (0, 2, 4) else ""
    print(f"# rocprofv3 MFMA counters of bench.py's config-{args.config} workload")
    print("# made on one MI355X from the repository root by:")
    print("#   rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_BF16 SQ_BUSY_CU_CYCLES SQ_LDS_BANK_CONFLICT "
          f"SQ_LDS_IDX_ACTIVE GRBM_GUI_ACTIVE -f csv -d prof/mfma -o mfma -- python3 bench.py{cfg} --steps 1 --warmup 1{ng}")
    print(f"#   python3 bench.py --rocprof-mfma prof{cfg}")
    print("# per kernel (mean over dispatches): MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs"
          " x 1024 SIMDs);")
    print("# issued = SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512 FLOPs per launch;"
          " LDS conflict = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE")
    print(f"{'dispatches':>10} {'MFMA busy':>10} {'issued GFLOP':>13} {'LDS conflict':>13}  kernel")
    rows = []
    for name, c in vals.items():
        if "(anonymous namespace)::" not in name or "at::" in name:
            continue
        busy = float(np.mean(c.get("SQ_VALU_MFMA_BUSY_CYCLES", [0.0])))
        act = float(np.mean(c.get("GRBM_GUI_ACTIVE", [1.0])))
        mops = float(np.mean(c.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", [0.0])))
        n = len(c.get("GRBM_GUI_ACTIVE", []))
        lds = float(np.mean(c.get("SQ_LDS_IDX_ACTIVE", [0.0])))
        conf = float(np.mean(c.get("SQ_LDS_BANK_CONFLICT", [0.0])))
        rows.append((busy / (act / 8.0 * 1024.0) if act else 0.0, mops * 512 / 1e9, n,
                     name.replace("(anonymous namespace)::", "").split("(")[0], conf / lds if lds else None))
    for frac, gf, n, name, cr in sorted(rows, key=lambda r: -r[1]):
        if gf > 0 or cr is not None:
            crs = f"{100 * cr:12.1f}%" if cr is not None else f"{'-':>13}"
            print(f"{n:10d} {100 * frac:9.1f}% {gf:13.2f} {crs}  {name}")
    return 0


SQ_PASSES = {  # two rocprofv3 --pmc passes (at most 8 SQ counters each)
    "sqa": ["SQ_WAVES", "SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY", "SQ_ACTIVE_INST_ANY",
            "SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_VMEM"],
    "sqb": ["SQ_INST_LEVEL_VMEM", "SQ_INSTS_VMEM_RD", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU", "SQ_INSTS_MFMA",
            "SQ_ACTIVE_INST_LDS", "SQ_WAIT_INST_LDS", "SQ_CYCLES"],
}


def rocprof_sq(args) -> int:
    """Per-kernel issue and memory-wait evidence from the two SQ counter passes of SQ_PASSES: where
    a wave's life goes (waiting on a counter or barrier, ready but not issued, issuing; all as shares
    of SQ_WAVE_CYCLES), the instructions per wave (VALU, MFMA, vector-memory reads) and the mean
    vector-memory latency (SQ_INST_LEVEL_VMEM / SQ_INSTS_VMEM_RD, in SQ cycles)."""
    import csv
    import collections

    d_dir = args.rocprof_sq
    vals = collections.defaultdict(lambda: collections.defaultdict(list))
    for pas in SQ_PASSES:
        for r in csv.DictReader(open(os.path.join(d_dir, pas, f"{pas}_counter_collection.csv"))):
            vals[r["Kernel_Name"]][r["Counter_Name"]].append(float(r["Counter_Value"]))
    cfg = " --no-bs1" if args.config == 2 else f" --config {args.config}"
    print(f"# rocprofv3 SQ counters of bench.py's config-{args.config} workload")
    print("# made on one MI355X from the repository root by:")
    for pas, cs in SQ_PASSES.items():
        print(f"#   rocprofv3 --pmc {' '.join(cs)} -f csv -d prof/{pas} -o {pas} -- python3 bench.py{cfg} --steps 1 "
              "--warmup 1 --no-graph")
    print(f"#   python3 bench.py --rocprof-sq prof{cfg}")
    print("# shares of SQ_WAVE_CYCLES: wait = SQ_WAIT_ANY (a counter or barrier), ready = SQ_WAIT_INST_ANY (an "
          "instruction ready, not issued), issue = SQ_ACTIVE_INST_ANY;")
    print("# per wave: VALU = SQ_INSTS_VALU / SQ_WAVES, MFMA = SQ_INSTS_MFMA / SQ_WAVES, VMEM rd = SQ_INSTS_VMEM_RD / "
          "SQ_WAVES; vmem latency = SQ_INST_LEVEL_VMEM / SQ_INSTS_VMEM_RD (SQ cycles)")
    print(f"{'waves':>8} {'wait':>6} {'ready':>6} {'issue':>6} {'VALU/w':>7} {'MFMA/w':>7} {'VMEMrd/w':>8} "
          f"{'vmem lat':>8}  kernel")
    for name, c in sorted(vals.items(), key=lambda kv: -float(np.mean(kv[1].get("SQ_WAVE_CYCLES", [0.0])))):
        if "(anonymous namespace)::" not in name or "at::" in name:
            continue
        m = {k: float(np.mean(v)) for k, v in c.items()}
        wc = m.get("SQ_WAVE_CYCLES", 0.0)
        w = m.get("SQ_WAVES", 0.0)
        if not wc or not w:
            continue
        rd = m.get("SQ_INSTS_VMEM_RD", 0.0)
        lat = m.get("SQ_INST_LEVEL_VMEM", 0.0) / rd if rd else 0.0
        print(f"{w:8.0f} {100 * m.get('SQ_WAIT_ANY', 0) / wc:5.1f}% {100 * m.get('SQ_WAIT_INST_ANY', 0) / wc:5.1f}% "
              f"{100 * m.get('SQ_ACTIVE_INST_ANY', 0) / wc:5.1f}% {m.get('SQ_INSTS_VALU', 0) / w:7.0f} "
              f"{m.get('SQ_INSTS_MFMA', 0) / w:7.1f} {rd / w:8.1f} {lat:8.0f}  "
              f"{name.replace('(anonymous namespace)::', '').split('(')[0]}")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--no-graph", action="store_true", help="time eager launches instead of a HIP graph replay")
    ap.add_argument("--no-cpu", action="store_true", help="leave out the CPU baseline (quick device-only runs)")
    ap.add_argument("--no-bs1", action="store_true",
                    help="config 2 only: skip the bs=1 (config 4) measurement reported beside it")
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--sampler", action="store_true", help="time the sampler's kernels (vocabulary 248,320)")
    ap.add_argument("--probe", action="store_true",
                    help="measure the streaming-read ceiling, the empty-launch floor and the grid-barrier cost")
    ap.add_argument("--attn-phases", action="store_true",
                    help="per-phase stamps of decode attention (the stamps build of csrc/attention.hip)")
    ap.add_argument("--gemv-phases", action="store_true",
                    help="per-phase stamps of the expert GEMVs (the stamps build of csrc/qmm.hip)")
    ap.add_argument("--probe-parts", default="read,launch,barrier",
                    help="which probe measurements to run (the barrier's cooperative launch ends rocprofv3 badly)")
    ap.add_argument("--rocprof-summary", metavar="DIR",
                    help="summarise rocprofv3 CSV output under DIR (kt/, fetch/, write/, cfetch/, cwrite/)")
    ap.add_argument("--op", default="paged_attention", choices=sorted(OP_KERNELS) + ["step"])
    ap.add_argument("--rocprof-mfma", metavar="DIR", help="summarise an MFMA counter pass under DIR/mfma/")
    ap.add_argument("--rocprof-sq", metavar="DIR", help="summarise the SQ counter passes under DIR/sqa/, DIR/sqb/")
    args = ap.parse_args()
    if args.rocprof_summary:
        return rocprof_summary(args)
    if args.rocprof_mfma:
        return rocprof_mfma(args)
    if args.rocprof_sq:
        return rocprof_sq(args)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        return 2
    dev = "cuda:0"
    torch.cuda.set_device(0)
    if args.copy_calibration:
        return copy_calibration(dev)
    if args.probe:
        return probe(dev, set(args.probe_parts.split(",")))
    if args.gemv_phases:
        return gemv_phases(dev)
    if args.attn_phases:
        return attn_phases(dev)
    if args.sampler:
        return bench_sampler(dev)
    if args.config == 1:
        res = bench_config1(args.steps, args.warmup, dev)
    elif args.config in (0, 2, 4):
        res = bench_decode(args.config, args.steps, args.warmup, dev, graph=not args.no_graph,
                           n_layers=args.layers, cpu=not args.no_cpu)
        if args.config == 2 and not args.no_bs1:
            # the metric's bs=1 half: config 4 on the same model, reported beside config 2
            # config 2's pools stay allocated while config 4 runs: an engine allocates its KV pool once
            # and keeps it, and config 4's 25.8 GB placed in the memory just freed by config 2's 16.6 GB
            # measured slower (attention 92.8 against 89.2 us a layer on one MI355X: the pool's random
            # 32 KB page reads depend on how its pages are mapped)
            model, keep = res.pop("_model"), res.pop("_pools")
            r4 = bench_decode(4, args.steps, args.warmup, dev, graph=not args.no_graph, model=model, cpu=False)
            res["bs1"] = {"workload": r4["config"]["workload"] + " (config 2's weights)",
                          "value": r4["value"], "unit": "tokens/s", "ms_per_step": r4["ms_per_step"],
                          "step_hbm": r4["step_hbm"], "north_star": r4["north_star"],
                          "hot_path_hbm": r4["hot_path_hbm"],
                          "op_us_per_step": r4["op_us_per_step"],
                          "attention": {k: r4["roofline"][k] for k in ("achieved", "alg_bytes_per_launch",
                                                                        "launch_us")} | {"unit": "GB/s"}}
            del r4, model, keep
    elif args.config == 3:
        res = bench_config3(args.steps, args.warmup, dev)
    else:
        print(f"config {args.config} is not wired into bench.py", file=sys.stderr)
        return 2
    res.pop("_y", None)
    res.pop("_model", None)
    res.pop("_pools", None)
    line = {"metric": res["metric"], "value": res["value"], "unit": res["unit"], "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": res["ms_per_step"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": res["dtype"],
            "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights quantized to MLX 4-bit g64)",
            "config": res["config"], "roofline": res["roofline"], "cpu_baseline": res.get("cpu_baseline")}
    for key in ("arithmetic", "step_hbm", "north_star", "hot_path_hbm", "step_tflops", "op_us", "op_us_per_step", "op_us_sum_per_step", "kernels_us",
                "bs1"):
        if key in res:
            line[key] = res[key]
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
