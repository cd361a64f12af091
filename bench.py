"""Benchmark of the ragged MoE decode step on one MI355X (prints ONE JSON line).

python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2] [--layers 48] [--no-graph]

config 2 (the default; BASELINE.json configs[2], the workload the metric is quoted on): ragged
continuous-batch decode of 32 sequences over the paged KV pool through 48 layers of the 4-bit
Qwen3-MoE-style block; a step decodes one token per sequence (value = tokens/s).  The step is
captured once as a HIP graph and replayed (--no-graph times eager launches).
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


class Timer:
    """Per-kernel HIP-event timing on the current stream."""

    def __init__(self):
        self.acc = {}

    def run(self, name, fn):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        out = fn()
        e.record()
        self.acc.setdefault(name, []).append((s, e))
        return out

    def means_us(self):
        torch.cuda.synchronize()
        return {k: 1e3 * float(np.mean([a.elapsed_time(b) for a, b in v])) for k, v in self.acc.items()}


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

    # per-kernel durations, same launches, events around each
    tm = Timer()
    for _ in range(max(steps, 10)):
        pk = tm.run("moe_pack", lambda: ops.moe_pack(inds, E))
        h = tm.run("gate_up_swiglu", lambda: ops.expert_gate_up(x, gu, pk))
        r = tm.run("down", lambda: ops.expert_down(h, dn, pk))
        tm.run("combine", lambda: ops.moe_combine(r, pk, scores))
    kus = tm.means_us()

    flat = inds.cpu().numpy().reshape(-1)
    U = int(np.unique(flat).size)
    P = B * k
    gu_bytes_e = 2 * I * D // 2 + 2 * (2 * I) * (D // 64) * 2
    dn_bytes_e = D * I // 2 + 2 * D * (I // 64) * 2
    alg_gate_up = U * gu_bytes_e + B * D * 2 + P * I * 2
    alg_down = U * dn_bytes_e + P * I * 2 + P * D * 2
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
    times = []
    for _ in range(3):
        c0 = time.perf_counter()
        oracle.moe_experts(x_np[:nb], ind_np, sc_np, gu_h, dn_h, E)
        times.append(time.perf_counter() - c0)
    cpu_tps = nb / float(np.median(times))

    return {
        "metric": "decode tok/s (bs=1, ragged bs=32) + achieved HBM GB/s as % of MI355X peak",
        "value": B / (ms * 1e-3),
        "unit": "tokens/s",
        "ms_per_step": ms,
        "dtype": "bf16 activations, 4-bit g64 weights, fp32 accumulate",
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
                                   f"the {B} tokens, median of 3"},
        "_y": y,
    }


def bench_config2(steps: int, warmup: int, dev: str, graph: bool, n_layers: int = 48) -> dict:
    """ragged continuous-batch decode over the paged KV pool -- 32 sequences
    with lengths log-uniform in [128, 32768], 16-token pages in a random permutation, the full
    Qwen3-MoE-style 4-bit decoder block for 48 layers with independent seeded weights.  A step
    decodes one token per sequence through all layers (each row writes position L_b and attends
    to L_b + 1 keys)."""
    import oracle
    from jitengine_amd import ops
    from jitengine_amd.model import DecoderLayer, MoEConfig, Model, make_step_state, random_layer_weights, rope_inv_freq

    cfg = MoEConfig(layers=n_layers)
    seed = seed_for(2)
    rng = np.random.default_rng(seed)
    B = 32
    lens = np.round(np.exp(rng.uniform(np.log(128), np.log(32768), B))).astype(np.int32)
    npg = (lens + 1 + 15) // 16
    num_pages = int(npg.sum())
    perm = rng.permutation(num_pages)
    table = np.zeros((B, int(npg.max())), np.int32)
    at = 0
    for b in range(B):
        table[b, :npg[b]] = perm[at:at + npg[b]]
        at += npg[b]
    layers, w0 = [], None
    for l in range(n_layers):
        w = random_layer_weights(cfg, seed * 100 + l, dev)
        layers.append(DecoderLayer(cfg, w))
        if l == 0:
            w0 = w
        del w
    model = Model.__new__(Model)
    model.cfg, model.layers = cfg, layers
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed + 7)
    pools = [torch.randn((num_pages, 2, cfg.kv_heads, 16 * 128), generator=gen, device=dev, dtype=torch.bfloat16)
             for _ in range(n_layers)]
    x = torch.randn((B, cfg.hidden), generator=gen, device=dev, dtype=torch.bfloat16)
    table_d = torch.from_numpy(table).to(dev)
    st = make_step_state(cfg, lens, table_d)
    torch.cuda.synchronize()

    # distinct experts per layer (for the algorithmic byte count), one eager step
    U = []
    xx = x
    for l, layer in enumerate(model.layers):
        d = {}
        xx = layer.step(xx, pools[l], st, debug=d)
        U.append(int(torch.unique(d["inds"]).numel()))
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

    # per-kernel durations over one eager step (events around each launch)
    tm = Timer()
    for _ in range(2):
        model.decode_step(x, pools, st, prof=tm.run)
    kus = {k: v * 1.0 for k, v in tm.means_us().items()}  # mean per launch
    launches = {k: len(v) for k, v in tm.acc.items()}
    total_us = {k: kus[k] * launches[k] / 2 for k in kus}  # per step

    dense = cfg.qkv_rows * cfg.hidden // 2 * 9 // 8 + cfg.hidden * cfg.heads * 128 // 2 * 9 // 8 \
        + cfg.experts * cfg.hidden // 2 * 9 // 8
    per_expert = 2654208
    kv = int((lens.astype(np.int64) + 1).sum()) * 2 * cfg.kv_heads * 128 * 2
    alg_step = n_layers * (dense + kv) + sum(U) * per_expert
    # the dominant kernel by time in the step
    dom = max(total_us, key=total_us.get)
    alg_kernel = {
        "paged_attention": kv + B * cfg.heads * 128 * 2 * 2,
        "gate_up_swiglu": float(np.mean(U)) * 1769472,
        "down": float(np.mean(U)) * 884736,
    }
    achieved = alg_kernel.get(dom, 0.0) / (kus[dom] * 1e-6) / 1e9 if dom in alg_kernel else None

    # CPU baseline: the oracle's decoder layer (layer 0) on a sample of rows, scaled to 48 layers
    nb = 4
    def host_q(lin):
        return (lin.weight.cpu().numpy().view(np.uint32), lin.scales.view(torch.int16).cpu().numpy().view(np.uint16),
                lin.biases.view(torch.int16).cpu().numpy().view(np.uint16))
    u16 = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)  # noqa: E731
    lw = {"input_norm": u16(w0["input_norm"]), "qkv": host_q(w0["qkv"]), "q_norm": u16(w0["q_norm"]),
          "k_norm": u16(w0["k_norm"]), "o": host_q(w0["o"]), "post_norm": u16(w0["post_norm"]),
          "router": host_q(w0["router"]), "gate_up": host_q(w0["gate_up"]), "down": host_q(w0["down"])}
    pool_h = u16(pools[0]).copy()
    ocfg = {"heads": cfg.heads, "kv_heads": cfg.kv_heads, "experts": cfg.experts, "top_k": cfg.top_k,
            "eps": cfg.eps, "inv_freq": rope_inv_freq(cfg.rope_theta, 128)}
    xs = u16(x)[:nb]
    c0 = time.perf_counter()
    oracle.decoder_layer(xs, lw, pool_h, table[:nb], lens[:nb], ocfg)
    t_cpu = time.perf_counter() - c0
    cpu_tps = nb / (t_cpu * n_layers)

    return {
        "metric": "decode tok/s (bs=1, ragged bs=32) + achieved HBM GB/s as % of MI355X peak",
        "value": B / (ms * 1e-3),
        "unit": "tokens/s",
        "ms_per_step": ms,
        "dtype": "bf16 activations, 4-bit g64 weights, fp32 accumulate",
        "config": {"workload": f"config2: ragged 32-sequence decode, {n_layers} layers of the Qwen3-MoE-style 4-bit "
                               "block, paged bf16 KV (16-token pages, permuted), lens log-uniform [128, 32768]",
                   "sequences": B, "layers": n_layers, "kv_tokens": int(lens.sum()), "lens_min": int(lens.min()),
                   "lens_max": int(lens.max()), "distinct_experts_mean": float(np.mean(U)),
                   "hip_graph": bool(graph), "ms_per_step_eager": ms_eager},
        "step_hbm": {"alg_bytes": alg_step, "GB_s": alg_step / (ms * 1e-3) / 1e9,
                     "frac": alg_step / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                     "split": {"experts": sum(U) * per_expert, "kv": n_layers * kv, "dense": n_layers * dense}},
        "kernels_us": kus,
        "kernels_us_per_step": total_us,
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": (achieved / HBM_PEAK_GBS) if achieved else None,
                     "alg_bytes_per_launch": alg_kernel.get(dom), "traffic": None},
        "cpu_baseline": {"value": cpu_tps, "unit": "tokens/s", "cores": oracle.num_threads(), "kind": "port",
                         "sample": f"oracle decoder layer 0 (float64 dots) for {nb} of the {B} rows "
                                   f"(lens {list(map(int, lens[:nb]))}), time x {n_layers} layers"},
        "_y": y,
    }


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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--no-graph", action="store_true", help="time eager launches instead of a HIP graph replay")
    ap.add_argument("--copy-calibration", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        return 2
    dev = "cuda:0"
    torch.cuda.set_device(0)
    if args.copy_calibration:
        return copy_calibration(dev)
    if args.config == 1:
        res = bench_config1(args.steps, args.warmup, dev)
    elif args.config == 2:
        res = bench_config2(args.steps, args.warmup, dev, graph=not args.no_graph, n_layers=args.layers)
    else:
        print(f"config {args.config} is not wired into bench.py", file=sys.stderr)
        return 2
    res.pop("_y", None)
    line = {"metric": res["metric"], "value": res["value"], "unit": res["unit"], "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": res["ms_per_step"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": res["dtype"],
            "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights quantized to MLX 4-bit g64)",
            "config": res["config"], "roofline": res["roofline"], "cpu_baseline": res["cpu_baseline"]}
    for key in ("step_hbm", "kernels_us", "kernels_us_per_step"):
        if key in res:
            line[key] = res[key]
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
