"""CPU oracle for the ragged MoE decode step -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package, and
only as the checker; the product path (jitengine_amd) never imports it.  The arithmetic lives in
jit_oracle.c (a C restatement of the reference's algorithm, each function citing the reference
lines it follows); this module wraps it with numpy.  bf16 arrays are numpy uint16 bit patterns.

Parity status of each function (how it is pinned, see tests/test_oracle.py):
  exp_neg, softmax_bf16   vs float64 math.exp / softmax (closed form), within the stated ulps
  topk_from_gates         vs numpy's stable argsort tail (a library routine), brute force
  router_topk             composition of the two above + bf16 sequential sum vs torch bf16 ops
  moe_pack                vs numpy stable argsort + np.unique (the FN reference's own calls)
  dequant4                known-answer words + an independent numpy unpack
  qmm                     vs torch float64 matmul of independently dequantized weights
  qmv_mlx_f32             vs float64 within fp32 accumulation bounds (it is only an error yardstick)
  exp_pos                 vs math.exp within 2 ulp over [0, 88.7] (closed form)
  sigmoid_bf16            exhaustively over every bf16 g vs an independent numpy restatement of the
                          SigmoidX bf16 steps (float64 exp); they differ only within 2^-16 of a tie
  swiglu_bf16             vs float64 silu(g) * u within bf16 rounding bounds
  moe_gate_up / moe_down  vs qmm + swiglu composed in numpy (different code path, same maths)
  moe_combine             vs torch bf16 ops in slot order (a library routine)
  kv_append_paged/gather  integer addressing: round trip, page-permutation invariance
  q4_prepack              a byte permutation (multiset of bytes preserved, every word placed once);
                          on the GPU, GEMMs on packed and MLX layouts agree bit for bit
  paged_decode_attn       vs torch scaled_dot_product_attention in float64 on gathered KV
  sdpa_mlx_f32            vs float64 within fp32 bounds; n = 1 gives v[0]; one-pass/two-pass routing
                          and the bf16 partials of the two-pass form (it is only an error yardstick)
  embed_q4                vs torch's own bf16 multiply and add (a library routine), q = 0 rows = bias
  argmax_rows             vs numpy argmax (first index of the maximum) on NaN-free rows
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

from . import build as _build

_LIB = None

_P = ctypes.c_void_p
_I = ctypes.c_int


def lib():
    """The loaded oracle library, built on first use if it is missing."""
    global _LIB
    if _LIB is None:
        path = _build.LIB
        if not os.path.exists(path):
            _build.build()
        _LIB = ctypes.CDLL(path)
        _LIB.jo_exp_neg.restype = ctypes.c_float
        _LIB.jo_exp_neg.argtypes = [ctypes.c_float]
        _LIB.jo_bf2f.restype = ctypes.c_float
        _LIB.jo_bf2f.argtypes = [ctypes.c_uint16]
        _LIB.jo_f2bf.restype = ctypes.c_uint16
        _LIB.jo_f2bf.argtypes = [ctypes.c_float]
        _LIB.jo_swiglu_bf16.restype = ctypes.c_uint16
        _LIB.jo_swiglu_bf16.argtypes = [ctypes.c_uint16, ctypes.c_uint16]
        _LIB.jo_paged_decode_attn.argtypes = [_P, _P, _P, _I, _P, _I, _I, _I, _I, ctypes.c_float, _P, _P]
        _LIB.jo_sdpa_mlx_f32.argtypes = [_P, _P, _P, _I, _P, _I, _I, _I, _I, ctypes.c_float, _P, _P]
        _LIB.jo_exp_pos.restype = ctypes.c_float
        _LIB.jo_exp_pos.argtypes = [ctypes.c_float]
        _LIB.jo_num_threads.restype = _I
        _LIB.jo_log_ge1.restype = ctypes.c_float
        _LIB.jo_log_ge1.argtypes = [ctypes.c_float]
        _LIB.jo_fix42_to_bf16.restype = ctypes.c_float
        _LIB.jo_fix42_to_bf16.argtypes = [ctypes.c_uint64]
        _LIB.jo_sample_rows.argtypes = [_P, _I, _I, ctypes.c_double, ctypes.c_double, _I, _P, _P, _P]
        _LIB.jo_threefry2x32.argtypes = [_P, _P, _P]
        _LIB.jo_threefry2x32.restype = None
        _LIB.jo_threefry_uniform.argtypes = [_P, _I, _P]
        _LIB.jo_threefry_uniform.restype = None
    return _LIB


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _check(rc: int, name: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {name} rejected its arguments (rc={rc})")


def _u16(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint16)


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint32)


# ----------------------------------------------------------------------------- bf16 helpers
def f32_to_bf16(x) -> np.ndarray:
    """Round float32 values to bf16 bit patterns (nearest-even), as the oracle and kernels do."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    with np.errstate(over="ignore"):  # only NaN patterns wrap, and those are replaced below
        r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    if nan.any():
        r = np.where(nan, ((u >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16), r)
    return r


def bf16_to_f32(h) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def num_threads() -> int:
    return int(lib().jo_num_threads())


def set_num_threads(n: int) -> None:
    lib().jo_set_num_threads(int(n))


def exp_neg(x: float) -> float:
    return float(lib().jo_exp_neg(float(x)))


def exp_pos(x: float) -> float:
    return float(lib().jo_exp_pos(float(x)))


def sigmoid_bf16(g) -> np.ndarray:
    """SigmoidX on bf16 g (any shape), each step rounded to bf16 (Q36/kernels/expert_solo.py:56-62)."""
    g = _u16(g)
    out = np.empty_like(g)
    _check(lib().jo_sigmoid_bf16_n(_p(g), int(g.size), _p(out)), "sigmoid_bf16")
    return out


def swiglu_bf16(g: int, u: int) -> int:
    return int(lib().jo_swiglu_bf16(int(g), int(u)))


# ----------------------------------------------------------------------------- router
def softmax_bf16(logits) -> np.ndarray:
    lg = _u16(logits)
    rows, n = lg.reshape(-1, lg.shape[-1]).shape
    g = np.empty_like(lg)
    _check(lib().jo_softmax_bf16(_p(lg), rows, n, _p(g)), "softmax_bf16")
    return g


def topk_from_gates(gates, k: int) -> np.ndarray:
    g = _u16(gates)
    n = g.shape[-1]
    rows = g.size // n
    out = np.empty((*g.shape[:-1], k), dtype=np.uint32)
    _check(lib().jo_topk_from_gates(_p(g), rows, n, int(k), _p(out)), "topk_from_gates")
    return out


def router_topk(logits, k: int, norm: bool):
    """(inds uint32 [..., k], scores bf16 [..., k], gates bf16 [..., N])."""
    lg = _u16(logits)
    n = lg.shape[-1]
    rows = lg.size // n
    inds = np.empty((*lg.shape[:-1], k), dtype=np.uint32)
    scores = np.empty((*lg.shape[:-1], k), dtype=np.uint16)
    gates = np.empty_like(lg)
    _check(
        lib().jo_router_topk(_p(lg), rows, n, int(k), int(bool(norm)), _p(inds), _p(scores), _p(gates)),
        "router_topk",
    )
    return inds, scores, gates


# ----------------------------------------------------------------------------- packing
def moe_pack(inds, n_experts: int) -> dict:
    """Packing tables of the flat (row, slot) pairs of inds [B, k] (see jit_oracle.c)."""
    ind = _u32(inds)
    k = ind.shape[-1]
    P = ind.size
    E = int(n_experts)
    out = {
        "order": np.empty(P, np.int32),
        "pair_row": np.empty(P, np.int32),
        "inv": np.empty(P, np.int32),
        "expert_cnt": np.empty(E, np.int32),
        "expert_off": np.empty(E, np.int32),
        "seg_expert": np.zeros(E, np.int32),
        "seg_start": np.zeros(E, np.int32),
        "seg_cnt": np.zeros(E, np.int32),
        "meta": np.zeros(2, np.int32),
    }
    _check(
        lib().jo_moe_pack(
            _p(ind), P, k, E, _p(out["order"]), _p(out["pair_row"]), _p(out["inv"]),
            _p(out["expert_cnt"]), _p(out["expert_off"]), _p(out["seg_expert"]),
            _p(out["seg_start"]), _p(out["seg_cnt"]), _p(out["meta"]),
        ),
        "moe_pack",
    )
    return out


# ----------------------------------------------------------------------------- quantized maths
def dequant4(w, s, b, bf16w: bool = False) -> np.ndarray:
    """[N, K] float64 weights s * q + b; with bf16w the segment GEMM's bf16(fma(s, q, b))."""
    w, s, b = _u32(w), _u16(s), _u16(b)
    N, K = w.shape[0], w.shape[1] * 8
    out = np.empty((N, K), np.float64)
    _check(lib().jo_dequant4(_p(w), _p(s), _p(b), N, K, int(bf16w), _p(out)), "dequant4")
    return out


def q4_prepack(w, s, b) -> np.ndarray:
    """The packed tile layout (uint8) of a stack w [E, N, K/8] (or a matrix [N, K/8])."""
    w, s, b = _u32(w), _u16(s), _u16(b)
    if w.ndim == 2:
        w, s, b = w[None], s[None], b[None]
    E, N, K = w.shape[0], w.shape[1], w.shape[2] * 8
    out = np.empty(E * (N // 16) * (K // 128) * 1152, np.uint8)
    _check(lib().jo_q4_prepack(_p(w), _p(s), _p(b), E, N, K, _p(out)), "q4_prepack")
    return out


def qmm(x, w, s, b):
    """x [T, K] bf16 against one [N, K] quantized matrix -> (float64 [T, N], bf16 [T, N])."""
    x, w, s, b = _u16(x), _u32(w), _u16(s), _u16(b)
    T, K = x.shape
    N = w.shape[0]
    f = np.empty((T, N), np.float64)
    h = np.empty((T, N), np.uint16)
    _check(lib().jo_qmm(_p(x), T, _p(w), _p(s), _p(b), N, K, _p(f), _p(h)), "qmm")
    return f, h


def qmv_mlx_f32(x, w, s, b) -> np.ndarray:
    x, w, s, b = _u16(x), _u32(w), _u16(s), _u16(b)
    T, K = x.shape
    N = w.shape[0]
    out = np.empty((T, N), np.float32)
    _check(lib().jo_qmv_mlx_f32(_p(x), T, _p(w), _p(s), _p(b), N, K, _p(out)), "qmv_mlx_f32")
    return out


# ----------------------------------------------------------------------------- experts
def moe_gate_up(x, inds, pack: dict, w, s, b, bf16w: bool = False) -> np.ndarray:
    """h [P, I] bf16 in sorted pair order; w [E, 2I, D/8], s/b [E, 2I, D/64]; bf16w: the segment
    GEMM's bf16 weights."""
    x, ind, w, s, b = _u16(x), _u32(inds), _u32(w), _u16(s), _u16(b)
    B, D = x.shape
    E, two_i = w.shape[0], w.shape[1]
    P = ind.size
    h = np.empty((P, two_i // 2), np.uint16)
    _check(
        lib().jo_moe_gate_up(
            _p(x), B, D, _p(ind), P, _p(pack["order"]), _p(pack["pair_row"]), _p(w), _p(s), _p(b),
            E, two_i // 2, int(bf16w), _p(h),
        ),
        "moe_gate_up",
    )
    return h


def moe_down(h, inds, pack: dict, w, s, b, bf16w: bool = False) -> np.ndarray:
    """r [P, D] bf16 in sorted pair order; w [E, D, I/8], s/b [E, D, I/64]; bf16w as in moe_gate_up."""
    h, ind, w, s, b = _u16(h), _u32(inds), _u32(w), _u16(s), _u16(b)
    P, I = h.shape
    E, D = w.shape[0], w.shape[1]
    r = np.empty((P, D), np.uint16)
    _check(
        lib().jo_moe_down(_p(h), P, I, _p(ind), _p(pack["order"]), _p(w), _p(s), _p(b), E, D, int(bf16w), _p(r)),
        "moe_down",
    )
    return r


def moe_combine(r, inv, scores) -> np.ndarray:
    r, inv, sc = _u16(r), _i32(inv), _u16(scores)
    B, k = sc.shape
    D = r.shape[1]
    y = np.empty((B, D), np.uint16)
    _check(lib().jo_moe_combine(_p(r), _p(inv), _p(sc), B, k, D, _p(y)), "moe_combine")
    return y


def moe_experts(x, inds, scores, gu: tuple, dn: tuple, n_experts: int) -> dict:
    """The whole routed-expert chain for given routing: pack -> gate_up -> down -> combine."""
    pack = moe_pack(inds, n_experts)
    h = moe_gate_up(x, inds, pack, *gu)
    r = moe_down(h, inds, pack, *dn)
    y = moe_combine(r, pack["inv"], scores)
    return {"pack": pack, "h": h, "r": r, "y": y}


# ----------------------------------------------------------------------------- decoder block
def rmsnorm(x, w, eps: float, resid=None):
    """(y, h): y = bf16(w * bf16(x * rsqrt(mean(x^2) + eps))) of h = x (+ resid)."""
    x, w = _u16(x), _u16(w)
    rows, D = x.shape
    y = np.empty_like(x)
    h = np.empty_like(x) if resid is not None else None
    rs = _u16(resid) if resid is not None else None
    lib().jo_rmsnorm.argtypes = [_P, _P, _I, _I, _P, ctypes.c_float, _P, _P]
    _check(lib().jo_rmsnorm(_p(x), _p(rs) if rs is not None else None, rows, D, _p(w), float(eps),
                            _p(h) if h is not None else None, _p(y)), "rmsnorm")
    return y, (h if h is not None else x)


def qk_norm_rope_append(qkv, H: int, Hkv: int, qn, kn, eps: float, inv_freq, pos, pool, page_table):
    """q [B, H, 128] bf16; writes k, v into pool (in place) at positions pos."""
    qkv, qn, kn = _u16(qkv), _u16(qn), _u16(kn)
    invf = np.ascontiguousarray(inv_freq, dtype=np.float32)
    ps, pt = _i32(pos), _i32(page_table)
    assert pool.flags["C_CONTIGUOUS"] and pool.dtype == np.uint16
    B = qkv.shape[0]
    q = np.empty((B, H, 128), np.uint16)
    lib().jo_qk_norm_rope_append.argtypes = [_P, _I, _I, _I, _P, _P, ctypes.c_float, _P, _P, _P, _I, _I, _P, _P]
    _check(lib().jo_qk_norm_rope_append(_p(qkv), B, H, Hkv, _p(qn), _p(kn), float(eps), _p(invf), _p(ps), _p(pt),
                                        pt.shape[1], pool.shape[0], _p(pool), _p(q)), "qk_norm_rope_append")
    return q


def decoder_layer(x, layer: dict, pool, page_table, pos, cfg: dict, routing=None) -> dict:
    """One decoder layer of the BASELINE geometry for rows x [B, D] (the reference's layer step,
    Q36/model/model.py:77-80 with Qwen3_5MoeAttention.step and the MoE block): input RMSNorm ->
    qkv -> q/k norm + RoPE + KV append -> attention over pos + 1 keys -> o_proj -> residual ->
    post-attention RMSNorm -> router -> experts -> combine + residual.  `layer` holds numpy
    weights (quantized ones as (w, s, b) triples); `pool` is updated in place.  `routing`
    (inds, scores) overrides the router's choice (used to compare against another
    implementation's routing).  Returns every intermediate."""
    H, Hkv, E, k = cfg["heads"], cfg["kv_heads"], cfg["experts"], cfg["top_k"]
    eps = cfg["eps"]
    xn, _ = rmsnorm(x, layer["input_norm"], eps)
    _, qkv = qmm(xn, *layer["qkv"])
    q = qk_norm_rope_append(qkv, H, Hkv, layer["q_norm"], layer["k_norm"], eps, cfg["inv_freq"], pos, pool, page_table)
    lens = np.asarray(pos, np.int64) + 1
    attn = paged_decode_attn(q, pool, page_table, lens, 128 ** -0.5)
    _, o = qmm(attn.reshape(x.shape[0], -1), *layer["o"])
    hn, h = rmsnorm(o, layer["post_norm"], eps, resid=x)
    _, logits = qmm(hn, *layer["router"])
    inds, scores, _ = router_topk(logits, k, True)
    if routing is not None:
        inds, scores = routing
    ex = moe_experts(hn, inds, scores, layer["gate_up"], layer["down"], E)
    y = f32_to_bf16(bf16_to_f32(h) + bf16_to_f32(ex["y"]))
    return {"xn": xn, "qkv": qkv, "q": q, "attn": attn, "o": o, "h": h, "hn": hn, "logits": logits,
            "inds": inds, "scores": scores, "y": y}


def decoder_layer_mlx_f32(x, layer: dict, pool, page_table, pos, cfg: dict) -> np.ndarray:
    """decoder_layer in the reference's own fp32 arithmetic (the MLX CPU op chain this build's CPU
    baseline times): the projections in MLX qmv's per-lane fp32 order (qmv_mlx_f32) rounded to
    bf16, attention as MLX's sdpa_vector / two-pass kernels (sdpa_mlx_f32), every expert pair's
    gate/up/down by qmv_mlx_f32 with the SigmoidX bf16 chain, and the slot-order bf16 combine.
    Returns the layer output y [B, D] bf16; `pool` is updated in place (the KV append)."""
    H, Hkv, E, k, eps = cfg["heads"], cfg["kv_heads"], cfg["experts"], cfg["top_k"], cfg["eps"]
    B = x.shape[0]
    xn, _ = rmsnorm(x, layer["input_norm"], eps)
    qkv = f32_to_bf16(qmv_mlx_f32(xn, *layer["qkv"]))
    q = qk_norm_rope_append(qkv, H, Hkv, layer["q_norm"], layer["k_norm"], eps, cfg["inv_freq"], pos, pool, page_table)
    attn, _ = sdpa_mlx_f32(q, pool, page_table, np.asarray(pos, np.int64) + 1, 128 ** -0.5)
    o = f32_to_bf16(qmv_mlx_f32(attn.reshape(B, -1), *layer["o"]))
    hn, h = rmsnorm(o, layer["post_norm"], eps, resid=x)
    logits = f32_to_bf16(qmv_mlx_f32(hn, *layer["router"]))
    inds, scores, _ = router_topk(logits, k, True)
    gw, gs, gb = layer["gate_up"]
    dw, ds, db = layer["down"]
    I = gw.shape[1] // 2
    r = np.zeros((B, k, hn.shape[1]), np.uint16)
    for e in np.unique(inds):
        rows, slots = np.nonzero(inds == e)
        gu = f32_to_bf16(qmv_mlx_f32(hn[rows], gw[e], gs[e], gb[e]))
        g, u = gu[:, :I], gu[:, I:]
        with np.errstate(over="ignore", invalid="ignore"):
            sl = f32_to_bf16(bf16_to_f32(g) * bf16_to_f32(sigmoid_bf16(g)))
            hh = f32_to_bf16(bf16_to_f32(sl) * bf16_to_f32(u))
        r[rows, slots] = f32_to_bf16(qmv_mlx_f32(hh, dw[e], ds[e], db[e]))
    acc = np.zeros(hn.shape, np.float32)
    for j in range(k):
        p = bf16_to_f32(f32_to_bf16(bf16_to_f32(r[:, j]) * bf16_to_f32(scores[:, j:j + 1])))
        acc = bf16_to_f32(f32_to_bf16(acc + p))
    return f32_to_bf16(bf16_to_f32(h) + acc)


# ----------------------------------------------------------------------------- paged KV
PAGE = 16


def kv_append_paged(pool, k, v, pos, page_table) -> None:
    """In place: pool [num_pages, Hkv, 2, 16*Dh] bf16; k, v [B, Hkv, Dh]; pos [B]."""
    assert pool.flags["C_CONTIGUOUS"] and pool.dtype == np.uint16
    k, v, pos, pt = _u16(k), _u16(v), _i32(pos), _i32(page_table)
    B, Hkv, Dh = k.shape
    _check(
        lib().jo_kv_append_paged(
            _p(k), _p(v), B, Hkv, Dh, _p(pos), _p(pt), pt.shape[1], pool.shape[0], _p(pool)
        ),
        "kv_append_paged",
    )


def kv_gather(pool, page_row, n: int, Hkv: int, Dh: int):
    """Contiguous K, V [Hkv, n, Dh] of one sequence's first n tokens."""
    pr = _i32(page_row)
    kc = np.empty((Hkv, n, Dh), np.uint16)
    vc = np.empty((Hkv, n, Dh), np.uint16)
    _check(lib().jo_kv_gather(_p(_u16(pool)), Hkv, Dh, _p(pr), int(n), _p(kc), _p(vc)), "kv_gather")
    return kc, vc


def paged_prefill_attn(q, pool, page_table, chunks, scale: float, exact: bool = False):
    """Causal attention of prefill chunks: q [T, H, Dh] bf16 holds the chunks' rows in order; chunk
    (seq, ctx, length) owns the next `length` rows, and its token t (position ctx + t of sequence
    seq) attends keys 0 .. ctx + t of page_table[seq] -- decode attention of that token over
    ctx + t + 1 keys (the causal mask of mx.fast.scaled_dot_product_attention, aligned to the last
    key), so this is paged_decode_attn row by row.  exact=True also returns the float64 values."""
    pt = _i32(page_table)
    lens, rows = [], []
    for seq, ctx, length in chunks:
        for t in range(length):
            lens.append(ctx + t + 1)
            rows.append(pt[seq])
    if not lens:
        e = np.empty_like(_u16(q))
        return (e, e.astype(np.float64)) if exact else e
    return paged_decode_attn(q, pool, np.stack(rows), np.array(lens, np.int32), scale, exact=exact)


def paged_decode_attn(q, pool, page_table, lens, scale: float, exact: bool = False):
    """q [B, H, Dh] bf16 -> out [B, H, Dh] bf16 (float64 softmax attention over lens[b] tokens);
    with exact=True also the float64 values before the bf16 rounding: (out, out64)."""
    q, pool, pt, ln = _u16(q), _u16(pool), _i32(page_table), _i32(lens)
    B, H, Dh = q.shape
    Hkv = pool.shape[1]
    out = np.empty_like(q)
    out64 = np.empty(q.shape, np.float64) if exact else None
    _check(
        lib().jo_paged_decode_attn(
            _p(q), _p(pool), _p(pt), pt.shape[1], _p(ln), B, H, Hkv, Dh, float(scale), _p(out),
            None if out64 is None else _p(out64),
        ),
        "paged_decode_attn",
    )
    return (out, out64) if exact else out


def sdpa_mlx_f32(q, pool, page_table, lens, scale: float):
    """The reference's stock decode attention in MLX's fp32 arithmetic (one-pass sdpa_vector, or the
    two-pass kernels with bf16 partials, routed as on the reference's M4 Pro): (out bf16, out fp32)."""
    q, pool, pt, ln = _u16(q), _u16(pool), _i32(page_table), _i32(lens)
    B, H, Dh = q.shape
    Hkv = pool.shape[1]
    out = np.empty_like(q)
    f32 = np.empty(q.shape, np.float32)
    _check(
        lib().jo_sdpa_mlx_f32(
            _p(q), _p(pool), _p(pt), pt.shape[1], _p(ln), B, H, Hkv, Dh, float(scale), _p(out), _p(f32)
        ),
        "sdpa_mlx_f32",
    )
    return out, f32


def embed_q4(ids, w, s, b) -> np.ndarray:
    """bf16 rows [B, D] of an MLX 4-bit table: mx.dequantize of the gathered rows
    (Q36/linear.py:680-690) in bf16 arithmetic, bf16(bf16(scale * q) + bias) per value; an id
    outside [0, V) gives a zero row."""
    ids = np.asarray(ids, np.int64)
    w, s, b = _u32(w), _u16(s), _u16(b)
    V, D = w.shape[0], w.shape[1] * 8
    out = np.zeros((ids.size, D), np.uint16)
    ok = (ids >= 0) & (ids < V)
    if ok.any():
        rows = ids[ok]
        q = ((w[rows][:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15).reshape(rows.size, D)
        sc = np.repeat(bf16_to_f32(s[rows]), 64, axis=1)
        bi = np.repeat(bf16_to_f32(b[rows]), 64, axis=1)
        sq = bf16_to_f32(f32_to_bf16((sc * q.astype(np.float32)).astype(np.float32)))
        out[ok] = f32_to_bf16((sq + bi).astype(np.float32))
    return out


def log_ge1(s: float) -> float:
    """ln s for s >= 1 (the build's own fp32 sequence, shared with the GPU)."""
    return float(lib().jo_log_ge1(ctypes.c_float(s)))


def fix42_to_bf16(c: int) -> float:
    """c 2^-42 rounded once (nearest even) to bf16."""
    return float(lib().jo_fix42_to_bf16(ctypes.c_uint64(c)))


def logprobs_rows(logits) -> np.ndarray:
    """bf16 [B, V]: lp = bf16(x - lse), lse = bf16(m0 + ln(S 2^-42)), S = sum floor(e^(x - m0)
    2^42) (logprobs_from_logits, Q36/sampler.py:295-297)."""
    x = np.ascontiguousarray(_u16(logits))
    B, V = x.shape
    out = np.empty_like(x)
    _check(lib().jo_logprobs_rows(_p(x), B, V, _p(out)), "logprobs_rows")
    return out


def sample_rows(logits, temperature: float, top_p: float, top_k: int, u=None, weights: bool = False):
    """int32 [B]: Sampler._sample_exact_full's draw per row (Q36/sampler.py:451-476) given fp32
    uniforms u [B]; temperature <= 0 is the greedy draw (the first index of the largest lp).
    weights=True also returns the rows' integer weights W [B, V] (uint64, 2^42-scaled)."""
    x = np.ascontiguousarray(_u16(logits))
    B, V = x.shape
    uu = np.zeros(B, np.float32) if u is None else np.ascontiguousarray(np.asarray(u, np.float32))
    out = np.zeros(B, np.int32)
    w = np.zeros((B, V), np.uint64) if weights else None
    _check(lib().jo_sample_rows(_p(x), B, V, float(temperature), float(top_p), int(top_k), _p(uu), _p(out),
                                _p(w) if weights else None), "sample_rows")
    return (out, w) if weights else out


def argmax_rows(logits) -> np.ndarray:
    """int32 [B]: the greedy draw, the first index of each row's largest log-probability
    (Sampler.__call__ with temperature 0, Q36/sampler.py:371-374)."""
    return sample_rows(logits, 0.0, 1.0, 0)


def threefry2x32(key, ctr) -> tuple:
    """Threefry-2x32-20 of one counter pair under one key pair (uint32 values)."""
    k = np.asarray(key, np.uint32)
    c = np.asarray(ctr, np.uint32)
    out = np.zeros(2, np.uint32)
    lib().jo_threefry2x32(_p(k), _p(c), _p(out))
    return int(out[0]), int(out[1])


def threefry_uniform(keys) -> np.ndarray:
    """fp32 [B]: min(fp32(threefry(key, (0, 0))[0]) / 2^32, 1 - 2^-24) per key pair [B, 2]."""
    k = np.ascontiguousarray(np.asarray(keys, np.uint32).reshape(-1, 2))
    out = np.zeros(k.shape[0], np.float32)
    lib().jo_threefry_uniform(_p(k), k.shape[0], _p(out))
    return out