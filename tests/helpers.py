"""Shared data generators and conversions for the tests (numpy uint16 = bf16 bit patterns)."""

from __future__ import annotations

import numpy as np
import torch

import oracle
from jitengine_amd.quant import QLinear, random_quantized
from oracle import bf16_to_f32, f32_to_bf16  # noqa: F401


def u16(t: torch.Tensor) -> np.ndarray:
    """bf16 torch tensor -> numpy uint16 bit patterns (on the host)."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def bf16_tensor(a: np.ndarray, device="cpu") -> torch.Tensor:
    """numpy uint16 bit patterns -> bf16 torch tensor."""
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).view(torch.bfloat16).to(device)


def normal_bf16(shape, seed: int, scale: float = 1.0) -> np.ndarray:
    """N(0, scale^2) values rounded to bf16 (drawn in float32: pools of 10^8 values stay quick)."""
    rng = np.random.default_rng(seed)
    out = np.empty(shape, np.uint16)
    flat = out.reshape(-1)
    buf = np.empty(min(flat.size, 1 << 21), np.float32)  # drawn in chunks: large pools touch little fresh memory
    for i in range(0, flat.size, buf.size):
        b = buf[:min(buf.size, flat.size - i)]
        rng.standard_normal(out=b, dtype=np.float32)
        if scale != 1.0:
            b *= np.float32(scale)
        flat[i:i + b.size] = f32_to_bf16(b)
    return out


def stack_np(q: QLinear):
    """(w uint32, s uint16, b uint16) numpy views of a CPU QLinear for the oracle."""
    w = q.weight.contiguous().numpy().view(np.uint32)
    s = q.scales.contiguous().view(torch.int16).numpy().view(np.uint16)
    b = q.biases.contiguous().view(torch.int16).numpy().view(np.uint16)
    return w, s, b


def make_stack(shape, seed: int) -> QLinear:
    return random_quantized(shape, seed)


def router_logits(kind: int, B: int, N: int, seed: int) -> np.ndarray:
    """The reference's router draws (Q36/kernels/router_topk.py:212-231): normal logits scaled by
    2, 8, 0.05, or integers in [-4, 4) (kind 2), all rounded to bf16."""
    rng = np.random.default_rng(seed)
    if kind % 4 == 2:
        lg = rng.integers(-4, 4, (B, N)).astype(np.float32)
    else:
        lg = rng.standard_normal((B, N)).astype(np.float32) * (2.0, 8.0, 1.0, 0.05)[kind % 4]
    return f32_to_bf16(lg)


def tie_gates(B: int, N: int, seed: int) -> np.ndarray:
    """Tie-heavy bf16 gates: softmax of integer-valued logits randint(0, 5) * 0.5
    (Q36T/metal/kernels/test_router_topk.py:6-21, every third draw)."""
    import oracle

    rng = np.random.default_rng(seed)
    lg = f32_to_bf16((rng.integers(0, 5, (B, N)) * 0.5).astype(np.float32))
    return oracle.softmax_bf16(lg)


def cosine(a: np.ndarray, b: np.ndarray) -> float:
    a = a.astype(np.float64).ravel()
    b = b.astype(np.float64).ravel()
    den = np.linalg.norm(a) * np.linalg.norm(b)
    return float(a @ b / den) if den else 1.0


def bf16_ulp(v: np.ndarray) -> np.ndarray:
    """One bf16 ulp at each value (2^(e - 7) for |v| in [2^e, 2^(e+1)))."""
    a = np.maximum(np.abs(v.astype(np.float64)), 2.0**-126)
    return 2.0 ** (np.floor(np.log2(a)) - 7)


def assert_close_bf16(got_u16: np.ndarray, want_u16: np.ndarray, max_abs: float = 2e-2, min_cos: float = 0.9995,
                      what: str = "", ulps: float = 2.0) -> dict:
    """The north-star float tolerance on bf16 outputs: every element within max(2e-2, `ulps` bf16
    ulps of the expected value) -- the absolute 2e-2 of the north star, widened to two ulps where
    values exceed |4| and one ulp alone is larger than 2e-2 -- and cosine >= 0.9995."""
    g = bf16_to_f32(got_u16).astype(np.float64)
    w = bf16_to_f32(want_u16).astype(np.float64)
    assert g.shape == w.shape, (g.shape, w.shape)
    assert np.all(np.isfinite(g)), f"{what}: non-finite outputs"
    diff = np.abs(g - w)
    bound = np.maximum(max_abs, ulps * bf16_ulp(w))
    err = float(diff.max()) if g.size else 0.0
    cos = cosine(g, w)
    exact = float(np.mean(got_u16 == want_u16)) if g.size else 1.0
    worst = float((diff / bound).max()) if g.size else 0.0
    assert worst <= 1.0, f"{what}: error {err:.3g} exceeds max({max_abs}, {ulps} ulp) (worst ratio {worst:.2f})"
    assert cos >= min_cos, f"{what}: cosine {cos:.6f} < {min_cos}"
    return {"max_abs": err, "cos": cos, "bit_equal": exact}


def assert_attention_parity(got_u16: np.ndarray, exact: np.ndarray, stock_u16: np.ndarray | None = None,
                            what: str = "", min_equal: float = 0.98, rel: float = 2.0**-14) -> dict:
    """The attention bar, on outputs [S, ..., Dh] (S = sequences or token rows, each checked alone):

    1. the reference's own criterion (FN/kernels/selfcheck.py:313-331), when `stock_u16` (the
       reference's fp32 arithmetic, oracle.sdpa_mlx_f32) is given: per sequence,
       max|got - exact| <= 8 max|stock - exact| + 4 * 2^-24 * max|exact|;
    2. every element within one bf16 ulp of the exact (float64) value plus `rel` of its row's
       largest |exact| (an fp32-accurate kernel's error is ~2^-18 of the row; one bf16-rounded P
       alone moves elements by ~2^-9 of the row);
    3. per sequence, at least `min_equal` of the elements equal the correctly rounded result
       bf16(exact) bit for bit.
    2 and 3 scale with each row's own magnitude, so they fail when a page is dropped or read from
    the wrong place at any context length (tests/test_attention_bar.py plants those mistakes in the
    oracle and checks that this bar rejects them)."""
    g = bf16_to_f32(got_u16).astype(np.float64)
    e = np.asarray(exact, np.float64)
    assert g.shape == e.shape, (g.shape, e.shape)
    assert np.all(np.isfinite(g)), f"{what}: non-finite outputs"
    S = g.shape[0]
    gs, es = g.reshape(S, -1, g.shape[-1]), e.reshape(S, -1, e.shape[-1])
    cr = f32_to_bf16(es.astype(np.float32))
    rowmax = np.abs(es).max(-1, keepdims=True)
    bound = bf16_ulp(es) + rel * rowmax
    ratio = np.abs(gs - es) / bound
    worst = float(ratio.max()) if g.size else 0.0
    if worst > 1.0:
        s, r, d = np.unravel_index(int(ratio.argmax()), ratio.shape)
        raise AssertionError(f"{what}: sequence {s} row {r} dim {d}: {gs[s, r, d]:.6g} against exact "
                             f"{es[s, r, d]:.6g} (bound {bound[s, r, d]:.3g}, worst ratio {worst:.2f})")
    eq = np.mean(f32_to_bf16(gs.astype(np.float32)) == cr, axis=(1, 2)) if g.size else np.ones(S)
    low = int(eq.argmin()) if S else 0
    assert S == 0 or eq.min() >= min_equal, (
        f"{what}: sequence {low}: {eq[low]:.4f} of the outputs equal the correctly rounded result "
        f"(floor {min_equal})")
    out = {"worst_ratio": worst, "min_equal": float(eq.min()) if S else 1.0, "mean_equal": float(eq.mean()) if S else 1.0}
    if stock_u16 is not None:
        st = bf16_to_f32(stock_u16).astype(np.float64).reshape(gs.shape)
        e_got = np.abs(gs - es).reshape(S, -1).max(1)
        e_stock = np.abs(st - es).reshape(S, -1).max(1)
        scale = np.abs(es).reshape(S, -1).max(1)
        lim = 8 * e_stock + 4 * 2.0**-24 * scale
        bad = np.flatnonzero(e_got > lim)
        assert bad.size == 0, (f"{what}: sequence {bad[0]}: error {e_got[bad[0]]:.3g} exceeds 8x the reference "
                               f"arithmetic's {e_stock[bad[0]]:.3g}")
        out["err_vs_stock"] = float((e_got / np.maximum(e_stock, 1e-300)).max())
    return out


def assert_fn_criterion(got_u16, x, w, s, b, f64) -> None:
    """The reference's criterion for a quantized projection (FN/kernels/selfcheck.py:313-331): the
    largest error of the result against the float64 product f64 is at most 8x that of the reference's
    own fp32 arithmetic (oracle.qmv_mlx_f32, rounded to bf16 as the reference returns it) plus 4 fp32
    ulps of the result's scale."""
    stock = f32_to_bf16(oracle.qmv_mlx_f32(x, w, s, b))
    e_got = np.abs(bf16_to_f32(got_u16) - f64).max()
    e_stock = np.abs(bf16_to_f32(stock) - f64).max()
    scale = np.abs(f64).max()
    assert e_stock <= 2.0**-6 * scale
    assert e_got <= 8 * e_stock + 4 * 2.0**-24 * scale, (e_got, e_stock)


def sampler_logits(kind: int, B: int, V: int, seed: int, scale: float = 1.0) -> np.ndarray:
    """bf16 [B, V] logit rows of the reference's sampler checks (Q36/sampler.py:546-604 and
    Q36T/metal/test_sampler.py): 0 normal * 3, 1 integers in [-3, 3) (heavy ties), 2 all equal,
    3 sparse spikes of 4, 4 three confident tokens (+30), 5 normal * 0.3, 6 normal * scale rounded
    to halves (ties), 7 normal * scale with a tenth of the entries at -inf."""
    rng = np.random.default_rng(seed)
    n = rng.standard_normal((B, V)).astype(np.float32)
    if kind == 0:
        x = n * 3
    elif kind == 1:
        x = rng.integers(-3, 3, (B, V)).astype(np.float32)
    elif kind == 2:
        x = np.zeros((B, V), np.float32)
    elif kind == 3:
        x = (rng.random((B, V)) < 0.001).astype(np.float32) * 4
    elif kind == 4:
        x = n + 30 * (np.arange(V) < 3)[None, :]
    elif kind == 5:
        x = n * 0.3
    elif kind == 6:
        x = np.round(n * scale * 2) / 2
    else:
        x = n * scale
        x[rng.random((B, V)) < 0.1] = -np.inf
    return f32_to_bf16(x.astype(np.float32))
