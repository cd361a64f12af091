"""Shared data generators and conversions for the tests (numpy uint16 = bf16 bit patterns)."""

from __future__ import annotations

import numpy as np
import torch

from jitengine_amd.quant import QLinear, random_quantized
from oracle import bf16_to_f32, f32_to_bf16  # noqa: F401


def u16(t: torch.Tensor) -> np.ndarray:
    """bf16 torch tensor -> numpy uint16 bit patterns (on the host)."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def bf16_tensor(a: np.ndarray, device="cpu") -> torch.Tensor:
    """numpy uint16 bit patterns -> bf16 torch tensor."""
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).view(torch.bfloat16).to(device)


def normal_bf16(shape, seed: int, scale: float = 1.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


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
