"""The MLX 4-bit affine quantized layout and the build's quantizer.

Layout (Q36/linear.py:101-128, FN/kernels/qmv_row_blocked.py:23-33): a matrix [N, K] is stored as
`weight` uint32 [N, K/8] (element j of row n is nibble j % 8 of word j / 8, low nibble first),
`scales` and `biases` bf16 [N, K/64], and w = scale * q + bias.  An expert stack prepends an
expert axis.  Gate and up projections of the experts are fused along the output axis as one
[E, 2I, K] stack, gate rows first (Q36/model/moe.py:70-74, Q36/linear.py:543-560).

Packed words are held in int32 tensors (the same 32 bits as MLX's uint32).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

GROUP = 64


@dataclass
class QLinear:
    """A quantized matrix or expert stack: weight int32 [..., N, K/8], scales/biases bf16
    [..., N, K/64].  Mirrors QLinear / _Stack (Q36/linear.py:101-128,
    Q36/kernels/expert_solo.py:404-421): bits and dims are inferred from the shapes."""

    weight: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor
    group_size: int = GROUP

    @property
    def in_dims(self) -> int:
        return self.scales.shape[-1] * self.group_size

    @property
    def out_dims(self) -> int:
        return self.weight.shape[-2]

    @property
    def bits(self) -> int:
        return self.weight.shape[-1] * 32 // self.in_dims

    @property
    def num_experts(self) -> int:
        return self.weight.shape[0] if self.weight.dim() == 3 else 1

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.weight, self.scales, self.biases))

    def to(self, device) -> "QLinear":
        return QLinear(
            self.weight.to(device), self.scales.to(device), self.biases.to(device), self.group_size
        )

    def validate(self) -> None:
        """Raise ValueError unless this is a 4-bit group-64 tensor set the kernels take."""
        if self.group_size != GROUP or self.bits != 4:
            raise ValueError(f"4-bit group-64 weights required, got bits={self.bits} group={self.group_size}")
        if self.weight.dtype != torch.int32 or self.scales.dtype != torch.bfloat16 or self.biases.dtype != torch.bfloat16:
            raise ValueError("weight must be int32 (packed nibbles) and scales/biases bf16")
        if self.scales.shape != self.biases.shape or self.scales.shape[:-1] != self.weight.shape[:-1]:
            raise ValueError("scales/biases must be [..., N, K/64] matching weight [..., N, K/8]")
        for t in (self.weight, self.scales, self.biases):
            if not t.is_contiguous():
                raise ValueError("quantized tensors must be contiguous")


def quantize4(w: torch.Tensor, group_size: int = GROUP) -> QLinear:
    """Affine 4-bit quantization of float weights [..., N, K] into the MLX layout.

    Per group of 64: scale = (max - min) / 15 and bias = min, both rounded to bf16; then
    q = clip(round((w - bias) / scale), 0, 15) against the rounded scale and bias.  Runs on the
    tensor's device.  (MLX's own quantizer places its grid slightly differently; parity never
    depends on it because every consumer reads the same packed bytes.)
    """
    if w.shape[-1] % group_size:
        raise ValueError(f"K = {w.shape[-1]} is not a multiple of {group_size}")
    *lead, N, K = w.shape
    g = w.float().reshape(*lead, N, K // group_size, group_size)
    mn = g.amin(-1)
    mx = g.amax(-1)
    scale = ((mx - mn) / 15.0).clamp_min(1e-8)
    s_bf = scale.to(torch.bfloat16)
    b_bf = mn.to(torch.bfloat16)
    q = torch.round((g - b_bf.float()[..., None]) / s_bf.float()[..., None]).clamp_(0, 15)
    del g
    q = q.to(torch.int64).reshape(*lead, N, K // 8, 8)
    shifts = torch.arange(8, device=w.device, dtype=torch.int64) * 4
    words = (q << shifts).sum(-1)
    del q
    words = torch.where(words >= 2**31, words - 2**32, words).to(torch.int32)
    return QLinear(words.contiguous(), s_bf.contiguous(), b_bf.contiguous(), group_size)


def dequantize4(q: QLinear) -> torch.Tensor:
    """float32 [..., N, K] values of a quantized tensor set (torch ops; used by tooling/tests)."""
    w = q.weight.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(8, device=w.device, dtype=torch.int64) * 4
    nib = ((w[..., None] >> shifts) & 0xF).reshape(*w.shape[:-1], w.shape[-1] * 8).float()
    s = q.scales.float().repeat_interleave(q.group_size, dim=-1)
    b = q.biases.float().repeat_interleave(q.group_size, dim=-1)
    return s * nib + b


def random_quantized(shape, seed: int, std: float = 0.02, device="cpu") -> QLinear:
    """N(0, std) weights of `shape` [..., N, K], rounded to bf16 and quantized (the configs'
    synthetic weights).  Seeded; generated on `device`."""
    gen = torch.Generator(device=device)
    gen.manual_seed(int(seed))
    w = torch.randn(*shape, generator=gen, device=device, dtype=torch.float32) * std
    w = w.to(torch.bfloat16).float()
    return quantize4(w)
