"""jitengine_amd: MI355X (gfx950) implementation of JITEngine's ragged-batch MoE decode step.

Router top-k, token-to-expert packing, 4-bit (MLX affine, group 64) expert projections and paged
GQA decode attention run as hand-written HIP kernels behind one C-ABI library
(include/jit_moe.h, built into jitengine_amd/_lib/libjit_moe.so); this package is the Python
surface that calls it from PyTorch-ROCm.
"""

from .quant import QLinear, quantize4, random_quantized  # noqa: F401

__all__ = ["QLinear", "quantize4", "random_quantized"]
