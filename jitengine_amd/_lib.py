"""Loader of the C-ABI library libjit_moe.so (include/jit_moe.h) through ctypes.

The library is the only compute path: if it is missing this module raises, it never falls back to
anything else.  Build it with `python -m jitengine_amd.build` (or `__graft_entry__.build()`).
"""

from __future__ import annotations

import ctypes
import os

from . import build as _build

JIT_OK = 0
JIT_EINVAL = -1
JIT_EUNSUPPORTED = -2
JIT_ELAUNCH = -3
JIT_ATTN_SCRATCH_BYTES = 16 << 20  # jit_paged_decode_attn_noalloc's partials limit

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float

# name -> argtypes (restype int unless listed in _RESTYPES)
_SIGNATURES = {
    "jit_last_error": [],
    "jit_version": [],
    "jit_router_topk": [_P, _I, _I, _I, _I, _P, _P, _P, _P],
    "jit_topk": [_P, _I, _I, _I, _P, _P],
    "jit_moe_pack": [_P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    "jit_moe_pack_workspace_bytes": [_I, _I],
    "jit_moe_pack_ws": [_P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, ctypes.c_int64, _P],
    "jit_route_pack": [_P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    "jit_q4_packed_bytes": [_I, _I, _I],
    "jit_q4_prepack": [_P, _P, _P, _I, _I, _I, _P, _P],
    "jit_qmm": [_P, _I, _I, _P, _P, _P, _I, _P, _P],
    "jit_qmm_packed": [_P, _I, _I, _P, _I, _P, _P],
    "jit_moe_gate_up_swiglu": [_P, _I, _P, _P, _P, _I, _P, _P, _P, _I, _I, _P, _P],
    "jit_moe_gate_up_swiglu_packed": [_P, _I, _P, _P, _P, _I, _P, _I, _I, _P, _P],
    "jit_moe_gate_up_swiglu_routed_packed": [_P, _I, _P, _I, _I, _I, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                             _P, _P, _P],
    "jit_swiglu": [_P, _P, ctypes.c_int64, _P, _P],
    "jit_moe_down": [_P, _I, _P, _P, _I, _P, _P, _P, _I, _I, _P, _P],
    "jit_moe_down_packed": [_P, _I, _P, _P, _I, _P, _I, _I, _P, _P],
    "jit_moe_gate_up_swiglu_seg": [_P, _I, _P, _P, _P, _I, _P, _I, _I, _P, _P],
    "jit_moe_down_seg": [_P, _I, _P, _P, _I, _P, _I, _I, _P, _P],
    "jit_qmm_seg": [_P, _I, _I, _P, _I, _P, _P],
    "jit_moe_combine": [_P, _P, _P, _I, _I, _I, _P, _P, _P],
    "jit_moe_combine_rmsnorm": [_P, _P, _P, _I, _I, _I, _P, _P, _P, _F, _P, _P],
    "jit_rmsnorm": [_P, _P, _I, _I, _P, _F, _P, _P, _P],
    "jit_qmm_packed_add_rmsnorm": [_P, _P, _P, _F, _I, _P, _I, _P, _P, _P, _P],
    "jit_qmm_packed_combine_rmsnorm": [_P, _P, _P, _I, _P, _P, _F, _I, _P, _I, _P, _P, _P],
    "jit_qk_norm_rope_append": [_P, _I, _I, _I, _P, _P, _F, _P, _P, _P, _I, _P, _P, _P],
    "jit_kv_append_paged": [_P, _P, _I, _I, _P, _P, _I, _P, _P],
    "jit_attn_chunk_tokens": [_I],
    "jit_attn_plan": [_P, _I, _P, _P, _I],
    "jit_attn_workspace_bytes": [_I, _I],
    "jit_paged_decode_attn": [_P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _F, _I, _P, _P, _P],
    "jit_paged_decode_attn_qkv": [_P, _P, _P, _F, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _F, _I, _P, _P, _P],
    "jit_paged_decode_attn_noalloc": [_P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _F, _I, _P, _P],
    "jit_prefill_block_tokens": [_I, _I],
    "jit_paged_prefill_attn": [_P, _P, _P, _I, _P, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P, _P, _P],
    "jit_prefill_part_keys": [],
    "jit_prefill_workspace_bytes": [_I, _I, _I],
    "jit_embed_q4": [_P, _I, _P, _P, _P, _I, _I, _P, _P],
    "jit_logprobs_rows": [_P, _I, _I, _P, _P],
    "jit_argmax_rows": [_P, _I, _I, _P, _P],
    "jit_sample_rows": [_P, _I, _I, ctypes.c_double, ctypes.c_double, _I, _P, _P, _P],
    "jit_threefry_uniform": [_P, _I, _P, _P],
    "jit_sampler_workspace_bytes": [],
    "jit_logprobs_rows_ws": [_P, _I, _I, _P, _P, ctypes.c_int64, _P],
    "jit_argmax_rows_ws": [_P, _I, _I, _P, _P, ctypes.c_int64, _P],
    "jit_sample_rows_ws": [_P, _I, _I, ctypes.c_double, ctypes.c_double, _I, _P, _P, _P, ctypes.c_int64, _P],
    "jit_kv_copy_pages": [_P, _I, _I, _P, _P, _I, _P],
}
_RESTYPES = {"jit_last_error": ctypes.c_char_p, "jit_attn_workspace_bytes": ctypes.c_int64,
             "jit_prefill_workspace_bytes": ctypes.c_int64,
             "jit_q4_packed_bytes": ctypes.c_int64, "jit_moe_pack_workspace_bytes": ctypes.c_int64,
             "jit_sampler_workspace_bytes": ctypes.c_int64}

_lib = None


class JitError(RuntimeError):
    """A HIP launch failure reported by the library."""


class UnsupportedShape(ValueError):
    """The shape is outside the kernel's coverage (where the reference takes its stock MLX op)."""


def library_path() -> str:
    return _build.LIB


def lib() -> ctypes.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        path = _build.LIB
        if not os.path.exists(path):
            raise RuntimeError(
                f"{path} is missing: the HIP extension is the only compute path; build it with "
                "`python -m jitengine_amd.build`"
            )
        h = ctypes.CDLL(path)
        for name, args in _SIGNATURES.items():
            fn = getattr(h, name)
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, _I)
        _lib = h
    return _lib


def exported_symbols() -> list:
    """The C-ABI entry points this module binds (each must exist in the library)."""
    return sorted(_SIGNATURES)


def check(rc: int, what: str) -> int:
    """Turn a negative status into the matching Python exception."""
    if rc >= 0:
        return rc
    msg = lib().jit_last_error().decode(errors="replace")
    if rc == JIT_EINVAL:
        raise ValueError(f"{what}: {msg}")
    if rc == JIT_EUNSUPPORTED:
        raise UnsupportedShape(f"{what}: {msg}")
    raise JitError(f"{what}: {msg} (status {rc})")
