"""Torch-facing operators of the hot path, each a thin call into the C-ABI (include/jit_moe.h).

Every function here mirrors a reference kernel entry point (named in its docstring) and calls the
HIP library on the current torch stream; contract breaks raise ValueError as the reference's do,
shapes outside the kernels' coverage raise UnsupportedShape.  There is no other compute path.
Tensors: bf16 as torch.bfloat16, packed 4-bit words and expert ids as torch.int32.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .quant import QLinear

PAGE = 16
HEAD_DIM = 128


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def upload(a, device, dtype=None) -> torch.Tensor:
    """A host array (numpy or list) as a device tensor without a host wait: staged in pinned host
    memory and copied asynchronously on the current stream (torch's caching host allocator keeps the
    staging block until the copy has run), so a step's small inputs can be queued while earlier steps
    still run.  A pageable copy would make the host wait for the stream."""
    t = torch.from_numpy(np.ascontiguousarray(a)) if isinstance(a, np.ndarray) else torch.tensor(a, dtype=dtype)
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    dev = torch.device(device)
    if dev.type != "cuda":
        return t.to(dev)
    return t.pin_memory().to(dev, non_blocking=True)


def _need(t: torch.Tensor, dtype, name: str) -> None:
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


# ----------------------------------------------------------------------------- router
def router_topk(logits: torch.Tensor, k: int, norm: bool, gates_out: bool = False):
    """logits [..., N] bf16 -> (inds int32 [..., k], scores bf16 [..., k][, gates bf16 [..., N]]).

    The fused router of Q36/kernels/router_topk.py:177-192 (softmax, rank top-k in ascending
    (value, index) order, gather, optional bf16 renormalisation)."""
    _need(logits, torch.bfloat16, "logits")
    n = logits.shape[-1]
    rows = logits.numel() // n if n else 0
    shp = (*logits.shape[:-1], k)
    inds = torch.empty(shp, dtype=torch.int32, device=logits.device)
    scores = torch.empty(shp, dtype=torch.bfloat16, device=logits.device)
    gates = torch.empty_like(logits) if gates_out else None
    _lib.check(
        _lib.lib().jit_router_topk(
            _p(logits), rows, n, int(k), int(bool(norm)), _p(inds), _p(scores), _p(gates), _stream()
        ),
        "router_topk",
    )
    return (inds, scores, gates) if gates_out else (inds, scores)


def topk(gates: torch.Tensor, k: int) -> torch.Tensor:
    """gates [..., N] bf16 -> int32 [..., k]: topk_stable (Q36/kernels/router_topk.py:36-66)."""
    _need(gates, torch.bfloat16, "gates")
    n = gates.shape[-1]
    rows = gates.numel() // n if n else 0
    out = torch.empty((*gates.shape[:-1], k), dtype=torch.int32, device=gates.device)
    _lib.check(_lib.lib().jit_topk(_p(gates), rows, n, int(k), _p(out), _stream()), "topk")
    return out


# ----------------------------------------------------------------------------- packing
@dataclass
class Packing:
    """Packing tables of P = B*k (row, slot) pairs sorted stably by expert (jit_moe_pack)."""

    order: torch.Tensor
    pair_row: torch.Tensor
    inv: torch.Tensor
    expert_cnt: torch.Tensor
    expert_off: torch.Tensor
    seg_expert: torch.Tensor
    seg_start: torch.Tensor
    seg_cnt: torch.Tensor
    meta: torch.Tensor
    P: int
    k: int
    E: int


def moe_pack(inds: torch.Tensor, n_experts: int) -> Packing:
    """inds [B, k] int32 -> Packing: Q36/model/moe.py:151-159 (_sort_pairs) and
    FN/model/moe/expert_mlp.py:39-49,147-163 (segment tables) in one launch."""
    _need(inds, torch.int32, "inds")
    pk = _packing_buffers(inds.numel(), inds.shape[-1], int(n_experts), inds.device)
    moe_pack_into(inds, pk)
    return pk


def moe_pack_into(inds: torch.Tensor, pk: Packing) -> None:
    """moe_pack into the tables pk (sized for inds: P = inds.numel(), k = inds.shape[-1])."""
    _need(inds, torch.int32, "inds")
    k, P, E = pk.k, pk.P, pk.E
    if inds.numel() != P or inds.shape[-1] != k:
        raise ValueError(f"packing tables of {P} pairs x k={k} do not fit inds {tuple(inds.shape)}")
    L = _lib.lib()
    ws_bytes = int(L.jit_moe_pack_workspace_bytes(P, E))
    if ws_bytes == 0:
        _lib.check(
            L.jit_moe_pack(
                _p(inds), P, k, E, _p(pk.order), _p(pk.pair_row), _p(pk.inv), _p(pk.expert_cnt),
                _p(pk.expert_off), _p(pk.seg_expert), _p(pk.seg_start), _p(pk.seg_cnt), _p(pk.meta),
                _stream(),
            ),
            "moe_pack",
        )
        return
    # a long batch: three launches over a workspace of per-tile counts (jit_moe_pack_ws)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=inds.device)
    _lib.check(
        L.jit_moe_pack_ws(
            _p(inds), P, k, E, _p(pk.order), _p(pk.pair_row), _p(pk.inv), _p(pk.expert_cnt),
            _p(pk.expert_off), _p(pk.seg_expert), _p(pk.seg_start), _p(pk.seg_cnt), _p(pk.meta),
            _p(ws), ws_bytes, _stream(),
        ),
        "moe_pack",
    )


ROUTE_PACK_MAX_ROWS = 4


def _tables_for(pk: Packing | None, P: int, k: int, E: int, device) -> Packing:
    """pk when it is sized for P pairs of k slots over E experts (ValueError otherwise), new tables
    when it is None."""
    if pk is None:
        return _packing_buffers(P, k, E, device)
    if (pk.P, pk.k, pk.E) != (P, k, E):
        raise ValueError(f"packing tables of (P, k, E) = {(pk.P, pk.k, pk.E)}, the call needs {(P, k, E)}")
    return pk


def route_pack(logits: torch.Tensor, k: int, norm: bool, pk: Packing | None = None):
    """router_topk then moe_pack of at most ROUTE_PACK_MAX_ROWS rows in one launch (jit_route_pack):
    (inds, scores, Packing), bit for bit the two-launch result; the expert count is N.  The tables
    go into pk when given."""
    _need(logits, torch.bfloat16, "logits")
    rows, n = logits.shape
    inds = torch.empty((rows, k), dtype=torch.int32, device=logits.device)
    scores = torch.empty((rows, k), dtype=torch.bfloat16, device=logits.device)
    pk = _tables_for(pk, rows * k, k, n, logits.device)
    _lib.check(
        _lib.lib().jit_route_pack(
            _p(logits), rows, n, int(k), int(bool(norm)), _p(inds), _p(scores), _p(pk.order), _p(pk.pair_row),
            _p(pk.inv), _p(pk.expert_cnt), _p(pk.expert_off), _p(pk.seg_expert), _p(pk.seg_start),
            _p(pk.seg_cnt), _p(pk.meta), _stream(),
        ),
        "route_pack",
    )
    return inds, scores, pk


def route_gate_up(x: torch.Tensor, logits: torch.Tensor, gate_up, k: int, norm: bool, pk: Packing | None = None):
    """One token's route_pack and expert_gate_up in one launch (jit_moe_gate_up_swiglu_routed_packed):
    x [1, K] bf16, logits [1, E] bf16, a packed [E, 2I, K] stack -> (inds, scores, Packing, h), bit
    for bit the two launches' results.  The tables go into pk when given."""
    _need(x, torch.bfloat16, "x")
    _need(logits, torch.bfloat16, "logits")
    _need_packed(gate_up, "route_gate_up")
    if x.shape[0] != 1 or logits.shape[0] != 1:
        raise _lib.UnsupportedShape("route_gate_up takes one token")
    E = logits.shape[1]
    if E != _experts_of(gate_up) or x.shape[-1] != gate_up.in_dims:
        raise ValueError("x / logits / stack disagree on K or E")
    I = gate_up.out_dims // 2
    inds = torch.empty((1, k), dtype=torch.int32, device=x.device)
    scores = torch.empty((1, k), dtype=torch.bfloat16, device=x.device)
    pk = _tables_for(pk, k, k, E, x.device)
    h = torch.empty((k, I), dtype=torch.bfloat16, device=x.device)
    _lib.check(
        _lib.lib().jit_moe_gate_up_swiglu_routed_packed(
            _p(x), x.shape[-1], _p(logits), E, int(k), int(bool(norm)), _p(gate_up.data), I, _p(h), _p(inds),
            _p(scores), _p(pk.order), _p(pk.pair_row), _p(pk.inv), _p(pk.expert_cnt), _p(pk.expert_off),
            _p(pk.seg_expert), _p(pk.seg_start), _p(pk.seg_cnt), _p(pk.meta), _stream(),
        ),
        "route_gate_up",
    )
    return inds, scores, pk, h


def _need_pairs(pk: Packing, rows: int, k: int, r: torch.Tensor | None, what: str) -> None:
    """The packing tables pk cover `rows` rows of k slots (P = rows k), and r (when given) holds their
    P pair rows: the kernels index inv, pair_row and r by these counts."""
    if pk.k != k or pk.P != rows * k:
        raise ValueError(f"{what}: packing tables of P={pk.P}, k={pk.k} for {rows} rows of {k} slots")
    if r is not None and (r.dim() != 2 or r.shape[0] != pk.P):
        raise ValueError(f"{what}: r {tuple(r.shape)} must hold the {pk.P} pair rows")


def _packing_buffers(P: int, k: int, E: int, device) -> Packing:
    buf = torch.empty(3 * P + 5 * E + 4, dtype=torch.int32, device=device)
    parts = torch.split(buf, [P, P, P, E, E, E, E, E, 4])
    return Packing(*parts, P=P, k=k, E=E)


# ----------------------------------------------------------------------------- packed layout
@dataclass
class PackedQ4:
    """A quantized matrix or expert stack [E, N, K] reordered into the MFMA tile layout
    (jit_q4_prepack): the same bytes as the MLX layout, read by the kernels with coalesced 1 KB
    loads.  `data` is a uint8 device tensor."""

    data: torch.Tensor
    E: int
    N: int
    K: int
    stacked: bool

    @property
    def in_dims(self) -> int:
        return self.K

    @property
    def out_dims(self) -> int:
        return self.N

    @property
    def nbytes(self) -> int:
        return self.data.numel()

    def __post_init__(self):
        # the kernels read E * N * K / 2 nibbles and their scales from `data`: a tensor of another size
        # (an operator handed a byte tensor and separate dims) is refused before anything reads it
        if self.data.dtype != torch.uint8 or not self.data.is_contiguous():
            raise ValueError("packed data must be a contiguous uint8 tensor")
        need = packed_bytes(self.E, self.N, self.K)
        if need <= 0:
            raise _lib.UnsupportedShape(f"the packed layout takes N % 16 == 0 and K % 128 == 0, got "
                                        f"[{self.E}, {self.N}, {self.K}]")
        if self.data.numel() != need:
            raise ValueError(f"packed data of {self.data.numel()} bytes for [{self.E}, {self.N}, {self.K}], "
                             f"which takes {need}")


def packed_bytes(E: int, N: int, K: int) -> int:
    return int(_lib.lib().jit_q4_packed_bytes(int(E), int(N), int(K)))


def prepack(lin: QLinear) -> PackedQ4:
    """Reorder a device QLinear (matrix [N, K] or stack [E, N, K]) into the packed tile layout."""
    lin.validate()
    if not lin.weight.is_cuda:
        raise ValueError("prepack takes device tensors")
    stacked = lin.weight.dim() == 3
    E = lin.weight.shape[0] if stacked else 1
    N, K = lin.out_dims, lin.in_dims
    nbytes = packed_bytes(E, N, K)
    if nbytes < 0:
        raise _lib.UnsupportedShape(f"prepack covers N % 16 == 0 and K % 128 == 0, got N={N} K={K}")
    out = torch.empty(nbytes, dtype=torch.uint8, device=lin.weight.device)
    _lib.check(
        _lib.lib().jit_q4_prepack(_p(lin.weight), _p(lin.scales), _p(lin.biases), E, N, K, _p(out), _stream()),
        "q4_prepack",
    )
    return PackedQ4(out, E, N, K, stacked)


# ----------------------------------------------------------------------------- projections
QMM_SEG_MIN_ROWS = 192  # the reference's switch to its prefill tile GEMM (Q36/kernels/qmm_prefill.py:75)


def qmm(x: torch.Tensor, lin, seg: bool | None = None) -> torch.Tensor:
    """x [T, K] bf16 -> [T, N] bf16 against a 4-bit matrix [N, K] (QLinear in the MLX layout or
    PackedQ4): QLinear.__call__ / .rows (Q36/linear.py:219-313).  A packed matrix and a batch of
    at least QMM_SEG_MIN_ROWS rows take the prefill tile GEMM (jit_qmm_seg: bf16-dequantized
    weights, as the reference's dense prefill kernel) where its shape allows; seg forces the
    choice."""
    _need(x, torch.bfloat16, "x")
    T, K = x.shape
    if K != lin.in_dims:
        raise ValueError(f"x has K = {K}, the matrix takes {lin.in_dims}")
    y = torch.empty((T, lin.out_dims), dtype=torch.bfloat16, device=x.device)
    if isinstance(lin, PackedQ4):
        if lin.stacked:
            raise ValueError("qmm takes one [N, K] matrix")
        if seg is None:
            seg = T >= QMM_SEG_MIN_ROWS and lin.N % 256 == 0 and K % 128 == 0
        if seg:
            _lib.check(_lib.lib().jit_qmm_seg(_p(x), T, K, _p(lin.data), lin.N, _p(y), _stream()), "qmm_seg")
        else:
            _lib.check(_lib.lib().jit_qmm_packed(_p(x), T, K, _p(lin.data), lin.N, _p(y), _stream()), "qmm_packed")
        return y
    if seg:
        raise ValueError("the prefill tile GEMM reads a packed matrix")
    if lin.weight.dim() != 2:
        raise ValueError("qmm takes one [N, K] matrix")
    lin.validate()
    _lib.check(
        _lib.lib().jit_qmm(
            _p(x), T, K, _p(lin.weight), _p(lin.scales), _p(lin.biases), lin.out_dims, _p(y), _stream()
        ),
        "qmm",
    )
    return y


def _experts_of(lin) -> int:
    if isinstance(lin, PackedQ4):
        if not lin.stacked:
            raise ValueError("expert projections take a stack [E, N, K]")
        return lin.E
    lin.validate()
    if lin.weight.dim() != 3:
        raise ValueError("expert projections take a stack [E, N, K]")
    return lin.weight.shape[0]


def _need_packed(lin, what: str) -> None:
    if not isinstance(lin, PackedQ4):
        raise ValueError(f"{what}: the segment GEMM takes packed stacks (ops.prepack)")


def expert_gate_up(x: torch.Tensor, gate_up, pk: Packing, seg: bool = False) -> torch.Tensor:
    """x [B, K] bf16, fused stack [E, 2I, K] -> h [P, I] bf16 in sorted pair order: the grouped
    gate||up + SwiGLU (expert_gate_up_exact(_rows), Q36/kernels/expert_solo.py:213-232,380-401).
    seg=True runs the segment GEMM of long expert segments instead (seg_gather_qmm,
    Q36/kernels/gather_qmm_prefill.py:226-257; bf16 weights, jit_moe_gate_up_swiglu_seg)."""
    _need(x, torch.bfloat16, "x")
    E = _experts_of(gate_up)
    if x.shape[-1] != gate_up.in_dims or E != pk.E:
        raise ValueError("x / stack / packing disagree on K or E")
    _need_pairs(pk, x.shape[0], pk.k, None, "expert_gate_up")  # (the pairs' rows are rows of x)
    I = gate_up.out_dims // 2
    h = torch.empty((pk.P, I), dtype=torch.bfloat16, device=x.device)
    L = _lib.lib()
    if seg:
        _need_packed(gate_up, "expert_gate_up")
        rc = L.jit_moe_gate_up_swiglu_seg(
            _p(x), x.shape[-1], _p(pk.pair_row), _p(pk.expert_cnt), _p(pk.expert_off), E, _p(gate_up.data),
            I, pk.P, _p(h), _stream(),
        )
    elif isinstance(gate_up, PackedQ4):
        rc = L.jit_moe_gate_up_swiglu_packed(
            _p(x), x.shape[-1], _p(pk.pair_row), _p(pk.expert_cnt), _p(pk.expert_off), E, _p(gate_up.data),
            I, pk.P, _p(h), _stream(),
        )
    else:
        rc = L.jit_moe_gate_up_swiglu(
            _p(x), x.shape[-1], _p(pk.pair_row), _p(pk.expert_cnt), _p(pk.expert_off), E,
            _p(gate_up.weight), _p(gate_up.scales), _p(gate_up.biases), I, pk.P, _p(h), _stream(),
        )
    _lib.check(rc, "moe_gate_up")
    return h


def swiglu(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """Elementwise SwiGLU of bf16 g, u (the stock swiglu, Q36/kernels/elementwise.py:14-15:
    nn.silu(gate) * up with every step rounded to bf16), via jit_swiglu."""
    _need(g, torch.bfloat16, "g")
    _need(u, torch.bfloat16, "u")
    if g.shape != u.shape:
        raise ValueError(f"g {tuple(g.shape)} and u {tuple(u.shape)} differ")
    h = torch.empty_like(g)
    _lib.check(_lib.lib().jit_swiglu(_p(g), _p(u), g.numel(), _p(h), _stream()), "swiglu")
    return h


def expert_down(h: torch.Tensor, down, pk: Packing, seg: bool = False) -> torch.Tensor:
    """h [P, I] bf16, stack [E, D, I] -> r [P, D] bf16 (the down gather, Q36/model/moe.py:193);
    seg=True: the segment GEMM (jit_moe_down_seg), as in expert_gate_up."""
    _need(h, torch.bfloat16, "h")
    E = _experts_of(down)
    D = down.out_dims
    if h.shape[-1] != down.in_dims or E != pk.E or h.shape[0] != pk.P:
        raise ValueError("h / stack / packing disagree on I, E or P")
    r = torch.empty((pk.P, D), dtype=torch.bfloat16, device=h.device)
    L = _lib.lib()
    if seg:
        _need_packed(down, "expert_down")
        rc = L.jit_moe_down_seg(
            _p(h), h.shape[-1], _p(pk.expert_cnt), _p(pk.expert_off), E, _p(down.data), D, pk.P, _p(r), _stream(),
        )
    elif isinstance(down, PackedQ4):
        rc = L.jit_moe_down_packed(
            _p(h), h.shape[-1], _p(pk.expert_cnt), _p(pk.expert_off), E, _p(down.data), D, pk.P, _p(r), _stream(),
        )
    else:
        rc = L.jit_moe_down(
            _p(h), h.shape[-1], _p(pk.expert_cnt), _p(pk.expert_off), E, _p(down.weight),
            _p(down.scales), _p(down.biases), D, pk.P, _p(r), _stream(),
        )
    _lib.check(rc, "moe_down")
    return r


def moe_combine(r: torch.Tensor, pk: Packing, scores: torch.Tensor, resid: torch.Tensor | None = None):
    """y [B, D] = sum over slots of bf16(r * score), sequential bf16 in slot order
    (Q36/kernels/expert_solo.py:155-163), plus resid if given (with_residual)."""
    _need(r, torch.bfloat16, "r")
    _need(scores, torch.bfloat16, "scores")
    B, k = scores.shape
    D = r.shape[-1]
    if resid is not None:
        _need(resid, torch.bfloat16, "resid")
        if resid.shape != (B, D):
            raise ValueError("resid must be [B, D]")
    _need_pairs(pk, B, k, r, "moe_combine")
    y = torch.empty((B, D), dtype=torch.bfloat16, device=r.device)
    _lib.check(
        _lib.lib().jit_moe_combine(_p(r), _p(pk.inv), _p(scores), B, k, D, _p(resid), _p(y), _stream()),
        "moe_combine",
    )
    return y


def moe_combine_rmsnorm(r: torch.Tensor, pk: Packing, scores: torch.Tensor, resid: torch.Tensor | None,
                        w: torch.Tensor, eps: float):
    """(y, xn): y = moe_combine(r, pk, scores, resid) and xn = rmsnorm(y, w, eps) in one launch
    (jit_moe_combine_rmsnorm; bit for bit the two calls) -- a layer's output and the next layer's
    normed input."""
    _need(r, torch.bfloat16, "r")
    _need(scores, torch.bfloat16, "scores")
    _need(w, torch.bfloat16, "w")
    B, k = scores.shape
    D = r.shape[-1]
    if resid is not None:
        _need(resid, torch.bfloat16, "resid")
        if resid.shape != (B, D):
            raise ValueError("resid must be [B, D]")
    if w.numel() != D:
        raise ValueError(f"norm weight of {w.numel()} for rows of {D}")
    _need_pairs(pk, B, k, r, "moe_combine_rmsnorm")
    y = torch.empty((B, D), dtype=torch.bfloat16, device=r.device)
    xn = torch.empty_like(y)
    _lib.check(
        _lib.lib().jit_moe_combine_rmsnorm(_p(r), _p(pk.inv), _p(scores), B, k, D, _p(resid), _p(y), _p(w),
                                           float(eps), _p(xn), _stream()),
        "moe_combine_rmsnorm",
    )
    return y, xn


def row_prologue_fits(lin, D: int) -> bool:
    """Whether a one-row projection can build its own normed input row (qmm_add_rmsnorm,
    qmm_combine_rmsnorm): a packed [N, D] matrix with D % 256 == 0, D <= 2048, N % 16 == 0."""
    return (isinstance(lin, PackedQ4) and not lin.stacked and lin.K == D and D % 256 == 0 and D <= 2048
            and lin.N % 16 == 0)


def _need_row_prologue(lin, D: int, what: str) -> None:
    if not row_prologue_fits(lin, D):
        raise _lib.UnsupportedShape(f"{what} takes a packed [N, {D}] matrix, D % 256 == 0, D <= 2048, N % 16 == 0")


def qmm_add_rmsnorm(a: torch.Tensor, resid: torch.Tensor, w: torch.Tensor, eps: float, lin):
    """(y, h, hn) for one row in one launch (jit_qmm_packed_add_rmsnorm): h = bf16(a + resid),
    hn = rmsnorm(h, w, eps), y = hn . W^T -- bit for bit rmsnorm(a, w, eps, resid, return_sum=True)
    and qmm(hn, lin) (the post-attention norm and the router projection of a one-token step)."""
    for t, name in ((a, "a"), (resid, "resid"), (w, "w")):
        _need(t, torch.bfloat16, name)
    D = a.shape[-1]
    if a.shape != (1, D) or resid.shape != (1, D) or w.numel() != D:
        raise ValueError("qmm_add_rmsnorm takes one row: a, resid [1, D], w [D]")
    _need_row_prologue(lin, D, "qmm_add_rmsnorm")
    y = torch.empty((1, lin.N), dtype=torch.bfloat16, device=a.device)
    h, hn = torch.empty_like(a), torch.empty_like(a)
    _lib.check(
        _lib.lib().jit_qmm_packed_add_rmsnorm(_p(a), _p(resid), _p(w), float(eps), D, _p(lin.data), lin.N, _p(h),
                                              _p(hn), _p(y), _stream()),
        "qmm_add_rmsnorm",
    )
    return y, h, hn


def qmm_combine_rmsnorm(r: torch.Tensor, pk: Packing, scores: torch.Tensor, resid: torch.Tensor | None,
                        w: torch.Tensor, eps: float, lin):
    """(y, out) for one row in one launch (jit_qmm_packed_combine_rmsnorm): y = moe_combine(r, pk,
    scores, resid) and out = rmsnorm(y, w, eps) . W^T -- bit for bit moe_combine_rmsnorm and qmm of its
    normed row (a layer's output and the next layer's qkv projection in a one-token step)."""
    _need(r, torch.bfloat16, "r")
    _need(scores, torch.bfloat16, "scores")
    _need(w, torch.bfloat16, "w")
    B, k = scores.shape
    D = r.shape[-1]
    if B != 1:
        raise _lib.UnsupportedShape("qmm_combine_rmsnorm takes one row")
    if resid is not None:
        _need(resid, torch.bfloat16, "resid")
        if resid.shape != (1, D):
            raise ValueError("resid must be [1, D]")
    if w.numel() != D:
        raise ValueError(f"norm weight of {w.numel()} for rows of {D}")
    _need_row_prologue(lin, D, "qmm_combine_rmsnorm")
    _need_pairs(pk, 1, k, r, "qmm_combine_rmsnorm")
    y = torch.empty((1, D), dtype=torch.bfloat16, device=r.device)
    out = torch.empty((1, lin.N), dtype=torch.bfloat16, device=r.device)
    _lib.check(
        _lib.lib().jit_qmm_packed_combine_rmsnorm(_p(r), _p(pk.inv), _p(scores), k, _p(resid), _p(w), float(eps), D,
                                                  _p(lin.data), lin.N, _p(y), _p(out), _stream()),
        "qmm_combine_rmsnorm",
    )
    return y, out


# ----------------------------------------------------------------------------- decoder block glue
def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, resid: torch.Tensor | None = None,
            return_sum: bool = False):
    """RMSNorm rows of x (mx.fast.rms_norm, Q36/model/model.py:65-80); with resid the normed row
    is h = x + resid, and return_sum=True returns (normed, h)."""
    _need(x, torch.bfloat16, "x")
    _need(w, torch.bfloat16, "w")
    rows, D = x.shape
    if w.shape != (D,):
        raise ValueError(f"norm weight must be [{D}]")
    if resid is not None:
        _need(resid, torch.bfloat16, "resid")
        if resid.shape != x.shape:
            raise ValueError("resid must match x")
    y = torch.empty_like(x)
    h = torch.empty_like(x) if (resid is not None and return_sum) else None
    _lib.check(
        _lib.lib().jit_rmsnorm(_p(x), _p(resid), rows, D, _p(w), float(eps), _p(h), _p(y), _stream()), "rmsnorm"
    )
    if return_sum:
        return y, (h if h is not None else x)
    return y


def qk_norm_rope_append(qkv: torch.Tensor, H: int, Hkv: int, q_norm: torch.Tensor, k_norm: torch.Tensor,
                        eps: float, inv_freq: torch.Tensor, pos: torch.Tensor, page_table: torch.Tensor,
                        pool: torch.Tensor) -> torch.Tensor:
    """qkv [B, (H + 2 Hkv) * 128] -> q [B, H, 128] (normed, rotated); k, v appended to the pool at
    pos (Q36/model/attention.py:99-119 + KVSlot.append)."""
    _need(qkv, torch.bfloat16, "qkv")
    _need(pool, torch.bfloat16, "pool")
    _need(pos, torch.int32, "pos")
    _need(page_table, torch.int32, "page_table")
    _need(inv_freq, torch.float32, "inv_freq")
    B = qkv.shape[0]
    if qkv.shape[1] != (H + 2 * Hkv) * HEAD_DIM or _pool_heads(pool) != Hkv or inv_freq.numel() != HEAD_DIM // 2:
        raise ValueError("qkv / pool / inv_freq do not match the head geometry")
    q = torch.empty((B, H, HEAD_DIM), dtype=torch.bfloat16, device=qkv.device)
    _lib.check(
        _lib.lib().jit_qk_norm_rope_append(
            _p(qkv), B, H, Hkv, _p(q_norm), _p(k_norm), float(eps), _p(inv_freq), _p(pos), _p(page_table),
            page_table.shape[1], _p(pool), _p(q), _stream(),
        ),
        "qk_norm_rope_append",
    )
    return q


# ----------------------------------------------------------------------------- paged KV
def _pool_heads(pool: torch.Tensor) -> int:
    """kv heads of a layer's pool [num_pages, Hkv, 2 (K, V), 16 * 128] (ValueError otherwise)."""
    if pool.dim() != 4 or pool.shape[2] != 2 or pool.shape[3] != PAGE * HEAD_DIM or not pool.is_contiguous():
        raise ValueError(f"a KV pool is a contiguous [pages, Hkv, 2, {PAGE * HEAD_DIM}] tensor, got {tuple(pool.shape)}")
    return int(pool.shape[1])


def kv_append_paged(pool: torch.Tensor, k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor,
                    page_table: torch.Tensor) -> None:
    """Write k, v [B, Hkv, 128] at positions pos [B] (KVSlot.append, Q36/kvcache/kv_cache.py:76-85)."""
    _need(pool, torch.bfloat16, "pool")
    _need(k, torch.bfloat16, "k")
    _need(v, torch.bfloat16, "v")
    _need(pos, torch.int32, "pos")
    _need(page_table, torch.int32, "page_table")
    B, Hkv, Dh = k.shape
    if Dh != HEAD_DIM or v.shape != k.shape or _pool_heads(pool) != Hkv:
        raise ValueError("kv_append_paged: k/v [B, Hkv, 128] must match the pool [pages, Hkv, 2, 2048]")
    _lib.check(
        _lib.lib().jit_kv_append_paged(
            _p(k), _p(v), B, Hkv, _p(pos), _p(page_table), page_table.shape[1], _p(pool), _stream()
        ),
        "kv_append_paged",
    )


@dataclass
class AttnPlan:
    """Split-K plan of one decode step: chunk boundaries per sequence (host and device copies)."""

    lens: torch.Tensor         # int32 [B] (device)
    chunk_start: torch.Tensor  # int32 [B + 1] (device)
    chunk_seq: torch.Tensor    # int32 [total] (device)
    total: int
    lens_host: np.ndarray


def attn_chunk_tokens(length: int) -> int:
    return int(_lib.lib().jit_attn_chunk_tokens(int(length)))


def attn_plan(lens_host, device) -> AttnPlan:
    """Plan the split of every sequence into key chunks (jit_attn_plan, host only)."""
    ln = np.ascontiguousarray(np.asarray(lens_host, dtype=np.int32))
    B = ln.size
    cs = np.empty(B + 1, np.int32)
    total = _lib.check(
        _lib.lib().jit_attn_plan(ln.ctypes.data_as(ctypes.c_void_p), B, cs.ctypes.data_as(ctypes.c_void_p), None, 0),
        "attn_plan",
    )
    seq = np.empty(max(total, 1), np.int32)
    _lib.check(
        _lib.lib().jit_attn_plan(
            ln.ctypes.data_as(ctypes.c_void_p), B, cs.ctypes.data_as(ctypes.c_void_p),
            seq.ctypes.data_as(ctypes.c_void_p), int(seq.size),
        ),
        "attn_plan",
    )
    dev = upload(np.concatenate([ln, cs, seq]), device)
    return AttnPlan(dev[:B], dev[B:2 * B + 1], dev[2 * B + 1:], int(total), ln)


def attn_workspace_bytes(total_chunks: int, H: int) -> int:
    return int(_lib.lib().jit_attn_workspace_bytes(int(total_chunks), int(H)))


@dataclass
class PrefillPlan:
    """Chunks (seq, ctx, length) of a prefill step in q-row order and their work items for
    jit_paged_prefill_attn (device int32 tables, built once on the host)."""

    chunks: list
    tables: torch.Tensor  # [4, C] chunk_seq, chunk_ctx, chunk_len, chunk_row
    blocks: torch.Tensor  # [3, nblk] blk_chunk, blk_q0, blk_part
    rows: int
    pmax: int = 1  # most key parts of a token (jit_prefill_part_keys keys a part)
    max_len: int = 0  # the longest chunk


def prefill_plan(chunks, H: int, Hkv: int, device) -> PrefillPlan:
    """Plan of causal prefill attention over chunks [(seq, ctx, length), ...]: every chunk cut
    into row blocks of jit_prefill_block_tokens tokens, each block's keys cut at multiples of
    jit_prefill_part_keys, one work item per (block, part), the items with the most key steps first."""
    lib = _lib.lib()
    bt = int(lib.jit_prefill_block_tokens(H, Hkv))
    if bt <= 0:
        raise _lib.UnsupportedShape(f"prefill attention covers H / Hkv in (1, 2, 4, 8, 16), got {H}/{Hkv}")
    part_keys = int(lib.jit_prefill_part_keys())
    step = 128
    part_steps = part_keys // step
    rows, tab, items, pmax, max_len = 0, [], [], 1, 0
    for c, (seq, ctx, length) in enumerate(chunks):
        if seq < 0 or ctx < 0 or length < 1:
            raise ValueError(f"chunk {c}: seq {seq}, ctx {ctx}, length {length}")
        tab.append((seq, ctx, length, rows))
        rows += length
        max_len = max(max_len, length)
        pmax = max(pmax, (ctx + length - 1) // part_keys + 1)
        for q0 in range(0, length, bt):
            keys = ctx + min(q0 + bt, length)
            nst = (keys + step - 1) // step
            for p in range((nst - 1) // part_steps + 1):
                items.append((min(nst, (p + 1) * part_steps) - p * part_steps, keys, c, q0, p))
    items.sort(key=lambda it: (-it[0], -it[1]))
    tables = upload(np.array(tab, np.int32).T.copy() if tab else np.zeros((4, 0), np.int32), device)
    blocks = upload(np.array([it[2:] for it in items], np.int32).T.copy() if items
                    else np.zeros((3, 0), np.int32), device)
    return PrefillPlan(list(chunks), tables.contiguous(), blocks.contiguous(), rows, pmax, max_len)


def prefill_workspace_bytes(plan: PrefillPlan, H: int) -> int:
    return int(_lib.lib().jit_prefill_workspace_bytes(plan.rows, plan.pmax, H))


def paged_prefill_attention(q: torch.Tensor, pool: torch.Tensor, page_table: torch.Tensor, plan: PrefillPlan,
                            scale: float, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """q [T, H, 128] bf16 (the plan's chunk rows) -> out [T, H, 128]: causal attention of each chunk
    token over its sequence's keys up to its own position (jit_paged_prefill_attn); tokens of
    several key parts go through a workspace of prefill_workspace_bytes (allocated when not given)."""
    _need(q, torch.bfloat16, "q")
    _need(pool, torch.bfloat16, "pool")
    _need(page_table, torch.int32, "page_table")
    T, H, Dh = q.shape
    Hkv = _pool_heads(pool)
    if Dh != HEAD_DIM:
        raise _lib.UnsupportedShape(f"paged_prefill_attention covers head_dim 128, got {Dh}")
    if T != plan.rows:
        raise ValueError(f"q has {T} rows, the plan's chunks {plan.rows}")
    for seq, ctx, length in plan.chunks:
        if seq >= page_table.shape[0] or (ctx + length + PAGE - 1) // PAGE > page_table.shape[1]:
            raise ValueError(f"chunk ({seq}, {ctx}, {length}) is outside page_table {tuple(page_table.shape)}")
    need = prefill_workspace_bytes(plan, H)
    if need > 0 and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    out = torch.empty_like(q)
    tb, bl = plan.tables, plan.blocks
    _lib.check(
        _lib.lib().jit_paged_prefill_attn(
            _p(q), _p(pool), _p(page_table), page_table.shape[1], _p(tb[0]), _p(tb[1]), _p(tb[2]), _p(tb[3]),
            tb.shape[1], _p(bl[0]), _p(bl[1]), _p(bl[2]), bl.shape[1], plan.pmax, plan.max_len, H, Hkv,
            float(scale), _p(workspace) if need > 0 else None, _p(out), _stream(),
        ),
        "paged_prefill_attn",
    )
    return out


def paged_decode_attention(q: torch.Tensor, pool: torch.Tensor, page_table: torch.Tensor,
                           plan: AttnPlan, scale: float, workspace: torch.Tensor | None = None):
    """q [B, H, 128] bf16 -> out [B, H, 128] bf16 over each sequence's first lens[b] keys of the
    paged pool: sdpa_decode(_rows) (Q36/kernels/sdpa_decode.py:448-476) with split-K."""
    _need(q, torch.bfloat16, "q")
    _need(pool, torch.bfloat16, "pool")
    _need(page_table, torch.int32, "page_table")
    B, H, Dh = q.shape
    Hkv = _pool_heads(pool)
    if Dh != HEAD_DIM:
        raise _lib.UnsupportedShape(f"paged_decode_attention covers head_dim 128, got {Dh}")
    if plan.lens.shape[0] != B or page_table.shape[0] != B:
        raise ValueError("q, page_table and plan disagree on the number of sequences")
    if B and int((plan.lens_host.max() + PAGE - 1) // PAGE) > page_table.shape[1]:
        raise ValueError(f"page_table has {page_table.shape[1]} columns, the longest sequence needs "
                         f"{int((plan.lens_host.max() + PAGE - 1) // PAGE)}")
    if H % Hkv:
        raise ValueError(f"{H} query heads over a pool of {Hkv} kv heads")
    need = attn_workspace_bytes(plan.total, H)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 4), dtype=torch.uint8, device=q.device)
    out = torch.empty_like(q)
    _lib.check(
        _lib.lib().jit_paged_decode_attn(
            _p(q), _p(pool), _p(page_table), page_table.shape[1], _p(plan.lens), _p(plan.chunk_start),
            _p(plan.chunk_seq), B, H, Hkv, float(scale), plan.total, _p(workspace), _p(out), _stream(),
        ),
        "paged_decode_attn",
    )
    return out


def paged_decode_attention_qkv(qkv: torch.Tensor, H: int, Hkv: int, q_norm: torch.Tensor, k_norm: torch.Tensor,
                               eps: float, inv_freq: torch.Tensor, pool: torch.Tensor, page_table: torch.Tensor,
                               plan: AttnPlan, scale: float, workspace: torch.Tensor | None = None):
    """qkv [B, (H + 2 Hkv) * 128] (the step's raw rows) -> out [B, H, 128]: qk_norm_rope_append of each
    row's token at position lens[b] - 1 and paged_decode_attention in one launch (the same bits);
    the token's K and V are written into the pool."""
    _need(qkv, torch.bfloat16, "qkv")
    _need(pool, torch.bfloat16, "pool")
    _need(page_table, torch.int32, "page_table")
    _need(inv_freq, torch.float32, "inv_freq")
    B = qkv.shape[0]
    if qkv.shape[1] != (H + 2 * Hkv) * HEAD_DIM or _pool_heads(pool) != Hkv or inv_freq.numel() != HEAD_DIM // 2:
        raise ValueError("qkv / pool / inv_freq do not match the head geometry")
    if plan.lens.shape[0] != B or page_table.shape[0] != B:
        raise ValueError("qkv, page_table and plan disagree on the number of sequences")
    if B and int((plan.lens_host.max() + PAGE - 1) // PAGE) > page_table.shape[1]:
        raise ValueError(f"page_table has {page_table.shape[1]} columns, the longest sequence needs "
                         f"{int((plan.lens_host.max() + PAGE - 1) // PAGE)}")
    need = attn_workspace_bytes(plan.total, H)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 4), dtype=torch.uint8, device=qkv.device)
    out = torch.empty((B, H, HEAD_DIM), dtype=torch.bfloat16, device=qkv.device)
    _lib.check(
        _lib.lib().jit_paged_decode_attn_qkv(
            _p(qkv), _p(q_norm), _p(k_norm), float(eps), _p(inv_freq), _p(pool), _p(page_table), page_table.shape[1],
            _p(plan.lens), _p(plan.chunk_start), _p(plan.chunk_seq), B, H, Hkv, float(scale), plan.total,
            _p(workspace), _p(out), _stream(),
        ),
        "paged_decode_attn_qkv",
    )
    return out


def paged_decode_attention_noalloc(q: torch.Tensor, pool: torch.Tensor, page_table: torch.Tensor,
                                   plan: AttnPlan, scale: float, out: torch.Tensor):
    """paged_decode_attention into a caller-given `out` [B, H, 128] bf16, with the split-K partials in
    the library's fixed device scratch (jit_paged_decode_attn_noalloc): nothing is allocated, for
    callers that cannot allocate.  Calls overlapping in time on one GPU race on that scratch."""
    _need(q, torch.bfloat16, "q")
    _need(pool, torch.bfloat16, "pool")
    _need(page_table, torch.int32, "page_table")
    _need(out, torch.bfloat16, "out")
    B, H, Dh = q.shape
    Hkv = _pool_heads(pool)
    if Dh != HEAD_DIM:
        raise _lib.UnsupportedShape(f"paged_decode_attention covers head_dim 128, got {Dh}")
    if out.shape != q.shape:
        raise ValueError(f"out {tuple(out.shape)} must match q {tuple(q.shape)}")
    if plan.lens.shape[0] != B or page_table.shape[0] != B:
        raise ValueError("q, page_table and plan disagree on the number of sequences")
    if B and int((plan.lens_host.max() + PAGE - 1) // PAGE) > page_table.shape[1]:
        raise ValueError(f"page_table has {page_table.shape[1]} columns, the longest sequence needs "
                         f"{int((plan.lens_host.max() + PAGE - 1) // PAGE)}")
    _lib.check(
        _lib.lib().jit_paged_decode_attn_noalloc(
            _p(q), _p(pool), _p(page_table), page_table.shape[1], _p(plan.lens), _p(plan.chunk_start),
            _p(plan.chunk_seq), B, H, Hkv, float(scale), plan.total, _p(out), _stream(),
        ),
        "paged_decode_attn_noalloc",
    )
    return out


# ----------------------------------------------------------------------------- step ends, KV pages
def embed_q4(ids: torch.Tensor, table: QLinear) -> torch.Tensor:
    """Embedding rows [B, D] bf16 of token ids [B] int32 from an MLX 4-bit table [V, D]
    (QEmbedding.lookup, Q36/linear.py:680-690: mx.dequantize of the gathered rows)."""
    _need(ids, torch.int32, "ids")
    for t, n in ((table.weight, "weight"), (table.scales, "scales"), (table.biases, "biases")):
        if not t.is_cuda:
            raise ValueError(f"embedding {n} must be a device tensor")
    if ids.dim() != 1 or table.weight.dim() != 2:
        raise ValueError("embed_q4 takes ids [B] and a [V, D] table")
    V, D = table.weight.shape[0], table.weight.shape[1] * 8
    out = torch.empty((ids.shape[0], D), dtype=torch.bfloat16, device=ids.device)
    _lib.check(_lib.lib().jit_embed_q4(_p(ids), ids.shape[0], _p(table.weight), _p(table.scales), _p(table.biases),
                                       V, D, _p(out), _stream()), "embed_q4")
    return out


def sampler_workspace(device) -> torch.Tensor:
    """A workspace for the sampling ops (jit_sampler_workspace_bytes bytes): a stream that samples
    while others do passes one of its own; without one the library's static buffer serves, and calls
    on several streams at once would race on it."""
    return torch.empty(int(_lib.lib().jit_sampler_workspace_bytes()), dtype=torch.uint8, device=device)


def _ws_args(workspace):
    if workspace is None:
        return None, 0
    _need(workspace, torch.uint8, "workspace")
    return _p(workspace), workspace.numel()


def logprobs_rows(logits: torch.Tensor, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """bf16 [B, V]: lp = bf16(x - lse) per row with lse = bf16(m0 + ln(S 2^-42)), S the exact
    integer sum of floor(e^(x - m0) 2^42) (logprobs_from_logits, Q36/sampler.py:295-297)."""
    _need(logits, torch.bfloat16, "logits")
    B, V = logits.shape
    out = torch.empty_like(logits)
    ws, nb = _ws_args(workspace)
    _lib.check(_lib.lib().jit_logprobs_rows_ws(_p(logits), B, V, _p(out), ws, nb, _stream()), "logprobs_rows")
    return out


def argmax_rows(logits: torch.Tensor, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """int32 [B]: the first index of each row's largest log-probability (the greedy draw,
    Q36/sampler.py:371-374)."""
    _need(logits, torch.bfloat16, "logits")
    B, V = logits.shape
    out = torch.empty(B, dtype=torch.int32, device=logits.device)
    ws, nb = _ws_args(workspace)
    _lib.check(_lib.lib().jit_argmax_rows_ws(_p(logits), B, V, _p(out), ws, nb, _stream()), "argmax_rows")
    return out


def sample_rows(logits: torch.Tensor, temperature: float, top_p: float, top_k: int,
                u: torch.Tensor | None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """int32 [B]: one draw per row of bf16 logits [B, V] under shared settings, given fp32
    uniforms u [B] (Sampler._sample_exact_full / sample_rows, Q36/sampler.py:451-476, 486-543;
    the definitions are jit_sample_rows'); temperature <= 0 is the greedy draw."""
    _need(logits, torch.bfloat16, "logits")
    B, V = logits.shape
    if temperature > 0:
        if u is None:
            raise ValueError("sample_rows needs uniforms when temperature > 0")
        _need(u, torch.float32, "u")
        if u.shape != (B,):
            raise ValueError(f"u must be [{B}], got {tuple(u.shape)}")
    out = torch.empty(B, dtype=torch.int32, device=logits.device)
    ws, nb = _ws_args(workspace)
    _lib.check(_lib.lib().jit_sample_rows_ws(_p(logits), B, V, float(temperature), float(top_p), int(top_k),
                                             _p(u) if u is not None else None, _p(out), ws, nb, _stream()),
               "sample_rows")
    return out


def threefry_uniform(keys: torch.Tensor) -> torch.Tensor:
    """fp32 [B]: the uniform of each uint32 key pair (keys [B, 2] as int32 bits): the first word
    of Threefry-2x32-20 at counter (0, 0), / 2^32, clamped below 1 (Sampler.uniform,
    Q36/sampler.py:367-369)."""
    _need(keys, torch.int32, "keys")
    if keys.dim() != 2 or keys.shape[1] != 2:
        raise ValueError("keys must be [B, 2]")
    out = torch.empty(keys.shape[0], dtype=torch.float32, device=keys.device)
    _lib.check(_lib.lib().jit_threefry_uniform(_p(keys), keys.shape[0], _p(out), _stream()), "threefry_uniform")
    return out


def kv_copy_pages(pool: torch.Tensor, src: torch.Tensor, dst: torch.Tensor) -> None:
    """Copy pages src[i] -> dst[i] (int32 device tensors) inside one layer's pool."""
    _need(pool, torch.bfloat16, "pool")
    _need(src, torch.int32, "src")
    _need(dst, torch.int32, "dst")
    if src.shape != dst.shape or src.dim() != 1:
        raise ValueError("src and dst must be equal-length 1-D page lists")
    _lib.check(_lib.lib().jit_kv_copy_pages(_p(pool), pool.shape[0], _pool_heads(pool), _p(src), _p(dst),
                                            src.shape[0], _stream()), "kv_copy_pages")
