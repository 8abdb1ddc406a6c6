"""PyTorch-ROCm custom ops (``torch.ops.aq.*``) over the libaq C ABI.

Each op takes tensors in the reference's packed layouts, validates shapes/dtypes on the host, and enqueues the HIP
kernels on the current stream of the tensors' device (no host synchronisation, no allocation). Outputs are
``Tensor(a!)`` arguments written in place. Only device tensors are accepted: there is no CPU implementation.
"""
from __future__ import annotations

import torch

from . import _lib

_LIB = torch.library.Library("aq", "DEF")


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _dev(*ts: torch.Tensor) -> None:
    d = ts[0].device
    for t in ts:
        _check(t.is_cuda, "aq ops take device (HIP) tensors only")
        _check(t.device == d, "all tensors must be on one device")
        _check(t.is_contiguous(), "tensors must be contiguous")


def _u32(t: torch.Tensor, name: str) -> None:
    _check(t.dtype in (torch.int32, torch.uint32), f"{name} must be int32/uint32 words")


def _f16bits(t: torch.Tensor, name: str) -> None:
    _check(t.dtype in (torch.float16, torch.int16, torch.uint16), f"{name} must be float16 (or its 16-bit pattern)")


# ---- int4 GEMV (decode / few tokens) ---------------------------------------------------------------------------

_LIB.define("gemv_q4(Tensor wq, Tensor ws, Tensor x, Tensor(a!) y, int group, bool add) -> ()")
_LIB.define("gate_up_q4(Tensor wq, Tensor ws, Tensor x, Tensor(a!) a, int group) -> ()")


def _gemv_q4_impl(wq, ws, x, y, group, add):
    _dev(wq, ws, x, y)
    _u32(wq, "wq")
    _f16bits(ws, "ws")
    _check(x.dtype == torch.float32 and y.dtype == torch.float32, "x and y must be float32")
    n, kw = wq.shape
    k = kw * 8
    xt = x.reshape(-1, k) if x.dim() != 1 else x.reshape(1, k)
    tokens = xt.shape[0]
    _check(x.numel() == tokens * k, "x must be [tokens, K]")
    _check(y.numel() == tokens * n, "y must be [tokens, N]")
    _check(ws.numel() == n * (k // group) and k % group == 0, "ws must be [N, K/group]")
    _lib.call("aq_gemv_q4", _ptr(wq), _ptr(ws), _ptr(x), _ptr(y), n, k, group, tokens, int(add), _stream(x))


def _gate_up_q4_impl(wq, ws, x, a, group):
    _dev(wq, ws, x, a)
    _u32(wq, "wq")
    _f16bits(ws, "ws")
    _check(x.dtype == torch.float32 and a.dtype == torch.float32, "x and a must be float32")
    rows, kw = wq.shape
    _check(rows % 2 == 0, "gate|up matrix must have 2f rows")
    f, k = rows // 2, kw * 8
    tokens = x.numel() // k
    _check(x.numel() == tokens * k and a.numel() == tokens * f, "x must be [tokens, K], a [tokens, f]")
    _check(ws.numel() == rows * (k // group) and k % group == 0, "ws must be [2f, K/group]")
    _lib.call("aq_gate_up_q4", _ptr(wq), _ptr(ws), _ptr(x), _ptr(a), f, k, group, tokens, _stream(x))


_LIB.impl("gemv_q4", _gemv_q4_impl, "CUDA")
_LIB.impl("gate_up_q4", _gate_up_q4_impl, "CUDA")


# ---- int4 GEMM (prefill, MFMA) ----------------------------------------------------------------------------------

_LIB.define("gemm_q4(Tensor x, Tensor wq, Tensor ws, Tensor(a!) y, int group, bool add, Tensor(b!) workspace) -> ()")

_WORKSPACE: dict = {}


def workspace(device: torch.device, nbytes: int, purpose: str = "gemm") -> torch.Tensor:
    """A per-(device, purpose) zero-filled scratch tensor of at least ``nbytes``, grown on demand and reused by later
    calls. Ops that keep arrival counters in it leave them at zero after every call."""
    key = (device.type, device.index, purpose)
    t = _WORKSPACE.get(key)
    if t is None or t.numel() < nbytes:
        t = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACE[key] = t
    return t


def _gemm_q4_impl(x, wq, ws, y, group, add, workspace):
    _dev(x, wq, ws, y)
    _u32(wq, "wq")
    _f16bits(ws, "ws")
    _check(x.dtype in (torch.float16, torch.float32), "x must be float16 or float32")
    _check(y.dtype == torch.float32, "y must be float32")
    n, kw = wq.shape
    k = kw * 8
    _check(x.dim() == 2 and x.shape[1] == k, "x must be [M, K]")
    m = x.shape[0]
    _check(tuple(y.shape) == (m, n), "y must be [M, N]")
    _check(ws.numel() == n * (k // group) and k % group == 0, "ws must be [N, K/group]")
    _dev(workspace)
    _lib.call("aq_gemm_q4", _ptr(x), int(x.dtype == torch.float32), _ptr(wq), _ptr(ws), _ptr(y), m, n, k, group,
              int(add), _ptr(workspace), workspace.numel() * workspace.element_size(), _stream(x))


_LIB.impl("gemm_q4", _gemm_q4_impl, "CUDA")


def gemm_q4(x: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor, y: torch.Tensor, group: int, add: bool = False):
    """``Y (+)= X . deq(W)^T`` on MFMA: X fp16/fp32 [M, K], Q4W ``wq [N, K/8]``, fp16 ``ws [N, K/group]``, Y fp32."""
    need = _lib.lib().aq_gemm_q4_workspace_bytes(x.shape[0], wq.shape[0], wq.shape[1] * 8)
    torch.ops.aq.gemm_q4(x, wq, ws, y, group, add, workspace(x.device, need))


def gemv_q4(wq: torch.Tensor, ws: torch.Tensor, x: torch.Tensor, y: torch.Tensor, group: int, add: bool = False):
    """``y[t] (+)= deq(W) . x[t]`` for Q4W ``wq [N, K/8]``, fp16 ``ws [N, K/group]``, fp32 ``x [T, K]``, T <= 16
    (9..16 rows: K <= 2048)."""
    torch.ops.aq.gemv_q4(wq, ws, x, y, group, add)


def gate_up_q4(wq: torch.Tensor, ws: torch.Tensor, x: torch.Tensor, a: torch.Tensor, group: int):
    """``a[t, j] = silu(W[j] . x[t]) * (W[f + j] . x[t])`` over the fused gate|up Q4W matrix ``[2f, K/8]``."""
    torch.ops.aq.gate_up_q4(wq, ws, x, a, group)


# ---- ternary (T2W) GEMV and X2H producers --------------------------------------------------------------------------

_LIB.define("t2_gemv(Tensor x2h, Tensor w, Tensor s, Tensor(a!) y, Tensor(b!) workspace) -> ()")
_LIB.define("t2_packed_linear(Tensor x2h, Tensor w, Tensor s, Tensor(a!) partials) -> ()")
_LIB.define("t2_packed_reduce(Tensor partials, Tensor(a!) y) -> ()")
_LIB.define("t2_head_argmax(Tensor x2h, Tensor w, Tensor s, Tensor(a!) logits, Tensor(b!) cand, Tensor(c!) token, "
            "Tensor(d!) pos, Tensor(e!) hist, int advance) -> ()")
_LIB.define("pack_half(Tensor x, Tensor(a!) q) -> ()")
_LIB.define("rmsnorm_pack(Tensor x, Tensor w, Tensor(a!) q, float eps) -> ()")
_LIB.define("swiglu_pack(Tensor gu, Tensor(a!) q) -> ()")


def _t2_shapes(x2h, w, s):
    _dev(x2h, w, s)
    _u32(x2h, "x2h")
    _u32(w, "w")
    _f16bits(s, "s")
    kw, n = w.shape
    k = kw * 16
    _check(x2h.numel() == k // 2, "x2h must hold K/2 fp16 pairs")
    _check(tuple(s.shape) == (k // 128, n), "s must be [K/128, N]")
    return n, k


def _t2_gemv_impl(x2h, w, s, y, workspace):
    n, k = _t2_shapes(x2h, w, s)
    _dev(y, workspace)
    _check(y.dtype == torch.float32 and y.numel() == n, "y must be float32 [N]")
    _lib.call("aq_t2_gemv", _ptr(x2h), _ptr(w), _ptr(s), _ptr(y), n, k, _ptr(workspace),
              workspace.numel() * workspace.element_size(), _stream(y))


def t2_head_candidates(n: int, k: int) -> int:
    """8-byte slots of the ternary head's cand for an N x K head: an argmax key per workgroup, then the arrival
    counters (HEAD_ARRIVAL_SLOTS). Allocate zero-filled."""
    return int(_lib.lib().aq_t2_head_candidates(n, k))


def _t2_head_argmax_impl(x2h, w, s, logits, cand, token, pos, hist, advance):
    n, k = _t2_shapes(x2h, w, s)
    _dev(logits, cand, token, pos, hist)
    _check(logits.dtype == torch.float32 and logits.numel() == n, "logits must be float32 [N]")
    _check(cand.dtype == torch.int64, "cand must be int64")
    _check(token.dtype == torch.int32 and pos.dtype == torch.int32 and hist.dtype == torch.int32,
           "int32 token/pos/hist")
    _lib.call("aq_t2_head_argmax", _ptr(x2h), _ptr(w), _ptr(s), _ptr(logits), n, k, _ptr(cand), cand.numel(),
              _ptr(token), _ptr(pos), _ptr(hist) if hist.numel() else None, hist.numel(), advance, _stream(logits))


def _t2_packed_linear_impl(x2h, w, s, partials):
    n, k = _t2_shapes(x2h, w, s)
    _dev(partials)
    _check(partials.dtype == torch.float32 and tuple(partials.shape) == ((k + 1023) // 1024, n),
           "partials must be float32 [ceil(K/1024), N]")
    _lib.call("aq_t2_packed_linear", _ptr(x2h), _ptr(w), _ptr(s), _ptr(partials), n, k, _stream(partials))


def _t2_packed_reduce_impl(partials, y):
    _dev(partials, y)
    _check(partials.dtype == torch.float32 and y.dtype == torch.float32, "float32 tensors")
    g, n = partials.shape
    _check(y.numel() == n, "y must be [N]")
    _lib.call("aq_t2_packed_reduce", _ptr(partials), _ptr(y), n, g, _stream(y))


def _pack_half_impl(x, q):
    _dev(x, q)
    _check(x.dtype == torch.float32, "x must be float32")
    _u32(q, "q")
    _check(q.numel() * 2 == x.numel(), "q must hold numel(x)/2 words")
    _lib.call("aq_pack_half", _ptr(x), _ptr(q), x.numel(), _stream(x))


def _rmsnorm_pack_impl(x, w, q, eps):
    _dev(x, w, q)
    _check(x.dtype == torch.float32 and w.dtype == torch.float32, "x and w must be float32")
    _u32(q, "q")
    n = w.numel()
    rows = x.numel() // n
    _check(x.numel() == rows * n and q.numel() * 2 == x.numel(), "x [rows, n], q [rows, n/2]")
    _lib.call("aq_rmsnorm_pack", _ptr(x), _ptr(w), _ptr(q), rows, n, float(eps), _stream(x))


def _swiglu_pack_impl(gu, q):
    _dev(gu, q)
    _check(gu.dtype == torch.float32, "gu must be float32")
    _u32(q, "q")
    n2 = gu.shape[-1]
    rows = gu.numel() // n2
    _check(n2 % 4 == 0 and q.numel() == rows * n2 // 4, "gu [rows, 2n], q [rows, n/2]")
    _lib.call("aq_swiglu_pack", _ptr(gu), _ptr(q), rows, n2 // 2, _stream(gu))


_LIB.impl("t2_gemv", _t2_gemv_impl, "CUDA")
_LIB.impl("t2_head_argmax", _t2_head_argmax_impl, "CUDA")
_LIB.impl("t2_packed_linear", _t2_packed_linear_impl, "CUDA")
_LIB.impl("t2_packed_reduce", _t2_packed_reduce_impl, "CUDA")
_LIB.impl("pack_half", _pack_half_impl, "CUDA")
_LIB.impl("rmsnorm_pack", _rmsnorm_pack_impl, "CUDA")
_LIB.impl("swiglu_pack", _swiglu_pack_impl, "CUDA")


def t2_gemv(x2h: torch.Tensor, w: torch.Tensor, s: torch.Tensor, y: torch.Tensor):
    """``y = deq_T2(W) . x`` for T2W ``w [K/16, N]``, fp16 ``s [K/128, N]``, X2H ``x2h [K/2]``; y fp32 [N]."""
    need = _lib.lib().aq_t2_gemv_workspace_bytes(w.shape[1], w.shape[0] * 16)
    torch.ops.aq.t2_gemv(x2h, w, s, y, workspace(y.device, need, "t2_gemv"))


def t2_packed_linear(x2h, w, s, partials):
    torch.ops.aq.t2_packed_linear(x2h, w, s, partials)


def t2_packed_reduce(partials, y):
    torch.ops.aq.t2_packed_reduce(partials, y)


def pack_half(x: torch.Tensor, q: torch.Tensor):
    torch.ops.aq.pack_half(x, q)


def rmsnorm_pack(x: torch.Tensor, w: torch.Tensor, q: torch.Tensor, eps: float = 1e-6):
    torch.ops.aq.rmsnorm_pack(x, w, q, eps)


def swiglu_pack(gu: torch.Tensor, q: torch.Tensor):
    torch.ops.aq.swiglu_pack(gu, q)


# ---- ternary (T2W) GEMM (prefill, MFMA) -----------------------------------------------------------------------------

_LIB.define("gemm_t2(Tensor x, Tensor w, Tensor s, Tensor(a!) y, bool add, Tensor(b!) workspace) -> ()")


def _gemm_t2_impl(x, w, s, y, add, workspace):
    _dev(x, w, s, y, workspace)
    _u32(w, "w")
    _f16bits(s, "s")
    _check(x.dtype in (torch.float16, torch.float32), "x must be float16 or float32")
    _check(y.dtype == torch.float32, "y must be float32")
    kw, n = w.shape
    k = kw * 16
    _check(x.dim() == 2 and x.shape[1] == k, "x must be [M, K]")
    m = x.shape[0]
    _check(tuple(y.shape) == (m, n), "y must be [M, N]")
    _check(tuple(s.shape) == (k // 128, n), "s must be [K/128, N]")
    _lib.call("aq_gemm_t2", _ptr(x), int(x.dtype == torch.float32), _ptr(w), _ptr(s), _ptr(y), m, n, k, int(add),
              _ptr(workspace), workspace.numel() * workspace.element_size(), _stream(x))


_LIB.impl("gemm_t2", _gemm_t2_impl, "CUDA")


def gemm_t2(x: torch.Tensor, w: torch.Tensor, s: torch.Tensor, y: torch.Tensor, add: bool = False):
    """``Y (+)= X . deq_T2(W)^T`` on MFMA: X fp16/fp32 [M, K], T2W ``w [K/16, N]``, fp16 ``s [K/128, N]``, Y fp32."""
    need = _lib.lib().aq_gemm_t2_workspace_bytes(x.shape[0], w.shape[1], w.shape[0] * 16)
    torch.ops.aq.gemm_t2(x, w, s, y, add, workspace(x.device, need))


# ---- mixture of experts -------------------------------------------------------------------------------------------

_LIB.define("moe_route(Tensor logits, Tensor(a!) ids, Tensor(b!) weights, int topk) -> ()")
_LIB.define("moe_route_pack(Tensor logits, Tensor(a!) ids, Tensor(b!) weights, int topk, Tensor x, "
            "Tensor(c!) xq) -> ()")
_LIB.define("moe_group(Tensor ids, int experts, int tm, Tensor(a!) counts, Tensor(b!) offs, Tensor(c!) slot, "
            "Tensor(d!) src, Tensor(e!) tiles, Tensor(f!) ntiles) -> ()")
_LIB.define("moe_gemm_q4(Tensor x, Tensor src, Tensor wq, Tensor ws, int experts, int group, Tensor tiles, "
            "Tensor ntiles, int tm, bool swiglu, Tensor(a!) out) -> ()")
_LIB.define("moe_combine(Tensor yd, Tensor slot, Tensor weights, Tensor(a!) y, bool add) -> ()")
_LIB.define("moe_gate_up_q4(Tensor wq, Tensor ws, int experts, Tensor ids, Tensor x, Tensor(a!) a, int group) -> ()")
_LIB.define("moe_down_q4(Tensor wq, Tensor ws, int experts, Tensor ids, Tensor weights, Tensor a, Tensor(a!) y, "
            "int group, bool add) -> ()")
_LIB.define("gemv_f32(Tensor w, Tensor x, Tensor(a!) y) -> ()")
_LIB.define("moe_expert_lists(Tensor ids, int experts, Tensor(a!) lists, Tensor(b!) counts, int items_tt, "
            "Tensor(c!) items, Tensor(d!) nitems, Tensor(e!) scratch) -> ()")


def _i32(*ts):
    for t in ts:
        _check(t.dtype == torch.int32, "index tensors must be int32")


def _moe_route_pack_impl(logits, ids, weights, topk, x, xq):
    _dev(logits, ids, weights, x, xq)
    _check(logits.dtype == torch.float32 and logits.dim() == 2, "logits must be float32 [T, E]")
    t, e = logits.shape
    _check(ids.dtype == torch.int32 and ids.numel() == t * topk, "ids must be int32 [T, topk]")
    _check(weights.dtype == torch.float32 and weights.numel() == t * topk, "weights must be float32 [T, topk]")
    _check(x.dtype == torch.float32 and x.dim() == 2 and x.shape[0] == t, "x must be float32 [T, d]")
    _u32(xq, "xq")
    d = x.shape[1]
    _check(xq.numel() * 2 == t * d, "xq must hold T * d / 2 words")
    _lib.call("aq_moe_route_pack", _ptr(logits), _ptr(ids), _ptr(weights), t, e, topk, _ptr(x), _ptr(xq), d,
              _stream(logits))


def _moe_route_impl(logits, ids, weights, topk):
    _dev(logits, ids, weights)
    _i32(ids)
    _check(logits.dtype == torch.float32 and weights.dtype == torch.float32, "logits/weights must be float32")
    t, e = logits.shape
    _check(ids.numel() == t * topk and weights.numel() == t * topk, "ids/weights must be [T, topk]")
    _lib.call("aq_moe_route", _ptr(logits), _ptr(ids), _ptr(weights), t, e, topk, _stream(logits))


def _moe_group_impl(ids, experts, tm, counts, offs, slot, src, tiles, ntiles):
    _dev(ids, counts, offs, slot, src, tiles, ntiles)
    _i32(ids, counts, offs, slot, src, tiles, ntiles)
    t, k = ids.shape
    _check(counts.numel() == experts and offs.numel() == experts + 1 and slot.numel() == t * k, "bad output sizes")
    _lib.call("aq_moe_group", _ptr(ids), t, k, experts, tm, _ptr(counts), _ptr(offs), _ptr(slot), _ptr(src),
              src.numel(), _ptr(tiles), tiles.numel() // 2, _ptr(ntiles), _stream(ids))


def _moe_gemm_q4_impl(x, src, wq, ws, experts, group, tiles, ntiles, tm, swiglu, out):
    _u32(wq, "wq")
    _f16bits(ws, "ws")
    _i32(tiles, ntiles)
    _check(x.dtype in (torch.float16, torch.float32), "x must be float16 or float32")
    rows, kw = wq.shape
    k = kw * 8
    _check(rows % experts == 0, "wq rows must be experts * n")
    n = rows // experts
    _check(x.dim() == 2 and x.shape[1] == k, "x must be [rows, K]")
    _check(group > 0 and k % group == 0 and ws.numel() == rows * (k // group), "ws must be [experts * n, K/group]")
    _check(out.dim() == 2, "out must be [rows_total, n] (or [rows_total, n/2] with swiglu)")
    if swiglu:
        _check(out.dtype == torch.float16 and out.shape[1] == n // 2, "swiglu out must be float16 [rows_total, n/2]")
    else:
        _check(out.dtype == torch.float32 and out.shape[1] == n, "out must be float32 [rows_total, n]")
    _dev(x, wq, ws, tiles, ntiles, out)
    src_ptr = 0
    if src.numel():
        _dev(src)
        _i32(src)
        src_ptr = _ptr(src)
    _lib.call("aq_moe_gemm_q4", _ptr(x), int(x.dtype == torch.float32), x.shape[0], src_ptr, _ptr(wq), _ptr(ws),
              experts, n, k, group, _ptr(tiles), _ptr(ntiles), tiles.numel() // 2, tm, out.shape[0], int(swiglu),
              _ptr(out), _stream(x))


def _moe_combine_impl(yd, slot, weights, y, add):
    # shapes and dtypes first: the kernel writes tokens * d floats of y and reads rows of yd through slot
    _check(yd.dtype == torch.float32 and y.dtype == torch.float32 and weights.dtype == torch.float32,
           "yd, weights and y must be float32")
    _check(weights.dim() == 2, "weights must be [T, topk]")
    t, k = weights.shape
    d = y.shape[-1]
    _check(y.numel() == t * d, "y must be [T, d]")
    _check(yd.dim() == 2 and yd.shape[1] == d, "yd must be [rows, d]")
    if slot.numel():
        _i32(slot)
        _check(slot.numel() == t * k, "slot must hold T * topk entries")
    _dev(yd, weights, y)
    slot_ptr = 0
    if slot.numel():
        _dev(yd, slot)
        slot_ptr = _ptr(slot)
    _lib.call("aq_moe_combine", _ptr(yd), yd.shape[0], slot_ptr, _ptr(weights), _ptr(y), t, d, k, int(add),
              _stream(y))


def _moe_gate_up_q4_impl(wq, ws, experts, ids, x, a, group):
    # shapes and dtypes first: the kernel writes topk * f floats of a
    _u32(wq, "wq")
    _f16bits(ws, "ws")
    _i32(ids)
    _check(wq.dim() == 2 and experts > 0 and wq.shape[0] % (2 * experts) == 0, "wq must be [experts * 2f, K/8]")
    rows, kw = wq.shape
    f, k = rows // experts // 2, kw * 8
    _check(group > 0 and k % group == 0 and ws.numel() == rows * (k // group), "ws must be [experts * 2f, K/group]")
    topk = ids.numel()
    _check(x.dtype == torch.float32 and x.numel() == k, "x must be float32 [K]")
    _check(a.dtype == torch.float32 and a.numel() == topk * f, "a must be float32 [topk, f]")
    _dev(wq, ws, ids, x, a)
    _lib.call("aq_moe_gate_up_q4", _ptr(wq), _ptr(ws), experts, _ptr(ids), _ptr(x), _ptr(a), f, k, group, topk,
              _stream(x))


def _moe_down_q4_impl(wq, ws, experts, ids, weights, a, y, group, add):
    # shapes and dtypes first: the kernel writes d floats of y
    _u32(wq, "wq")
    _f16bits(ws, "ws")
    _i32(ids)
    _check(wq.dim() == 2 and experts > 0 and wq.shape[0] % experts == 0, "wq must be [experts * d, f/8]")
    rows, kw = wq.shape
    d, f = rows // experts, kw * 8
    _check(group > 0 and f % group == 0 and ws.numel() == rows * (f // group), "ws must be [experts * d, f/group]")
    topk = ids.numel()
    _check(weights.dtype == torch.float32 and weights.numel() == topk, "weights must be float32 [topk]")
    _check(a.dtype == torch.float32 and a.numel() == topk * f, "a must be float32 [topk, f]")
    _check(y.dtype == torch.float32 and y.numel() == d, "y must be float32 [d]")
    _dev(wq, ws, ids, weights, a, y)
    _lib.call("aq_moe_down_q4", _ptr(wq), _ptr(ws), experts, _ptr(ids), _ptr(weights), _ptr(a), _ptr(y), d, f,
              group, topk, int(add), _stream(y))


def _gemv_f32_impl(w, x, y):
    _dev(w, x, y)
    n, k = w.shape
    tokens = x.numel() // k
    _check(y.numel() == n * tokens, "y must be [tokens, N]")
    _lib.call("aq_gemv_f32", _ptr(w), _ptr(x), _ptr(y), n, k, tokens, _stream(y))


def _moe_expert_lists_impl(ids, experts, lists, counts, items_tt, items, nitems, scratch):
    _dev(ids, lists, counts, scratch)
    _i32(ids, lists, counts, scratch)
    t, k = ids.shape
    items_ptr = nitems_ptr = 0
    if items.numel():
        _dev(items, nitems)
        items_ptr, nitems_ptr = _ptr(items), _ptr(nitems)
    _lib.call("aq_moe_expert_lists", _ptr(ids), t, k, experts, lists.shape[1], _ptr(lists), _ptr(counts), items_tt,
              items_ptr, items.numel() // 2, nitems_ptr, _ptr(scratch), scratch.numel(), _stream(ids))


for _name, _fn in (("moe_route", _moe_route_impl), ("moe_route_pack", _moe_route_pack_impl),
                   ("moe_group", _moe_group_impl), ("moe_gemm_q4", _moe_gemm_q4_impl),
                   ("moe_combine", _moe_combine_impl), ("moe_gate_up_q4", _moe_gate_up_q4_impl),
                   ("moe_down_q4", _moe_down_q4_impl), ("gemv_f32", _gemv_f32_impl),
                   ("moe_expert_lists", _moe_expert_lists_impl)):
    _LIB.impl(_name, _fn, "CUDA")


# ---- Llama decode step: fused norms, embedding, attention, lm_head + argmax -----------------------------------------

HEAD_CANDIDATES = 4096  # AQ_HEAD_CANDIDATES: argmax key slots of a head launch (the int4 head keeps its arrival
#                         counters in the last HEAD_ARRIVAL_SLOTS: allocate zero-filled)
HEAD_ARRIVAL_SLOTS = 17  # AQ_HEAD_ARRIVAL_SLOTS
ATTN_MAX_SPLITS = 8     # AQ_ATTN_MAX_SPLITS


def attn_parts_numel(heads: int, splits: int) -> int:
    """Floats of the split-attention state buffer: o [heads][splits][64], then (m, l) [heads][splits][2]."""
    return heads * splits * 66

_LIB.define("rmsnorm_gemv_q4(Tensor wq, Tensor ws, Tensor x, Tensor norm_w, float eps, Tensor(a!) y, int group) -> ()")
_LIB.define("rmsnorm_gate_up_q4(Tensor wq, Tensor ws, Tensor x, Tensor norm_w, float eps, Tensor(a!) a, int group)"
            " -> ()")
_LIB.define("embed_f16(Tensor table, Tensor token, Tensor(a!) x) -> ()")
_LIB.define("attn_decode(Tensor qkv, Tensor cos, Tensor sin, Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor pos, "
            "int heads, int kv_heads, Tensor(c!) out) -> ()")
_LIB.define("attn_decode_split(Tensor qkv, Tensor cos, Tensor sin, Tensor(a!) k_cache, Tensor(b!) v_cache, "
            "Tensor pos, int heads, int kv_heads, int splits, Tensor(c!) parts) -> ()")
_LIB.define("attn_out_q4(Tensor wq, Tensor ws, Tensor parts, int splits, Tensor(a!) y, int group) -> ()")
_LIB.define("head_argmax_q4(Tensor wq, Tensor ws, Tensor x, Tensor norm_w, float eps, Tensor(a!) logits, int group, "
            "Tensor(b!) cand, Tensor(c!) token, Tensor(d!) pos, Tensor(e!) hist, int advance) -> ()")


def _q4_shape(wq, ws, group):
    _u32(wq, "wq")
    _f16bits(ws, "ws")
    n, kw = wq.shape
    k = kw * 8
    _check(k % group == 0 and ws.numel() == n * (k // group), "ws must be [N, K/group]")
    return n, k


def _rmsnorm_gemv_q4_impl(wq, ws, x, norm_w, eps, y, group):
    _dev(wq, ws, x, norm_w, y)
    n, k = _q4_shape(wq, ws, group)
    _f16bits(norm_w, "norm_w")
    _check(x.dtype == torch.float32 and y.dtype == torch.float32, "x and y must be float32")
    tokens = x.numel() // k
    _check(x.numel() == tokens * k and y.numel() == tokens * n and norm_w.numel() == k,
           "x [T, K], y [T, N], norm_w [K]")
    _lib.call("aq_rmsnorm_gemv_q4", _ptr(wq), _ptr(ws), _ptr(x), _ptr(norm_w), eps, _ptr(y), n, k, group, tokens,
              _stream(x))


def _rmsnorm_gate_up_q4_impl(wq, ws, x, norm_w, eps, a, group):
    _dev(wq, ws, x, norm_w, a)
    rows, k = _q4_shape(wq, ws, group)
    _f16bits(norm_w, "norm_w")
    _check(rows % 2 == 0, "gate|up matrix must have 2f rows")
    f = rows // 2
    _check(x.dtype == torch.float32 and a.dtype == torch.float32, "x and a must be float32")
    tokens = x.numel() // k
    _check(x.numel() == tokens * k and a.numel() == tokens * f and norm_w.numel() == k, "x [T, K], a [T, f], norm_w [K]")
    _lib.call("aq_rmsnorm_gate_up_q4", _ptr(wq), _ptr(ws), _ptr(x), _ptr(norm_w), eps, _ptr(a), f, k, group, tokens,
              _stream(x))


def _embed_f16_impl(table, token, x):
    _dev(table, token, x)
    _f16bits(table, "table")
    _check(token.dtype == torch.int32 and token.numel() >= 1, "token must be int32 on the device")
    _check(x.dtype == torch.float32 and table.dim() == 2 and x.numel() == table.shape[1], "x must be float32 [d]")
    _lib.call("aq_embed_f16", _ptr(table), table.shape[0], table.shape[1], _ptr(token), _ptr(x), _stream(x))


def _attn_decode_impl(qkv, cos, sin, k_cache, v_cache, pos, heads, kv_heads, out):
    _dev(qkv, cos, sin, k_cache, v_cache, pos, out)
    _check(qkv.dtype == torch.float32 and out.dtype == torch.float32, "qkv and out must be float32")
    _check(cos.dtype == torch.float32 and sin.dtype == torch.float32, "cos/sin must be float32")
    _f16bits(k_cache, "k_cache")
    _f16bits(v_cache, "v_cache")
    _check(pos.dtype == torch.int32 and pos.numel() >= 1, "pos must be int32 on the device")
    _check(k_cache.dim() == 3 and k_cache.shape[0] == kv_heads and k_cache.shape[2] == 64, "k_cache [kv_heads, P, 64]")
    max_pos = k_cache.shape[1]
    _check(tuple(v_cache.shape) == tuple(k_cache.shape), "v_cache must match k_cache")
    _check(qkv.numel() == (heads + 2 * kv_heads) * 64 and out.numel() == heads * 64, "qkv/out sizes")
    _check(cos.numel() == max_pos * 32 and sin.numel() == max_pos * 32, "cos/sin must be [max_pos, 32]")
    _lib.call("aq_attn_decode", _ptr(qkv), _ptr(cos), _ptr(sin), _ptr(k_cache), _ptr(v_cache), _ptr(pos), heads,
              kv_heads, 64, max_pos, _ptr(out), _stream(qkv))


def _attn_decode_split_impl(qkv, cos, sin, k_cache, v_cache, pos, heads, kv_heads, splits, parts):
    _dev(qkv, cos, sin, k_cache, v_cache, pos, parts)
    _check(qkv.dtype == torch.float32 and parts.dtype == torch.float32, "qkv and parts must be float32")
    _check(cos.dtype == torch.float32 and sin.dtype == torch.float32, "cos/sin must be float32")
    _f16bits(k_cache, "k_cache")
    _f16bits(v_cache, "v_cache")
    _check(pos.dtype == torch.int32 and pos.numel() >= 1, "pos must be int32 on the device")
    _check(k_cache.dim() == 3 and k_cache.shape[0] == kv_heads and k_cache.shape[2] == 64, "k_cache [kv_heads, P, 64]")
    max_pos = k_cache.shape[1]
    _check(tuple(v_cache.shape) == tuple(k_cache.shape), "v_cache must match k_cache")
    _check(qkv.numel() == (heads + 2 * kv_heads) * 64, "qkv size")
    _check(cos.numel() == max_pos * 32 and sin.numel() == max_pos * 32, "cos/sin must be [max_pos, 32]")
    _check(parts.numel() >= attn_parts_numel(heads, splits), "parts too small")
    _lib.call("aq_attn_decode_split", _ptr(qkv), _ptr(cos), _ptr(sin), _ptr(k_cache), _ptr(v_cache), _ptr(pos), heads,
              kv_heads, 64, max_pos, splits, _ptr(parts), _stream(qkv))


def _attn_out_q4_impl(wq, ws, parts, splits, y, group):
    _dev(wq, ws, parts, y)
    n, k = _q4_shape(wq, ws, group)
    _check(parts.dtype == torch.float32 and y.dtype == torch.float32, "parts and y must be float32")
    _check(k % 64 == 0 and parts.numel() >= attn_parts_numel(k // 64, splits), "parts too small for K / 64 heads")
    _check(y.numel() == n, "y must be [N]")
    _lib.call("aq_attn_out_q4", _ptr(wq), _ptr(ws), _ptr(parts), splits, _ptr(y), n, k, group, _stream(y))


def _head_argmax_q4_impl(wq, ws, x, norm_w, eps, logits, group, cand, token, pos, hist, advance):
    _dev(wq, ws, x, logits, cand, token, pos)
    vocab, k = _q4_shape(wq, ws, group)
    _check(x.dtype == torch.float32 and x.numel() == k, "x must be float32 [K]")
    _check(logits.dtype == torch.float32 and logits.numel() == vocab, "logits must be float32 [vocab]")
    _check(cand.dtype in (torch.int64, torch.uint64), "cand must be 64-bit")
    _check(token.dtype == torch.int32 and pos.dtype == torch.int32, "token and pos must be int32")
    nw = 0
    if norm_w.numel():
        _dev(norm_w)
        _f16bits(norm_w, "norm_w")
        _check(norm_w.numel() == k, "norm_w must be [K]")
        nw = _ptr(norm_w)
    hp = 0
    if hist.numel():
        _dev(hist)
        _check(hist.dtype == torch.int32, "hist must be int32")
        hp = _ptr(hist)
    _lib.call("aq_head_argmax_q4", _ptr(wq), _ptr(ws), _ptr(x), nw, eps, _ptr(logits), vocab, k, group, _ptr(cand),
              cand.numel(), _ptr(token), _ptr(pos), hp, hist.numel(), advance, _stream(x))


# ---- Q6_K tied head / embedding (Q6W: q uint8 [rows, cols/256, 208], d fp16 [rows, cols/256]) -------------------

_LIB.define("gemv_q6(Tensor q, Tensor d, Tensor x, Tensor(a!) y) -> ()")
_LIB.define("head_argmax_q6(Tensor q, Tensor d, Tensor x, Tensor norm_w, float eps, Tensor(a!) logits, "
            "Tensor(b!) cand, Tensor(c!) token, Tensor(d!) pos, Tensor(e!) hist, int advance) -> ()")
_LIB.define("embed_q6(Tensor q, Tensor d, Tensor ids, Tensor(a!) x) -> ()")


def head_q6_candidates(rows: int, cols: int) -> int:
    """8-byte slots of the Q6_K head's cand: an argmax key per workgroup, then the arrival counters (at most
    HEAD_CANDIDATES). Allocate zero-filled."""
    return int(_lib.lib().aq_head_q6_candidates(rows, cols))


def _q6_shape(q, d):
    _check(q.dtype == torch.uint8 and q.dim() == 3 and q.shape[2] == 208 and q.is_contiguous(),
           "q must be contiguous uint8 [rows, cols/256, 208]")
    _f16bits(d, "d")
    rows, nb = q.shape[0], q.shape[1]
    _check(d.numel() == rows * nb, "d must be [rows, cols/256]")
    return rows, nb * 256


def _gemv_q6_impl(q, d, x, y):
    _dev(q, d, x, y)
    rows, cols = _q6_shape(q, d)
    _check(x.dtype == torch.float32 and x.numel() == cols, "x must be float32 [cols]")
    _check(y.dtype == torch.float32 and y.numel() == rows, "y must be float32 [rows]")
    _lib.call("aq_gemv_q6", _ptr(q), _ptr(d), _ptr(x), _ptr(y), rows, cols, _stream(x))


def _head_argmax_q6_impl(q, d, x, norm_w, eps, logits, cand, token, pos, hist, advance):
    _dev(q, d, x, logits, cand, token, pos)
    rows, cols = _q6_shape(q, d)
    _check(x.dtype == torch.float32 and x.numel() == cols, "x must be float32 [cols]")
    _check(logits.dtype == torch.float32 and logits.numel() == rows, "logits must be float32 [rows]")
    _check(cand.dtype == torch.int64, "cand must be int64")
    _check(token.dtype == torch.int32 and pos.dtype == torch.int32, "token and pos must be int32")
    nw = 0
    if norm_w.numel():
        _dev(norm_w)
        _f16bits(norm_w, "norm_w")
        _check(norm_w.numel() == cols, "norm_w must be [cols]")
        nw = _ptr(norm_w)
    hp = 0
    if hist.numel():
        _dev(hist)
        _check(hist.dtype == torch.int32, "hist must be int32")
        hp = _ptr(hist)
    _lib.call("aq_head_argmax_q6", _ptr(q), _ptr(d), _ptr(x), nw, eps, _ptr(logits), rows, cols, _ptr(cand),
              cand.numel(), _ptr(token), _ptr(pos), hp, hist.numel(), advance, _stream(x))


def _embed_q6_impl(q, d, ids, x):
    _dev(q, d, ids, x)
    rows, cols = _q6_shape(q, d)
    _check(ids.dtype == torch.int32 and ids.numel() >= 1, "ids must be int32 on the device")
    _check(x.dtype == torch.float32 and x.numel() == ids.numel() * cols, "x must be float32 [len(ids), cols]")
    _lib.call("aq_embed_q6", _ptr(q), _ptr(d), rows, cols, _ptr(ids), ids.numel(), _ptr(x), _stream(x))


for _name, _fn in (("gemv_q6", _gemv_q6_impl), ("head_argmax_q6", _head_argmax_q6_impl), ("embed_q6", _embed_q6_impl)):
    _LIB.impl(_name, _fn, "CUDA")


for _name, _fn in (("rmsnorm_gemv_q4", _rmsnorm_gemv_q4_impl), ("rmsnorm_gate_up_q4", _rmsnorm_gate_up_q4_impl),
                   ("embed_f16", _embed_f16_impl), ("attn_decode", _attn_decode_impl),
                   ("attn_decode_split", _attn_decode_split_impl), ("attn_out_q4", _attn_out_q4_impl),
                   ("head_argmax_q4", _head_argmax_q4_impl)):
    _LIB.impl(_name, _fn, "CUDA")


# ---- measurement ---------------------------------------------------------------------------------------------------

STREAM_READ_MAX_BLOCKS = 8192
_LIB.define("stream_read(Tensor p, Tensor(a!) sink, int blocks) -> ()")


def _stream_read_impl(p, sink, blocks):
    """sink[4 b + w] = XOR of the 32-bit words wave w of workgroup b reads; every byte of p read once (the
    streaming-read ceiling)."""
    _dev(p, sink)
    nbytes = p.numel() * p.element_size()
    _check(nbytes % 16 == 0, "p must hold a multiple of 16 bytes")
    _check(0 <= blocks <= STREAM_READ_MAX_BLOCKS, f"blocks must be in 0..{STREAM_READ_MAX_BLOCKS}")
    _check(sink.dtype in (torch.int32, torch.uint32), "sink must be int32/uint32 words")
    need = 4 * (blocks if blocks else min(STREAM_READ_MAX_BLOCKS, -(-(nbytes // 16) // 512)))
    _check(sink.numel() >= need, f"sink must hold {need} words")
    _lib.call("aq_stream_read", _ptr(p), nbytes, blocks, _ptr(sink), _stream(p))


_LIB.impl("stream_read", _stream_read_impl, "CUDA")
