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


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A per-device scratch tensor of at least ``nbytes`` (grown on demand, reused by later calls on that device)."""
    key = (device.type, device.index)
    t = _WORKSPACE.get(key)
    if t is None or t.numel() < nbytes:
        t = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
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
    """``y[t] (+)= deq(W) . x[t]`` for Q4W ``wq [N, K/8]``, fp16 ``ws [N, K/group]``, fp32 ``x [T, K]``, T <= 8."""
    torch.ops.aq.gemv_q4(wq, ws, x, y, group, add)


def gate_up_q4(wq: torch.Tensor, ws: torch.Tensor, x: torch.Tensor, a: torch.Tensor, group: int):
    """``a[t, j] = silu(W[j] . x[t]) * (W[f + j] . x[t])`` over the fused gate|up Q4W matrix ``[2f, K/8]``."""
    torch.ops.aq.gate_up_q4(wq, ws, x, a, group)
