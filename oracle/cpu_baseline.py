"""CPU baseline for bench.py: the reference's own CPU path, restated. TEST/MEASUREMENT INFRASTRUCTURE ONLY.

The reference checks this arithmetic on the CPU with PyTorch over *dequantised* weights: qwen3moe/reference.py:53-65
dequantises the int4 words with numpy and runs fp32 torch layers (:121-129), its MoE block as transformers'
Qwen3MoeSparseMoeBlock (softmax, top-k, renormalise, a loop over the hit experts with ``index_add_``); llama/run.py:
77-86,186-198 does the same for Llama. This module restates that path with torch on the host cores (fp32 ``F.linear`` over a dequantised
matrix; dequantisation timed separately), so bench.py can report it beside the GPU numbers. Only bench.py's
``cpu_baseline`` leg imports it.
"""
from __future__ import annotations

import os
import platform
import time

import numpy as np
import torch


def threads() -> int:
    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    return n


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def dequant_q4(wq: np.ndarray, ws: np.ndarray, group: int) -> torch.Tensor:
    """Q4W -> fp32 [N, K] as qwen3moe/reference.py:53-65 (``((nib ^ 8) - 8) * scale``), in torch on the CPU."""
    w = torch.from_numpy(np.ascontiguousarray(wq).view(np.int32))
    shifts = torch.arange(0, 32, 4, dtype=torch.int32)
    nib = (w.unsqueeze(-1) >> shifts) & 15
    q = ((nib ^ 8) - 8).reshape(w.shape[0], -1).to(torch.float32)
    s = torch.from_numpy(np.ascontiguousarray(ws).astype(np.float32))
    return (q.reshape(w.shape[0], -1, group) * s.unsqueeze(-1)).reshape(q.shape)


def median_time(fn, reps: int, budget_s: float) -> float:
    fn()  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > t_end and len(times) >= 3:
            break
    return float(np.median(times))


def gemv_q4(wq, ws, x, group, reps=20, budget_s=4.0):
    """Seconds for (matmul only, dequant + matmul) of one int4 GEMV, fp32."""
    w = dequant_q4(wq, ws, group)
    xt = torch.from_numpy(np.asarray(x, np.float32))
    t_mm = median_time(lambda: torch.mv(w, xt), reps, budget_s / 2)
    t_all = median_time(lambda: torch.mv(dequant_q4(wq, ws, group), xt), max(3, reps // 4), budget_s / 2)
    return t_mm, t_all


def gemm_layer(mats: dict, xs: dict, group: int, reps=5, budget_s=8.0):
    """Seconds for one layer's projections ``F.linear(X, W_deq)`` in fp32 (matmul only), X fp32 copies of the fp16
    activations."""
    ws = {name: dequant_q4(q, s, group) for name, (q, s) in mats.items()}
    xt = {k: torch.from_numpy(v.astype(np.float32)) for k, v in xs.items()}

    def run():
        for name, w in ws.items():
            torch.nn.functional.linear(xt[w.shape[1]], w)

    return median_time(run, reps, budget_s)


def llama_decode(mats: dict, head: tuple, dim: int, heads: int, kv_heads: int, ffn: int, context: int,
                 group: int, reps=5, budget_s=10.0):
    """Seconds for one decode step's layers (as many as ``mats`` holds) and for the head, fp32 torch on the CPU over
    dequantised weights: rmsnorm, fused qkv, RoPE, attention over ``context`` cached positions (fp32 cache), o +
    residual, rmsnorm, gate|up, SiLU product, down + residual (llama/model.mojo:140-166, the arithmetic run.py checks
    with transformers). ``mats[layer] = {name: (words, scales)}`` for wqkv, wo, wgu, wdown; ``head`` = lm_head words,
    scales. Returns (seconds for the layers, seconds for final norm + lm_head + argmax)."""
    hd = dim // heads
    lw = [{name: dequant_q4(q, s, group) for name, (q, s) in m.items()} for m in mats]
    lm = dequant_q4(*head, group)
    g = torch.Generator().manual_seed(0)
    kc = [torch.randn(kv_heads, context, hd, generator=g) for _ in lw]
    vc = [torch.randn(kv_heads, context, hd, generator=g) for _ in lw]
    nw = torch.ones(dim)
    cos, sin = torch.rand(hd // 2, generator=g), torch.rand(hd // 2, generator=g)
    x0 = torch.randn(dim, generator=g)
    F = torch.nn.functional

    def rms(x):
        return x * torch.rsqrt((x * x).mean() + 1e-5) * nw

    def rope(v):
        a, b = v[..., :hd // 2], v[..., hd // 2:]
        return torch.cat([a * cos - b * sin, b * cos + a * sin], dim=-1)

    def layers():
        x = x0.clone()
        for i, w in enumerate(lw):
            qkv = F.linear(rms(x), w["wqkv"])
            q = rope(qkv[:heads * hd].view(heads, hd))
            kc[i][:, -1] = rope(qkv[heads * hd:(heads + kv_heads) * hd].view(kv_heads, hd))
            vc[i][:, -1] = qkv[(heads + kv_heads) * hd:].view(kv_heads, hd)
            k = kc[i].repeat_interleave(heads // kv_heads, 0)
            v = vc[i].repeat_interleave(heads // kv_heads, 0)
            p = torch.softmax(torch.einsum("hd,hsd->hs", q, k) / hd ** 0.5, dim=-1)
            x = x + F.linear(torch.einsum("hs,hsd->hd", p, v).reshape(-1), w["wo"])
            h = F.linear(rms(x), w["wgu"])
            x = x + F.linear(F.silu(h[:ffn]) * h[ffn:], w["wdown"])
        return x

    def head_fn():
        return int(torch.argmax(F.linear(rms(x0), lm)))

    return median_time(layers, reps, budget_s / 2), median_time(head_fn, reps, budget_s / 2)


def dequant_t2(w: np.ndarray, s: np.ndarray) -> torch.Tensor:
    """T2W words [K/16, N] and fp16 scales [K/128, N] -> fp32 [N, K]: ``(code - 1) * scale`` with code (k, n) at bits
    2 (k % 16) of word (k / 16, n) (bonsai/kernels/prefill.mojo:228-230,260)."""
    wt = torch.from_numpy(np.ascontiguousarray(w).view(np.int32))
    shifts = torch.arange(0, 32, 2, dtype=torch.int32)
    codes = (wt.unsqueeze(-1) >> shifts) & 3                       # [K/16, N, 16]
    q = (codes.permute(1, 0, 2).reshape(wt.shape[1], -1) - 1).to(torch.float32)
    sc = torch.from_numpy(np.ascontiguousarray(s).astype(np.float32)).t()  # [N, K/128]
    return (q.reshape(q.shape[0], -1, 128) * sc.unsqueeze(-1)).reshape(q.shape)


def ternary(mats: dict, xv: dict, xs: dict, reps=5, budget_s=8.0):
    """Seconds for one gate/up/down triple of fp32 ``mv`` (the GEMV) and of ``F.linear`` at M rows (the GEMM) over
    the dequantised ternary matrices. ``mats[name] = (words, scales)``; xv / xs keyed by K."""
    ws = [dequant_t2(w, s) for w, s in mats.values()]
    v = {k: torch.from_numpy(np.asarray(a, np.float32)) for k, a in xv.items()}
    m = {k: torch.from_numpy(np.asarray(a, np.float32)) for k, a in xs.items()}
    t_mv = median_time(lambda: [torch.mv(w, v[w.shape[1]]) for w in ws], reps * 4, budget_s / 2)
    t_mm = median_time(lambda: [torch.nn.functional.linear(m[w.shape[1]], w) for w in ws], reps, budget_s / 2)
    return t_mv, t_mm


def moe_block(d: dict, reps=5, budget_s=10.0):
    """Seconds for one MoE block over d["tokens"] tokens (``moe_forward``)."""
    return median_time(moe_forward(d), reps, budget_s)


def moe_forward(d: dict, topk: int = 8):
    """One MoE block over d["tokens"] tokens as transformers' Qwen3MoeSparseMoeBlock computes it in fp32 on
    dequantised experts (qwen3moe/reference.py:121-129): softmax of the router logits, top-k, renormalise, then for
    every expert that was hit, ``down(silu(gate x) * up x)`` of its tokens times their weights, ``index_add_`` into
    the output. Returns the block as a function of no arguments (the experts dequantised once)."""
    E, D, F, G = d["experts"], d["hidden"], d["ffn"], d["group"]
    gu = dequant_q4(d["gu_q"], d["gu_s"], G).view(E, 2 * F, D)
    dn = dequant_q4(d["dn_q"], d["dn_s"], G).view(E, D, F)
    x = torch.from_numpy(d["x"])
    logits = torch.from_numpy(d["logits"])
    lin = torch.nn.functional.linear

    def run():
        p = torch.softmax(logits, dim=-1)
        w, ids = torch.topk(p, topk, dim=-1)
        w = w / w.sum(dim=-1, keepdim=True)
        out = torch.zeros_like(x)
        mask = torch.nn.functional.one_hot(ids, E).permute(2, 1, 0)  # [E, topk, T]
        for e in torch.nonzero(mask.sum(dim=(1, 2))).flatten().tolist():
            slot, tok = torch.where(mask[e])
            h = lin(x[tok], gu[e])
            y = lin(torch.nn.functional.silu(h[:, :F]) * h[:, F:], dn[e]) * w[tok, slot, None]
            out.index_add_(0, tok, y)
        return out

    return run
