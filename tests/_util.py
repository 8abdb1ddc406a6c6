"""Helpers shared by the tests (device copies of numpy arrays, error norms)."""
from __future__ import annotations

import numpy as np


def to_dev(a: np.ndarray, dev):
    """numpy -> contiguous device tensor; uint32 words travel as int32 (same bits)."""
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    elif a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).to(dev)


def to_np(t) -> np.ndarray:
    return t.detach().cpu().numpy()


def rel_inf(got, ref) -> float:
    """max |got - ref| / max |ref| (normwise relative error, infinity norm)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(got - ref)) / (den if den > 0 else 1.0))


def rel_l2(got, ref) -> float:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (den if den > 0 else 1.0))


def kat_int4(rng: np.random.Generator, n: int, k: int, group: int, tokens: int = 1):
    """Integer-exact known-answer inputs: small-integer x, power-of-two scales, so every partial sum is exact in fp32
    and the true product is an exact dyadic rational (the idea of the reference's runner/check.h:53-64)."""
    vals = rng.integers(-8, 8, size=(n, k))
    exps = rng.integers(-3, 2, size=(n, k // group)).astype(np.float32)
    ws = np.exp2(exps).astype(np.float16)
    x = rng.integers(-3, 4, size=(tokens, k)).astype(np.float32)
    return vals, ws, x


def exact_int4_product(vals: np.ndarray, ws: np.ndarray, x: np.ndarray, group: int) -> np.ndarray:
    """y[t, n] = sum_k vals[n,k] * ws[n,k/G] * x[t,k] in exact integer arithmetic (scales are 2^e, e >= -3)."""
    n, k = vals.shape
    scale8 = (ws.astype(np.float64) * 8).astype(np.int64)  # 2^(e+3), an integer
    w8 = vals.astype(np.int64) * np.repeat(scale8, group, axis=1)
    y8 = x.astype(np.int64) @ w8.T
    return y8.astype(np.float64) / 8.0
