"""CPU restatement (numpy) of mojo-adreno's weight-quantized matmul path. TEST INFRASTRUCTURE ONLY.

This module is the checker the HIP kernels are compared with. It is imported only by ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg; the product never calls it.

Every function names the reference file:line whose arithmetic it restates (paths relative to the reference
checkout). Values are computed in float64 from the exact float32 dequantisation, so the oracle carries no
reduction-order error of its own; integer work (unpacking, routing, grouping) is exact.

Layouts (the reference's on-device ABI):
  Q4W  ``wq: uint32 [N, K/8]``, element k of row n in bits 4*(k%8) of word k/8 (low nibble first), stored as 4-bit
       two's complement; ``ws: float16 [N, K/G]``; value ``(((nib ^ 8) - 8) * ws[n, k/G])``.
  T2W  ``w: uint32 [K/16, N]`` (transposed), the 2-bit code of (n, k) in bits 2*(k%16) of word (k/16)*N + n;
       ``s: float16 [K/128, N]``; value ``(code - 1) * s[k/128, n]``.
  X2H  ``uint32 [K/2]``: two float16 per word, the even k in the low half.

Pinning status (how each function is checked, see tests/test_oracle_*.py):
  * q4w_values/q4w_pack/q4w_dequant, t2w_*, x2h_*: known-answer words and a pure-Python bit loop (textbook
    two's complement), round trips.
  * gemv/gemm/ternary/MoE values: integer-exact known-answer tests (small-integer x, power-of-two scales) against
    Python integer arithmetic, plus pure-Python brute force on tiny shapes.
  * route_top8: brute force (sort by (-logit, index)), forced ties, softmax->top-k->renormalise identity.
  * expert_lists/expert_items/p_group/combine: brute force with a stable sort (a library routine).
  * quantize4 / quantize4_searched / gguf_q4_0_to_q4w / gguf_q4_0_dequant: bit-exact against the reference's own C
    (llama/st2bin.c "q4", qwen3moe/convert.c "q4" for G = 32/64/128, lfm2/convert.c "q4" and "h4"), compiled from the
    reference sources by oracle/Makefile: golden vectors in tests/golden/ref_*.npz (zero groups, .5 ties, fp16
    subnormals, negative maxima) and, where oracle/_ref is built, fresh runs of the binaries
    (tests/test_oracle_golden.py). Also ggml's published Q4_0 block layout, re-derived independently.
  * mlx_to_t2w: MLX's published 2-bit affine layout (weight = code*scale + bias): its T2W output, dequantised, equals a
    pure-Python bit walk of the MLX input (tests/test_formats.py::test_t2w_from_mlx_closed_form).
The exact fp32 bits of the reference's Mojo kernels (its reduction order and MAX's warp/coop-matrix primitives)
cannot be reproduced here: that part is "parity unpinned" and parity is defined by tolerance.
"""
from __future__ import annotations

import numpy as np

# ----------------------------------------------------------------------------------------------------------------
# int4 words (Q4W)
# ----------------------------------------------------------------------------------------------------------------


def q4w_values(wq: np.ndarray) -> np.ndarray:
    """Signed int4 values of Q4W words: ``((word >> 4j) & 15) ^ 8) - 8``.

    Follows llama/kernels/gemv_q4.mojo:24-26 and qwen3moe/reference.py:62-63. Returns int8 [..., 8*W].
    """
    wq = np.ascontiguousarray(np.asarray(wq, dtype="<u4"))  # little-endian: byte b of a word holds nibbles 2b, 2b+1
    b = wq.view(np.uint8)
    nib = np.empty(b.shape + (2,), np.uint8)
    np.bitwise_and(b, 15, out=nib[..., 0])
    np.right_shift(b, 4, out=nib[..., 1])
    nib ^= 8
    vals = nib.view(np.int8)
    vals -= 8
    return vals.reshape(*wq.shape[:-1], wq.shape[-1] * 8)


def q4w_pack(q: np.ndarray) -> np.ndarray:
    """Pack int values in -8..7 ([..., K], K % 8 == 0) into Q4W words, low nibble first.

    Follows llama/run.py:64-69 (``q & 0xF`` shifted by 4*j).
    """
    q = np.asarray(q)
    if q.shape[-1] % 8:
        raise ValueError("K must be a multiple of 8")
    if q.min(initial=0) < -8 or q.max(initial=0) > 7:
        raise ValueError("int4 values must lie in -8..7")
    nib = (q.astype(np.int32) & 0xF).astype(np.uint32).reshape(*q.shape[:-1], q.shape[-1] // 8, 8)
    return np.bitwise_or.reduce(nib << (np.arange(8, dtype=np.uint32) * 4), axis=-1).astype(np.uint32)


def q4w_dequant(wq: np.ndarray, ws: np.ndarray, group: int) -> np.ndarray:
    """Exact float32 dequantisation ``q * float(ws[n, k/G])`` of a Q4W matrix, [N, K].

    Follows qwen3moe/reference.py:53-65 (``Weights.int4``) and the per-element arithmetic of
    llama/kernels/gemv_q4.mojo:25-27 (scale index n*(K/G) + k/G). The product of an int in -8..7 and an fp16 is
    exact in float32.
    """
    vals = q4w_values(wq).astype(np.float32)
    n, k = vals.shape
    if k % group:
        raise ValueError("K must be a multiple of the group size")
    s = np.asarray(ws, dtype=np.float16).astype(np.float32).reshape(n, k // group)
    return (vals.reshape(n, k // group, group) * s[:, :, None]).reshape(n, k)


def gemv_q4(wq, ws, x, group: int, y0=None) -> np.ndarray:
    """``y[n] = sum_k W[n,k] x[k]`` (+ ``y0`` for the residual form), float64.

    Follows llama/kernels/gemv_q4.mojo:13-30 (``gemv_q4``), llama/kernels/gemv_add_q4.mojo:13-30 (``y[r] += s``),
    lfm2/kernels/lk.mojo:38-72,134-143 (``dot_q4``/``dot_q4b``/``gemv_q4``, G=32) and
    qwen3moe/kernels/moek.mojo:30-45 (``dot_q4_row[G]``).
    """
    w = q4w_dequant(wq, ws, group).astype(np.float64)
    y = w @ np.asarray(x, dtype=np.float64)
    if y0 is not None:
        y = y + np.asarray(y0, dtype=np.float64)
    return y


def silu(g):
    """``g / (1 + exp(-g))`` (lfm2/kernels/lk.mojo:33-34, moek.mojo:209)."""
    g = np.asarray(g, dtype=np.float64)
    return g / (1.0 + np.exp(-g))


def gate_up_q4(wq, ws, x, group: int, f: int) -> np.ndarray:
    """``a[j] = silu(W[j].x) * (W[f+j].x)`` over the fused gate|up rows, float64.

    Follows lfm2/kernels/lk.mojo:154-167 (``gate_up_q4``) and qwen3moe/kernels/moek.mojo:200-210.
    """
    h = gemv_q4(wq, ws, x, group)
    return silu(h[:f]) * h[f:2 * f]


def gemm_q4(wq, ws, x, group: int, y0=None) -> np.ndarray:
    """``Y[M,N] = X[M,K] . deq(W)^T`` (+ ``y0``), float64.

    Follows llama/kernels/prefill/p_gemm_q4.mojo:106-142 (G=64), lfm2/kernels/lk.mojo:458-495 (G=32) and the
    few-token ``t_gemv_q4`` of qwen3moe/kernels/moek.mojo:528-545 (with its ``add`` flag).
    """
    w = q4w_dequant(wq, ws, group).astype(np.float64)
    y = np.asarray(x, dtype=np.float64) @ w.T
    if y0 is not None:
        y = y + np.asarray(y0, dtype=np.float64)
    return y


# ----------------------------------------------------------------------------------------------------------------
# ternary 2-bit words (T2W) and fp16 pairs (X2H)
# ----------------------------------------------------------------------------------------------------------------

T2_GROUP = 128  # weights per ternary scale (bonsai/kernels/prefill.mojo:158-159)


def t2w_pack(codes: np.ndarray) -> np.ndarray:
    """Pack codes [N, K] (0..3) into T2W words [K/16, N]: code of (n, k) at bits 2*(k%16) of word (k/16, n).

    Follows the index map of bonsai/kernels/prefill.mojo:228-230,252-261 (``w[(k/16)*n + col]``) and the transpose
    of qwen3/convert.cpp:64-66.
    """
    codes = np.asarray(codes)
    n, k = codes.shape
    if k % 16:
        raise ValueError("K must be a multiple of 16")
    c = codes.astype(np.uint32).reshape(n, k // 16, 16)
    words = np.bitwise_or.reduce(c << (np.arange(16, dtype=np.uint32) * 2), axis=-1).astype(np.uint32)
    return np.ascontiguousarray(words.T)


def t2w_codes(w: np.ndarray) -> np.ndarray:
    """Codes [N, K] (0..3) of T2W words [K/16, N] (bonsai/kernels/kernels.mojo:209-214)."""
    w = np.asarray(w, dtype=np.uint32)
    kw, n = w.shape
    c = (w.T[..., None] >> (np.arange(16, dtype=np.uint32) * 2)) & np.uint32(3)
    return c.reshape(n, kw * 16).astype(np.int8)


def t2w_dequant(w: np.ndarray, s: np.ndarray) -> np.ndarray:
    """Exact float32 ``(code - 1) * s[k/128, n]`` as [N, K] (bonsai/kernels/prefill.mojo:258-261)."""
    codes = t2w_codes(w).astype(np.float32) - 1.0
    n, k = codes.shape
    sc = np.asarray(s, dtype=np.float16).astype(np.float32)
    if sc.shape != (k // T2_GROUP, n):
        raise ValueError(f"scales must be [K/128, N] = {(k // T2_GROUP, n)}, got {sc.shape}")
    return (codes.reshape(n, k // T2_GROUP, T2_GROUP) * sc.T[:, :, None]).reshape(n, k)


def x2h_pack(x: np.ndarray) -> np.ndarray:
    """fp32 [..., K] -> X2H uint32 [..., K/2]: fp16 (round to nearest even) pairs, even k in the low half.

    Follows qwen3/kernels/qwen3k.mojo:17-19 (``pack``) and :45-48 (``pack_half``).
    """
    h = np.ascontiguousarray(np.asarray(x, dtype=np.float32).astype(np.float16))
    if h.shape[-1] % 2:
        raise ValueError("K must be even")
    return h.view(np.uint32)


def x2h_unpack(q: np.ndarray) -> np.ndarray:
    """X2H uint32 [..., K/2] -> float32 [..., K] (the fp16 values, exactly)."""
    return np.ascontiguousarray(np.asarray(q, dtype=np.uint32)).view(np.float16).astype(np.float32)


def rmsnorm_pack(x, w, eps: float = 1e-6) -> np.ndarray:
    """``pack(x * rsqrt(mean(x^2) + eps) * w)`` (qwen3/kernels/qwen3k.mojo:30-42), fp32 math."""
    x = np.asarray(x, dtype=np.float32)
    r = np.float32(1.0) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + eps)
    return x2h_pack(x * np.float32(r) * np.asarray(w, dtype=np.float32))


def swiglu_pack(gu, n: int) -> np.ndarray:
    """``pack(silu(gate) * up)`` over gu = gate (n) | up (n) (qwen3/kernels/qwen3k.mojo:51-59)."""
    gu = np.asarray(gu, dtype=np.float64)
    return x2h_pack((silu(gu[:n]) * gu[n:2 * n]).astype(np.float32))


def ternary_partials(w, s, xh, n: int, k: int) -> np.ndarray:
    """``partials[g, col] = sum over k in [1024 g, 1024 g + 1024) of W[col, k] x[k]``, float64.

    Follows bonsai/kernels/kernels.mojo:283-325 (``packed_linear``: eight 128-groups per partial, grid
    (ceil(N/64), ceil(K/1024))). Returns [ceil(K/1024), N].
    """
    wd = t2w_dequant(w, s).astype(np.float64)
    x = x2h_unpack(xh).astype(np.float64)
    chunks = (k + 1023) // 1024
    out = np.zeros((chunks, n))
    for g in range(chunks):
        out[g] = wd[:, g * 1024:(g + 1) * 1024] @ x[g * 1024:(g + 1) * 1024]
    return out


def ternary_gemv(w, s, xh, n: int, k: int) -> np.ndarray:
    """``y = deq_T2(W) . x`` with x given as X2H, float64.

    Follows bonsai/kernels/kernels.mojo:283-325 then :437-448 (``packed_linear`` + ``packed_reduce``).
    """
    return t2w_dequant(w, s).astype(np.float64) @ x2h_unpack(xh).astype(np.float64)


def ternary_gemm(x, w, s) -> np.ndarray:
    """``Y[M,N] = X[M,K] . deq_T2(W)^T``, float64 (bonsai/kernels/prefill.mojo:155-164,174-313)."""
    return np.asarray(x, dtype=np.float64) @ t2w_dequant(w, s).astype(np.float64).T


# ----------------------------------------------------------------------------------------------------------------
# MoE: routing, grouping, combine
# ----------------------------------------------------------------------------------------------------------------


def route_top8(logits: np.ndarray, topk: int = 8):
    """Top-k experts per token (descending logit, lowest index among equals) and their weights.

    Follows qwen3moe/kernels/moek.mojo:156-197 (``route``) and :385-425 (``p_route``): iterated argmax with ties to the
    lower index, ``w_k = exp(l_k - l_max) / sum_top exp(l_j - l_max)``. Returns (ids int32 [T, k], weights float64
    [T, k]).
    """
    lg = np.asarray(logits, dtype=np.float32)
    t, e = lg.shape
    # lexsort: last key is primary -> sort by -logit, then by index ascending
    order = np.lexsort((np.broadcast_to(np.arange(e), (t, e)), -lg.astype(np.float64)), axis=1)
    ids = order[:, :topk].astype(np.int32)
    top = np.take_along_axis(lg, ids, axis=1).astype(np.float64)
    ex = np.exp(top - top[:, :1])
    return ids, ex / ex.sum(axis=1, keepdims=True)


def expert_lists(ids: np.ndarray, n_experts: int, capacity: int):
    """Per expert e, the list entries ``i = t*K + k`` with ``ids[i] == e`` in ascending i, and their count.

    Follows qwen3moe/kernels/moek.mojo:432-442 (``p_expert_lists``; there capacity is PMAX = 256). Returns
    (lists int32 [E, capacity] padded with -1, counts int32 [E]).
    """
    flat = np.asarray(ids, dtype=np.int64).ravel()
    lists = np.full((n_experts, capacity), -1, dtype=np.int32)
    counts = np.zeros(n_experts, dtype=np.int32)
    order = np.argsort(flat, kind="stable")
    for i in order:
        e = flat[i]
        if counts[e] >= capacity:
            raise ValueError("expert list overflow")
        lists[e, counts[e]] = i
        counts[e] += 1
    return lists, counts


def expert_items(counts: np.ndarray, tt: int = 8) -> np.ndarray:
    """Work items ``(e, c)`` for c = 0, tt, ... < counts[e], in expert order (qwen3moe/kernels/moek.mojo:548-557).

    Returns int32 [nitems, 2].
    """
    items = [(e, c) for e in range(len(counts)) for c in range(0, int(counts[e]), tt)]
    return np.asarray(items, dtype=np.int32).reshape(-1, 2)


def p_group(ids: np.ndarray, n_experts: int, tm: int):
    """Device grouping of lfm2moe/kernels/mk.mojo:123-161 (``p_group``).

    Histogram ``cnt[e]``; exclusive prefix sum of the counts padded to multiples of ``tm`` (``offs[e]``); permute:
    ``slot[i]`` = grouped row of pair i (ascending i within an expert), ``src[row]`` = its token (-1 on padding);
    work tiles ``(e, first row)`` every ``tm`` rows of an expert's segment, in expert order.
    Returns dict(cnt, offs, slot, src, tiles [ntiles, 2], rows_total).
    """
    ids = np.asarray(ids, dtype=np.int64)
    t, k = ids.shape
    flat = ids.ravel()
    cnt = np.bincount(flat, minlength=n_experts).astype(np.int32)
    padded = (cnt + tm - 1) // tm * tm
    offs = np.concatenate([[0], np.cumsum(padded)[:-1]]).astype(np.int32)
    rows_total = int(padded.sum())
    slot = np.zeros(t * k, dtype=np.int32)
    src = np.full(rows_total, -1, dtype=np.int32)
    fill = offs.copy()
    for i in range(t * k):
        e = flat[i]
        slot[i] = fill[e]
        src[fill[e]] = i // k
        fill[e] += 1
    tiles = [(e, offs[e] + t0) for e in range(n_experts) for t0 in range(0, int(cnt[e]), tm)]
    return dict(cnt=cnt, offs=offs, slot=slot, src=src, tiles=np.asarray(tiles, np.int32).reshape(-1, 2),
                rows_total=rows_total)


def p_gather(x: np.ndarray, src: np.ndarray) -> np.ndarray:
    """Grouped row r = x[src[r]], zeros where src[r] < 0 (lfm2moe/kernels/mk.mojo:164-176)."""
    x = np.asarray(x)
    src = np.asarray(src)
    out = np.zeros((len(src), x.shape[1]), dtype=x.dtype)
    ok = src >= 0
    out[ok] = x[src[ok]]
    return out


def p_combine(yd: np.ndarray, slot: np.ndarray, wts: np.ndarray) -> np.ndarray:
    """``y[t] = sum_k wts[t,k] * yd[slot[t*K+k]]`` in k order (lfm2moe/kernels/mk.mojo:189-199), float64."""
    wts = np.asarray(wts, dtype=np.float64)
    t, k = wts.shape
    yd = np.asarray(yd, dtype=np.float64)
    slot = np.asarray(slot).reshape(t, k)
    y = np.zeros((t, yd.shape[1]))
    for j in range(k):
        y += wts[:, j:j + 1] * yd[slot[:, j]]
    return y


def moe_layer(x, logits, gu_q, gu_s, dn_q, dn_s, group: int, fe: int, topk: int = 8, residual=None):
    """One Qwen3-MoE expert block: route, SwiGLU experts, weighted combine, float64.

    ``y[t] = (residual[t] +) sum_k w[t,k] * down_e(silu(gate_e x[t]) * up_e x[t])`` with e = ids[t,k].
    Expert e's gate rows are gu rows ``e*2F .. e*2F+F-1``, up rows ``e*2F+F ..`` and down rows ``e*D ..``
    (qwen3moe/export.py:17-18 stacking; arithmetic of qwen3moe/kernels/moek.mojo:200-223 for one token and
    :479-488,560-608 for a batch). Returns (y float64 [T, D], ids, weights).
    """
    x = np.asarray(x, dtype=np.float32)
    t, d = x.shape
    ids, wts = route_top8(logits, topk)
    y = np.zeros((t, d)) if residual is None else np.asarray(residual, dtype=np.float64).copy()
    for e in np.unique(ids):
        tok, kk = np.nonzero(ids == e)
        gu = q4w_dequant(gu_q[e * 2 * fe:(e + 1) * 2 * fe], gu_s[e * 2 * fe:(e + 1) * 2 * fe], group)
        dn = q4w_dequant(dn_q[e * d:(e + 1) * d], dn_s[e * d:(e + 1) * d], group)
        h = x[tok].astype(np.float64) @ gu.astype(np.float64).T
        a = silu(h[:, :fe]) * h[:, fe:]
        out = a @ dn.astype(np.float64).T
        y[tok] += wts[tok, kk][:, None] * out
    return y, ids, wts


# ----------------------------------------------------------------------------------------------------------------
# Llama decode step (embedding, RMSNorm, RoPE, attention over the KV cache, SwiGLU MLP, lm_head, greedy argmax)
# ----------------------------------------------------------------------------------------------------------------


def rmsnorm(x, w, eps: float = 1e-5) -> np.ndarray:
    """``x / sqrt(mean(x^2) + eps) * w``, float64 (llama/kernels/rmsnorm.mojo:17-35; w fp16)."""
    x = np.asarray(x, dtype=np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * np.asarray(w, dtype=np.float64)


def rope(v, cos_p, sin_p) -> np.ndarray:
    """rotate_half RoPE of head vectors ``v [..., 64]`` at one position: pairs (i, i + 32) ->
    ``(a c_i - b s_i, b c_i + a s_i)`` (llama/kernels/rope_kv.mojo:27-33), float64."""
    v = np.asarray(v, dtype=np.float64)
    h = v.shape[-1] // 2
    a, b = v[..., :h], v[..., h:]
    c, s = np.asarray(cos_p, dtype=np.float64), np.asarray(sin_p, dtype=np.float64)
    return np.concatenate([a * c - b * s, b * c + a * s], axis=-1)


def attention_decode(q, kc, vc, n: int) -> np.ndarray:
    """Grouped-query attention of one token over cache rows s < n: ``out_h = softmax_s(q_h . k_s / sqrt(d)) . v_s`` with
    KV head h // (H / KVH) (llama/kernels/attention.mojo:19-66). q [H, d], kc/vc [KVH, P, d] -> [H, d], float64."""
    q = np.asarray(q, dtype=np.float64)
    heads, d = q.shape
    kv = kc.shape[0]
    out = np.empty((heads, d))
    for h in range(heads):
        g = h // (heads // kv)
        k = np.asarray(kc[g, :n], dtype=np.float64)
        sc = (k @ q[h]) / np.sqrt(d)
        p = np.exp(sc - sc.max())
        out[h] = (p @ np.asarray(vc[g, :n], dtype=np.float64)) / p.sum()
    return out


def argmax_first(v) -> int:
    """The first index of the largest value (llama/llama.mojo:72-75: ``if logits[i] > logits[best]``); numpy's argmax
    returns the first occurrence of the maximum."""
    return int(np.argmax(np.asarray(v)))


class LlamaDecodeOracle:
    """One-token-at-a-time Llama decode, float64 on dequantised weights: the forward pass of llama/model.mojo:140-166
    (embed; per layer rmsnorm, qkv, rope_kv, attention, o + residual, rmsnorm, gate|up, silu_mul, down + residual;
    final rmsnorm, lm_head). ``kv_dtype`` rounds what the cache stores (np.float16 for an fp16 cache, None to keep
    float64, as the reference's fp32 cache is for these purposes).

    ``arrays`` as ``aq.llama.LlamaWeights.from_numpy`` takes them; ``cos``/``sin`` [max_pos, d/2] tables."""

    def __init__(self, arrays: dict, cfg, cos, sin, kv_dtype=np.float16, weights_dtype=np.float64):
        self.cfg, self.cos, self.sin, self.kv_dtype = cfg, np.asarray(cos), np.asarray(sin), kv_dtype
        g = cfg.group
        # the dequantised weights are exact in float32 (int4 times fp16); float32 storage halves the memory of a
        # whole-depth model and changes no product, since every matrix-vector product is taken in float64 (_mv)
        deq = lambda name: q4w_dequant(arrays[name + ".q"], arrays[name + ".s"], g).astype(weights_dtype,  # noqa: E731
                                                                                       copy=False)
        self.embed = np.asarray(arrays["embed"], dtype=np.float16)
        self.layers = []
        for i in range(cfg.layers):
            p = f"l{i}."
            self.layers.append({"attn_norm": np.asarray(arrays[p + "attn_norm"], np.float16),
                                "mlp_norm": np.asarray(arrays[p + "mlp_norm"], np.float16),
                                **{m: deq(p + m) for m in ("wqkv", "wo", "wgu", "wdown")}})
        self.final_norm = np.asarray(arrays["final_norm"], np.float16)
        self.lm = deq("lm")
        shape = (cfg.kv_heads, cfg.max_pos, cfg.head_dim)
        self.kc = [np.zeros(shape) for _ in range(cfg.layers)]
        self.vc = [np.zeros(shape) for _ in range(cfg.layers)]

    def _store(self, v):
        return v.astype(self.kv_dtype).astype(np.float64) if self.kv_dtype is not None else v

    @staticmethod
    def _mv(w, x):
        """w @ x in float64, in row blocks (a float32 w is widened one block at a time)."""
        if w.dtype == np.float64:
            return w @ x
        return np.concatenate([w[r:r + 4096].astype(np.float64) @ x for r in range(0, w.shape[0], 4096)])

    def step(self, token: int, pos: int) -> np.ndarray:
        """Logits (float64 [vocab]) of ``token`` at ``pos``; appends this position's keys and values to the cache."""
        cfg = self.cfg
        hd, nh, nkv = cfg.head_dim, cfg.heads, cfg.kv_heads
        x = self.embed[token].astype(np.float64)
        for i, lw in enumerate(self.layers):
            qkv = self._mv(lw["wqkv"], rmsnorm(x, lw["attn_norm"], cfg.eps))
            q = rope(qkv[:nh * hd].reshape(nh, hd), self.cos[pos], self.sin[pos])
            k = rope(qkv[nh * hd:(nh + nkv) * hd].reshape(nkv, hd), self.cos[pos], self.sin[pos])
            v = qkv[(nh + nkv) * hd:].reshape(nkv, hd)
            self.kc[i][:, pos] = self._store(k)
            self.vc[i][:, pos] = self._store(v)
            att = attention_decode(q, self.kc[i], self.vc[i], pos + 1)
            x = x + self._mv(lw["wo"], att.reshape(-1))
            h = self._mv(lw["wgu"], rmsnorm(x, lw["mlp_norm"], cfg.eps))
            x = x + self._mv(lw["wdown"], silu(h[:cfg.ffn]) * h[cfg.ffn:])
        return self._mv(self.lm, rmsnorm(x, self.final_norm, cfg.eps))


# ----------------------------------------------------------------------------------------------------------------
# weight formats (host side)
# ----------------------------------------------------------------------------------------------------------------


def quantize4(w16: np.ndarray, group: int = 64):
    """Symmetric int4 per group: ``s = fp16(max|w| / 7)``, ``q = clip(rint(w / s), -8, 7)`` (0 where s == 0).

    Follows llama/run.py:56-70 (``quantize4``, float32 math on fp16 input; llama/st2bin.c:49-66 is the same in C).
    Returns (Q4W words [N, K/8], fp16 scales [N, K/G], exact dequantised float32 [N, K]).
    """
    w = np.asarray(w16, dtype=np.float16).astype(np.float32)
    n, k = w.shape
    wg = w.reshape(n, k // group, group)
    s16 = (np.abs(wg).max(-1) / np.float32(7)).astype(np.float16)
    sf = s16.astype(np.float32)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(sf > 0, np.rint(wg / sf), np.float32(0))
    q = np.clip(q, -8, 7).astype(np.int32).reshape(n, k)
    return q4w_pack(q), s16, (q.reshape(n, k // group, group) * sf).reshape(n, k).astype(np.float32)


def quantize4_searched(w: np.ndarray, group: int):
    """int4 with the least-squared-error scale: ``s = fp16(m / d)`` for d = 6.5, 6.75, ..., 9 (first minimum wins).

    Follows qwen3moe/convert.c:120-159 (= gemma4/convert.c:57-81): float32 arithmetic throughout, the error summed
    in element order, ``rintf`` (ties to even), a scale that is not > 0 ends the search. ``w`` holds the bf16 inputs
    as float32. Returns (Q4W words [N, K/8], fp16 scales [N, K/G]).
    """
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    if k % group or group % 8 or group > 256:
        raise ValueError("bad group")
    wg = w.reshape(-1, group)
    m = np.abs(wg).max(axis=1)
    best = np.full(len(wg), np.inf, dtype=np.float32)
    sf = np.zeros(len(wg), dtype=np.float32)
    alive = np.ones(len(wg), dtype=bool)
    d = np.float32(6.5)
    while d <= np.float32(9.0):
        t = (m / d).astype(np.float16).astype(np.float32)
        alive &= t > 0
        e = np.zeros(len(wg), dtype=np.float32)
        tt = np.where(alive, t, np.float32(1))
        for j in range(group):
            v = np.clip(np.rint(wg[:, j] / tt), np.float32(-8), np.float32(7)).astype(np.float32)
            r = (wg[:, j] - v * tt).astype(np.float32)
            e = (e + r * r).astype(np.float32)
        better = alive & (e < best)
        best = np.where(better, e, best)
        sf = np.where(better, t, sf)
        d = np.float32(d + np.float32(0.25))
    s16 = sf.astype(np.float16)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(sf[:, None] > 0, np.clip(np.rint(wg / np.where(sf > 0, sf, 1)[:, None]), -8, 7), 0)
    return q4w_pack(q.astype(np.int32).reshape(n, k)), s16.reshape(n, k // group)


def gguf_q4_0_to_q4w(raw: bytes | np.ndarray, rows: int, cols: int):
    """GGUF Q4_0 blocks (18 bytes: fp16 d, 16 bytes qs) -> Q4W words and fp16 scales (G=32).

    Element j < 16 of a block is the low nibble of qs[j], element j + 16 its high nibble; the stored Q4W nibble is
    ``nib ^ 8`` and the scale is copied. Follows lfm2/convert.c:59-71 (``q4_block``).
    """
    b = np.frombuffer(bytes(raw), np.uint8).reshape(rows * cols // 32, 18)
    d = b[:, :2].copy().view(np.float16).reshape(rows, cols // 32)
    qs = b[:, 2:]
    nib = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.uint32) ^ np.uint32(8)  # [blocks, 32]
    words = np.bitwise_or.reduce(nib.reshape(-1, 4, 8) << (np.arange(8, dtype=np.uint32) * 4), axis=-1)
    return words.astype(np.uint32).reshape(rows, cols // 8), d


def gguf_q4_0_dequant(raw: bytes | np.ndarray, rows: int, cols: int) -> np.ndarray:
    """ggml's Q4_0 dequantisation ``(nib - 8) * d`` (lfm2/weights.py:61-68, lfm2/convert.c:73-80)."""
    b = np.frombuffer(bytes(raw), np.uint8).reshape(-1, 18)
    d = b[:, :2].copy().view(np.float16).astype(np.float32)
    qs = b[:, 2:]
    q = np.concatenate([(qs & 15).astype(np.int8) - 8, (qs >> 4).astype(np.int8) - 8], axis=1)
    return (q.astype(np.float32) * d).reshape(rows, cols)


def gguf_q6_k_to_q6w(raw: bytes | np.ndarray, rows: int, cols: int):
    """GGUF Q6_K super-blocks (210 bytes: ql[128], qh[64], int8 scales[16], fp16 d) -> Q6W: the first 208 bytes of
    each super-block [rows, cols/256, 208] and d fp16 [rows, cols/256] (lfm2/convert.c:148-155, recipe "q6")."""
    b = np.frombuffer(bytes(raw), np.uint8).reshape(rows, cols // 256, 210)
    return b[:, :, :208].copy(), b[:, :, 208:].copy().view(np.float16).reshape(rows, cols // 256)


def q6w_values(q: np.ndarray, d: np.ndarray):
    """Q6W -> (q6 - 32 as int [rows, cols], per-16 scales d * sc as float32 [rows, cols/16]).

    Element 128 h + 32 j + l of a super-block (h < 2, j < 4, l < 32) is the low (j < 2) or high nibble of
    ql[64 h + 32 (j % 2) + l] with bits 2 j, 2 j + 1 of qh[32 h + l] above it, minus 32; its scale is
    sc[8 h + 2 j + l // 16] (lfm2/convert.c:82-103 ``q6_dequant``; lfm2/kernels/lk.mojo:88-129 ``q6_chunk``).
    """
    rows, nb, _ = q.shape
    ql = q[:, :, :128].reshape(rows, nb, 2, 2, 32).astype(np.int32)   # [.., h, j % 2, l]
    qh = q[:, :, 128:192].reshape(rows, nb, 2, 1, 32).astype(np.int32)  # [.., h, -, l]
    sc = q[:, :, 192:208].view(np.int8).reshape(rows, nb, 2, 4, 2).astype(np.float32)  # [.., h, j, l // 16]
    lo = np.concatenate([ql & 15, ql >> 4], axis=3)                     # j = 0, 1 low nibbles; 2, 3 high
    hi = (qh >> (2 * np.arange(4).reshape(1, 1, 1, 4, 1))) & 3
    vals = (lo | (hi << 4)) - 32                                         # [rows, nb, h, j, l]
    ds = d.astype(np.float32).reshape(rows, nb, 1, 1, 1) * sc            # fp32 d * sc
    return vals.reshape(rows, nb * 256), ds.reshape(rows, nb * 16)


def q6w_dequant(q: np.ndarray, d: np.ndarray) -> np.ndarray:
    """ggml's Q6_K dequantisation ``(d * sc) * (q - 32)``, float32 step by step (lfm2/convert.c:82-103, as
    lfm2/kernels/lk.mojo ``embed_q6`` writes it)."""
    vals, ds = q6w_values(q, d)
    return (np.repeat(ds, 16, axis=1) * vals.astype(np.float32)).astype(np.float32)


def gemv_q6(q: np.ndarray, d: np.ndarray, x: np.ndarray) -> np.ndarray:
    """``y[r] = E[r] . x`` over a Q6W matrix, float64 of the dequantised weights (lfm2/kernels/lk.mojo:179-191
    ``head_q6``)."""
    return q6w_dequant(q, d).astype(np.float64) @ np.asarray(x, np.float64)


def bonsai_pairs_to_t2w_scales(params: np.ndarray) -> np.ndarray:
    """bonsai/convert.cpp:44-61 (``emitPacked``) stores each 128-group's fp16 scale and bias as an fp32 pair
    [K/128, N, 2] next to the transposed codes; a ternary group has bias == -scale, and T2W keeps the scale in fp16
    (exact: it came from fp16). ValueError for any other group."""
    p = np.asarray(params, np.float32)
    sc, b = p[..., 0], p[..., 1]
    if np.any(b != -sc) or np.any(sc.astype(np.float16).astype(np.float32) != sc):
        raise ValueError("not ternary, or a scale that fp16 does not hold")
    return sc.astype(np.float16)


def mlx_to_t2w(parts, k: int):
    """MLX 2-bit affine matrices -> one fused T2W matrix (qwen3/convert.cpp:39-74, ``addPacked``).

    ``parts`` is a list of (codes uint32 [n_i, K/16], scales fp16 [n_i, K/128], biases fp16 [n_i, K/128]). Every group
    must be ternary (``bias == -scale``) or ValueError is raised. Returns (w uint32 [K/16, sum n_i],
    s fp16 [K/128, sum n_i]).
    """
    ws, ss = [], []
    for codes, scales, biases in parts:
        sc = np.asarray(scales, np.float16).astype(np.float32)
        bi = np.asarray(biases, np.float16).astype(np.float32)
        if np.any(bi != -sc):
            raise ValueError("not ternary (bias != -scale)")
        ws.append(np.asarray(codes, np.uint32))
        ss.append(np.asarray(scales, np.float16))
    w = np.ascontiguousarray(np.concatenate(ws, axis=0).T)
    s = np.ascontiguousarray(np.concatenate(ss, axis=0).T)
    return w, s
