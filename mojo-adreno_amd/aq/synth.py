"""Seeded synthetic inputs for the benchmark configurations (numpy ``default_rng``; no checkpoints are used).

C0 int4 decode GEMV (Llama-3.2-1B FFN up, 8192 x 2048), C1 int4 prefill GEMM (Llama-3.2-1B projections, M = 431),
C2 ternary GEMV/GEMM (Qwen3-8B shapes), C3 Qwen3-30B-A3B MoE layer (128 experts, top 8), C4 Llama-3.2-1B decode
step (``llama_arrays``; the benchmark draws the full-size model on the device, ``aq.llama.LlamaWeights.random``). Weight values follow the
stated distributions: int4 offset-8 values uniform in 0..15 (the stored nibble ``q ^ 8`` is then uniform too, so
the packed words are uniform 32-bit integers), fp16 scales ``|N(0, 0.02)| + 1e-3`` per 32-weight group; ternary
codes uniform in {0, 1, 2} with fp16 scales ``|N(0, 0.02)|`` per 128.
"""
from __future__ import annotations

import numpy as np

LLAMA_1B = dict(hidden=2048, ffn=8192, heads=32, kv_heads=8, head_dim=64, layers=16, vocab=128256)

# C1: every Llama-3.2-1B layer projection as (name, N, K)
C1_PROJECTIONS = (("q", 2048, 2048), ("k", 512, 2048), ("v", 512, 2048), ("o", 2048, 2048),
                  ("gate", 8192, 2048), ("up", 8192, 2048), ("down", 2048, 8192))
C1_TOKENS = 431

QWEN3_8B = dict(hidden=4096, ffn=12288)
C2_GEMM_TOKENS = 412

QWEN3_MOE = dict(experts=128, hidden=2048, ffn=768, topk=8, group=32)
C3_TOKENS = 404


LFM2_HEAD = dict(vocab=128000, hidden=2048)  # LFM2.5's tied Q6_K embedding / output head (lfm2/README.md:116)
BONSAI_HEAD = dict(vocab=248320, hidden=2048)  # Bonsai's ternary vocabulary head (bonsai/bonsai_vk.c:39)


def q6_matrix(rng: np.random.Generator, rows: int, cols: int):
    """Q6W: q uint8 [rows, cols/256, 208] with uniform ql/qh bytes and int8 scales uniform in [-32, 31], and
    d fp16 [rows, cols/256] = |N(0, 0.001)| + 1e-5 (ggml's Q6_K quantizer gives per-16 scales of that kind)."""
    nb = cols // 256
    q = rng.integers(0, 256, size=(rows, nb, 208), dtype=np.uint8)
    q[:, :, 192:] = rng.integers(-32, 32, size=(rows, nb, 16), dtype=np.int8).view(np.uint8)
    d = (np.abs(rng.standard_normal((rows, nb), dtype=np.float32) * np.float32(0.001)) + np.float32(1e-5))
    return q, d.astype(np.float16)


def int4_matrix(rng: np.random.Generator, n: int, k: int, group: int = 32):
    """Q4W words [n, k/8] (uniform nibbles) and fp16 scales [n, k/group] = |N(0, 0.02)| + 1e-3."""
    wq = rng.integers(0, 2 ** 32, size=(n, k // 8), dtype=np.uint32)
    ws = (np.abs(rng.standard_normal((n, k // group), dtype=np.float32) * np.float32(0.02))
          + np.float32(1e-3)).astype(np.float16)
    return wq, ws


def ternary_matrix(rng: np.random.Generator, n: int, k: int, group: int = 128):
    """T2W words [k/16, n] with codes uniform in {0, 1, 2} and fp16 scales [k/group, n] = |N(0, 0.02)|."""
    codes = rng.integers(0, 3, size=(n, k), dtype=np.uint32)
    c = codes.reshape(n, k // 16, 16) << (np.arange(16, dtype=np.uint32) * 2)
    words = np.bitwise_or.reduce(c, axis=-1).astype(np.uint32)
    s = np.abs(rng.standard_normal((k // group, n), dtype=np.float32) * np.float32(0.02)).astype(np.float16)
    return np.ascontiguousarray(words.T), s


def c0(seed: int = 0, n: int = 8192, k: int = 2048, group: int = 32):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(k, dtype=np.float32)
    wq, ws = int4_matrix(rng, n, k, group)
    return dict(x=x, wq=wq, ws=ws, n=n, k=k, group=group)


def c1(seed: int = 1, tokens: int = C1_TOKENS, group: int = 32, projections=C1_PROJECTIONS):
    rng = np.random.default_rng(seed)
    mats = {}
    for name, n, k in projections:
        mats[name] = int4_matrix(rng, n, k, group)
    xs = {k: rng.standard_normal((tokens, k), dtype=np.float32).astype(np.float16)
          for k in sorted({k for _, _, k in projections})}
    return dict(mats=mats, x=xs, tokens=tokens, group=group, projections=projections)


def c2(seed: int = 2, tokens: int = C2_GEMM_TOKENS):
    rng = np.random.default_rng(seed)
    h, f = QWEN3_8B["hidden"], QWEN3_8B["ffn"]
    mats = {"gate": ternary_matrix(rng, f, h), "up": ternary_matrix(rng, f, h), "down": ternary_matrix(rng, h, f)}
    shapes = {"gate": (f, h), "up": (f, h), "down": (h, f)}
    xs = {kk: rng.standard_normal((tokens, kk), dtype=np.float32).astype(np.float16) for kk in (h, f)}
    xv = {kk: rng.standard_normal(kk, dtype=np.float32).astype(np.float16) for kk in (h, f)}
    return dict(mats=mats, shapes=shapes, x=xs, xv=xv, tokens=tokens)


def c3(seed: int = 3, tokens: int = C3_TOKENS, experts: int = 128, hidden: int = 2048, ffn: int = 768,
       group: int = 32):
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((tokens, experts), dtype=np.float32)
    x = rng.standard_normal((tokens, hidden), dtype=np.float32)
    gu_q, gu_s = int4_matrix(rng, experts * 2 * ffn, hidden, group)
    dn_q, dn_s = int4_matrix(rng, experts * hidden, ffn, group)
    return dict(logits=logits, x=x, gu_q=gu_q, gu_s=gu_s, dn_q=dn_q, dn_s=dn_s, experts=experts, hidden=hidden,
                ffn=ffn, group=group, tokens=tokens)


def llama_arrays(cfg, seed: int = 4) -> dict:
    """Host arrays of a random Llama model of shape ``cfg`` (an ``aq.llama.LlamaConfig``), in the names
    ``aq.llama.LlamaWeights.from_numpy`` takes: int4 linears as ``int4_matrix``, fp16 norm weights N(1, 0.1), fp16
    embedding N(0, 1)."""
    rng = np.random.default_rng(seed)
    d, f = cfg.dim, cfg.ffn
    a = {"embed": rng.standard_normal((cfg.vocab, d), dtype=np.float32).astype(np.float16)}
    norm = lambda: (1 + 0.1 * rng.standard_normal(d, dtype=np.float32)).astype(np.float16)  # noqa: E731
    for i in range(cfg.layers):
        p = f"l{i}."
        a[p + "attn_norm"] = norm()
        a[p + "mlp_norm"] = norm()
        for name, (n, k) in (("wqkv", (cfg.qkv, d)), ("wo", (d, cfg.heads * cfg.head_dim)), ("wgu", (2 * f, d)),
                             ("wdown", (d, f))):
            a[p + name + ".q"], a[p + name + ".s"] = int4_matrix(rng, n, k, cfg.group)
    a["final_norm"] = norm()
    a["lm.q"], a["lm.s"] = int4_matrix(rng, cfg.vocab, d, cfg.group)
    return a
