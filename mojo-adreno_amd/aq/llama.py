"""Llama-3.2-1B-architecture decode on the aq kernels: int4 (Q4W) weights on every linear including the lm_head, an
fp16 embedding table, an fp16 KV cache, fp32 activations.

The role of the reference's ``Llama.forward`` + ``Llama.head`` (llama/model.mojo:128-166) and of the greedy loop of
llama/llama.mojo:50-80 (one token at a time; its batched ``prefill`` is the GEMM path, not this one). A step is
1 + 5 per layer + 2 launches:

    embed(token)                                   aq_embed_f16
    per layer:  qkv = Wqkv . rmsnorm(x)           aq_rmsnorm_gemv_q4      (rmsnorm fused into the x staging)
                att = attention(rope(qkv), cache)  aq_attn_decode_split    (RoPE + cache append + softmax . V over
                                                                            spans of positions: partial states)
                x += Wo . att                      aq_attn_out_q4          (the spans combined on staging)
                a = silu(Wg . rmsnorm(x)) * (Wu . rmsnorm(x))   aq_rmsnorm_gate_up_q4
                x += Wdown . a                     aq_gemv_q4 (add)
    logits = Wlm . rmsnorm(x); token = argmax      aq_head_argmax_q4        (argmax on the device)

The token and the position live in device memory: a step reads them and its last launch writes the argmax token and
advances the position, so a captured step (``capture``) replays token after token with no host work between.
Every buffer is allocated at construction; a step allocates nothing.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from . import ops  # noqa: F401  (registers torch.ops.aq.*)


@dataclass(frozen=True)
class LlamaConfig:
    """Llama-3.2-1B by default (llama/model.mojo:31-41; llama/run.py:36-41 for the RoPE scaling)."""
    dim: int = 2048
    layers: int = 16
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 64
    ffn: int = 8192
    vocab: int = 128256
    max_pos: int = 512
    group: int = 32
    eps: float = 1e-5
    rope_theta: float = 500000.0
    rope_factor: float = 32.0       # Llama 3 frequency scaling ("llama3" rope type); factor 1 with
    rope_low: float = 1.0           # rope_orig 0 turns it off
    rope_high: float = 4.0
    rope_orig: int = 8192

    @property
    def qkv(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    def weight_bytes(self) -> int:
        """Bytes of the int4 linears (words + fp16 scales) a decode step streams: every layer's and the lm_head."""
        per = lambda n, k: n * k // 2 + n * (k // self.group) * 2  # noqa: E731
        d, f = self.dim, self.ffn
        layer = per(self.qkv, d) + per(d, self.heads * self.head_dim) + per(2 * f, d) + per(d, f)
        return self.layers * layer + per(self.vocab, d)

    def kv_bytes(self, n: int) -> int:
        """fp16 KV-cache bytes a step at context n reads (keys and values of every layer)."""
        return self.layers * 2 * self.kv_heads * n * self.head_dim * 2


def rope_tables(cfg: LlamaConfig):
    """cos/sin float32 [max_pos, head_dim/2] of the rotate_half RoPE, with Llama 3's frequency scaling.

    The reference exports these tables from transformers' rotary embedding (llama/run.py:161-163); this evaluates the
    same published rule in float32 on the CPU: inv_freq_i = 1 / theta^(2i/d); frequencies whose wavelength exceeds
    rope_orig/rope_low are divided by the factor, those under rope_orig/rope_high are kept, and those between are
    interpolated with smooth = (rope_orig / wavelength - rope_low) / (rope_high - rope_low); angle = pos * inv_freq.
    """
    d = cfg.head_dim
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))
    if cfg.rope_orig:
        wavelen = 2 * math.pi / inv
        low_wl = cfg.rope_orig / cfg.rope_low
        high_wl = cfg.rope_orig / cfg.rope_high
        scaled = torch.where(wavelen > low_wl, inv / cfg.rope_factor, inv)
        smooth = (cfg.rope_orig / wavelen - cfg.rope_low) / (cfg.rope_high - cfg.rope_low)
        mid = (1 - smooth) * scaled / cfg.rope_factor + smooth * scaled
        medium = ~(wavelen < high_wl) & ~(wavelen > low_wl)
        inv = torch.where(medium, mid, scaled)
    ang = inv[None, :, None].float() @ torch.arange(cfg.max_pos, dtype=torch.float32)[None, None, :]
    ang = ang.transpose(1, 2)[0]
    return (np.ascontiguousarray(ang.cos().numpy(), dtype=np.float32),
            np.ascontiguousarray(ang.sin().numpy(), dtype=np.float32))


class LlamaWeights:
    """Device tensors of one model: ``embed`` fp16 [vocab, dim]; per layer ``attn_norm``, ``mlp_norm`` fp16 [dim] and
    Q4W pairs (words int32 [N, K/8], fp16 scales [N, K/group]) ``wqkv`` [qkv, dim] (q | k | v rows, as
    llama/run.py:115-117 fuses them), ``wo`` [dim, dim], ``wgu`` [2 ffn, dim] (gate | up) and ``wdown`` [dim, ffn];
    ``final_norm`` fp16 [dim] and ``lm`` [vocab, dim]."""

    def __init__(self, cfg: LlamaConfig, embed, layers, final_norm, lm):
        self.cfg, self.embed, self.layers, self.final_norm, self.lm = cfg, embed, layers, final_norm, lm

    @staticmethod
    def from_numpy(cfg: LlamaConfig, arrays: dict, device) -> "LlamaWeights":
        """From host arrays: ``embed``, ``final_norm``, ``lm.q``/``lm.s`` and ``l{i}.{name}`` (``.q``/``.s`` for the
        int4 matrices)."""
        dev = torch.device(device)

        def t(a, dtype=None):
            a = np.ascontiguousarray(a)
            if a.dtype == np.uint32:
                a = a.view(np.int32)
            return torch.from_numpy(a).to(dev)

        layers = []
        for i in range(cfg.layers):
            p = f"l{i}."
            layers.append({"attn_norm": t(arrays[p + "attn_norm"]), "mlp_norm": t(arrays[p + "mlp_norm"]),
                           **{m: (t(arrays[p + m + ".q"]), t(arrays[p + m + ".s"]))
                              for m in ("wqkv", "wo", "wgu", "wdown")}})
        return LlamaWeights(cfg, t(arrays["embed"]), layers, t(arrays["final_norm"]),
                            (t(arrays["lm.q"]), t(arrays["lm.s"])))

    @staticmethod
    def random(cfg: LlamaConfig, seed: int, device) -> "LlamaWeights":
        """Random init on the device (no host copy): int4 values uniform in -8..7 (uniform words), scales
        |N(0, 0.02)| + 1e-3, norm weights N(1, 0.1), embedding N(0, 1), all rounded to fp16."""
        dev = torch.device(device)
        g = torch.Generator(device=dev)
        g.manual_seed(seed)

        def q4(n, k):
            wq = torch.randint(-2 ** 31, 2 ** 31 - 1, (n, k // 8), dtype=torch.int32, device=dev, generator=g)
            ws = (torch.randn((n, k // cfg.group), device=dev, generator=g).abs() * 0.02 + 1e-3).half()
            return wq, ws

        def norm():
            return (1 + 0.1 * torch.randn(cfg.dim, device=dev, generator=g)).half()

        d, f = cfg.dim, cfg.ffn
        embed = torch.randn((cfg.vocab, d), device=dev, generator=g).half()
        layers = [{"attn_norm": norm(), "wqkv": q4(cfg.qkv, d), "wo": q4(d, cfg.heads * cfg.head_dim),
                   "mlp_norm": norm(), "wgu": q4(2 * f, d), "wdown": q4(d, f)} for _ in range(cfg.layers)]
        return LlamaWeights(cfg, embed, layers, norm(), q4(cfg.vocab, d))


class LlamaDecoder:
    """Greedy one-token-at-a-time decode. ``forward(token, pos)`` runs one step and returns the logits (the reference's
    ``Llama.forward``); ``generate`` runs a prompt and new tokens, the new ones as replays of a captured step."""

    def __init__(self, weights: LlamaWeights):
        cfg = self.cfg = weights.cfg
        if cfg.dim != cfg.heads * cfg.head_dim:
            raise ValueError("dim must equal heads * head_dim")
        self.w = weights
        dev = self.device = weights.embed.device
        f32 = dict(dtype=torch.float32, device=dev)
        self.x = torch.zeros(cfg.dim, **f32)
        self.qkv = torch.zeros(cfg.qkv, **f32)
        # split attention: spans of >= 64 positions, at most 8 (the states are combined by the o projection)
        self.splits = max(1, min(ops.ATTN_MAX_SPLITS, cfg.max_pos // 64))
        self.parts = torch.zeros(ops.attn_parts_numel(cfg.heads, self.splits), **f32)
        self.act = torch.zeros(cfg.ffn, **f32)
        self.logits = torch.zeros(cfg.vocab, **f32)
        shape = (cfg.kv_heads, cfg.max_pos, cfg.head_dim)
        self.kc = [torch.zeros(shape, dtype=torch.float16, device=dev) for _ in range(cfg.layers)]
        self.vc = [torch.zeros(shape, dtype=torch.float16, device=dev) for _ in range(cfg.layers)]
        cos, sin = rope_tables(cfg)
        self.cos, self.sin = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
        self.cand = torch.zeros(ops.HEAD_CANDIDATES, dtype=torch.int64, device=dev)
        self.token = torch.zeros(1, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self.hist = torch.full((cfg.max_pos,), -1, dtype=torch.int32, device=dev)
        self.graph = None

    def step(self, advance: int = 1) -> None:
        """Enqueue one decode step of the token in ``self.token`` at position ``self.pos``."""
        cfg, w, a = self.cfg, self.w, torch.ops.aq
        a.embed_f16(w.embed, self.token, self.x)
        for i, lw in enumerate(w.layers):
            a.rmsnorm_gemv_q4(*lw["wqkv"], self.x, lw["attn_norm"], cfg.eps, self.qkv, cfg.group)
            a.attn_decode_split(self.qkv, self.cos, self.sin, self.kc[i], self.vc[i], self.pos, cfg.heads,
                                cfg.kv_heads, self.splits, self.parts)
            a.attn_out_q4(*lw["wo"], self.parts, self.splits, self.x, cfg.group)
            a.rmsnorm_gate_up_q4(*lw["wgu"], self.x, lw["mlp_norm"], cfg.eps, self.act, cfg.group)
            a.gemv_q4(*lw["wdown"], self.act, self.x, cfg.group, True)
        a.head_argmax_q4(*w.lm, self.x, w.final_norm, cfg.eps, self.logits, cfg.group, self.cand, self.token, self.pos,
                         self.hist, advance)

    def forward(self, token: int, pos: int) -> torch.Tensor:
        """Logits [vocab] of ``token`` at position ``pos`` (the cache must hold positions < pos)."""
        if not 0 <= pos < self.cfg.max_pos:
            raise ValueError(f"position {pos} outside [0, {self.cfg.max_pos})")
        self.token.fill_(int(token))
        self.pos.fill_(int(pos))
        self.step(advance=1)
        return self.logits

    def capture(self, advance: int = 1) -> torch.cuda.CUDAGraph:
        """A HIP graph of one step (warmed up once eagerly first, which runs a step at the current token and
        position: capture before a run, not in the middle of one)."""
        saved_t, saved_p = self.token.clone(), self.pos.clone()
        self.step(advance=0)
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step(advance=advance)
        self.token.copy_(saved_t)
        self.pos.copy_(saved_p)
        self.graph = g
        return g

    def generate(self, prompt: list[int], max_new: int, eos=()) -> list[int]:
        """Greedy decode: the prompt one token at a time, then ``max_new`` tokens (stopping after the first in
        ``eos``), as llama/llama.mojo:50-80 does without LLAMA_PREFILL. The new tokens are graph replays with the token
        and position carried on the device; the host reads them once at the end."""
        n = len(prompt)
        if n < 1 or n + max_new > self.cfg.max_pos + 1:
            raise ValueError("prompt + new tokens exceed the cache")
        if self.graph is None:
            self.capture()
        self.hist.fill_(-1)
        self.pos.fill_(0)
        for t in prompt:  # forced tokens: the host writes each before its step
            self.token.fill_(int(t))
            self.graph.replay()
        for _ in range(max_new - 1):
            self.graph.replay()
        toks = self.hist[n - 1:n - 1 + max_new].cpu().tolist()
        for i, t in enumerate(toks):
            if t in eos:
                return toks[:i + 1]
        return toks
