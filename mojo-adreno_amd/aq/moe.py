"""Host plan of a Qwen3-MoE expert block on the aq kernels (the role of qwen3moe/model.mojo:207-214 for a token and
:253-266 for a prompt, and of lfm2moe/model.mojo:468-492's grouped prefill).

Prompt (T tokens): route (top-k of the router logits) -> group (device histogram, padded prefix sum, stable
permute, work tiles of ``tm`` rows) -> fp32 tokens rounded to fp16 once -> grouped gate|up GEMM with the SwiGLU
product in its epilogue (fp16 activations) -> grouped down GEMM -> weighted combine in k order (+ residual). Decode
(one token): route -> gate|up over the k chosen experts -> down summed over them. All buffers are allocated once, at construction, for at most
``max_tokens`` tokens; a forward call allocates nothing and never synchronises with the host.
"""
from __future__ import annotations

import torch

from . import _lib, ops


class MoeBlock:
    """Expert weights in the reference's stacked layout (qwen3moe/export.py:17-18): gate|up Q4W
    ``[E * 2F, D/8]`` (expert e's gate rows at e*2F, up rows at e*2F + F) and down Q4W ``[E * D, F/8]``."""

    def __init__(self, gu_q, gu_s, dn_q, dn_s, experts: int, hidden: int, ffn: int, group: int, topk: int = 8,
                 max_tokens: int = 512, tm: int = 32):
        self.gu_q, self.gu_s, self.dn_q, self.dn_s = gu_q, gu_s, dn_q, dn_s
        self.E, self.D, self.F, self.G, self.K, self.tm = experts, hidden, ffn, group, topk, tm
        dev = gu_q.device
        i32 = dict(dtype=torch.int32, device=dev)
        self.max_tokens = max_tokens
        self.max_rows = _lib.lib().aq_moe_group_max_rows(max_tokens, topk, experts, tm)
        self.max_tiles = _lib.lib().aq_moe_group_max_tiles(max_tokens, topk, experts, tm)
        self.ids = torch.empty((max_tokens, topk), **i32)
        self.wts = torch.empty((max_tokens, topk), dtype=torch.float32, device=dev)
        self.counts = torch.empty(experts, **i32)
        self.offs = torch.empty(experts + 1, **i32)
        self.slot = torch.empty(max_tokens * topk, **i32)
        self.src = torch.empty(self.max_rows, **i32)
        self.tiles = torch.empty(2 * self.max_tiles, **i32)
        self.ntiles = torch.empty(1, **i32)
        self.act = torch.empty((self.max_rows, ffn), dtype=torch.float16, device=dev)
        self.xq = torch.empty((max_tokens, hidden // 2), **i32)  # fp32 tokens rounded to fp16 once (pairs)
        self.yd = torch.empty((self.max_rows, hidden), dtype=torch.float32, device=dev)
        self.a1 = torch.empty((topk, ffn), dtype=torch.float32, device=dev)
        self.none = torch.empty(0, **i32)

    def forward(self, x: torch.Tensor, logits: torch.Tensor, out: torch.Tensor, add: bool = False):
        """out[t] (+)= sum_k w[t,k] * down_e(silu(gate_e x[t]) * up_e x[t]) for T <= max_tokens tokens."""
        t = x.shape[0]
        if t > self.max_tokens:
            raise ValueError(f"{t} tokens > max_tokens {self.max_tokens}")
        ids, wts = self.ids[:t], self.wts[:t]
        ops_ = torch.ops.aq
        if x.dtype == torch.float32 and x.shape[1] % 8 == 0:
            # routing and one rounding of x to fp16 (instead of one per expert tile in the GEMM) in one launch
            ops_.moe_route_pack(logits, ids, wts, self.K, x, self.xq[:t])
            x = self.xq[:t].view(torch.float16)
        else:
            ops_.moe_route(logits, ids, wts, self.K)
        ops_.moe_group(ids, self.E, self.tm, self.counts, self.offs, self.slot[:t * self.K], self.src, self.tiles,
                       self.ntiles)
        if x.dtype == torch.float32:  # one rounding to fp16 here, instead of one per expert tile in the GEMM
            ops_.pack_half(x, self.xq[:t])
            x = self.xq[:t].view(torch.float16)
        ops_.moe_gemm_q4(x, self.src, self.gu_q, self.gu_s, self.E, self.G, self.tiles, self.ntiles, self.tm, True,
                         self.act)
        ops_.moe_gemm_q4(self.act, self.none, self.dn_q, self.dn_s, self.E, self.G, self.tiles, self.ntiles, self.tm,
                         False, self.yd)
        ops_.moe_combine(self.yd, self.slot[:t * self.K], wts, out, add)

    def decode(self, x: torch.Tensor, logits: torch.Tensor, out: torch.Tensor, add: bool = False):
        """One token: out (+)= sum_k w_k * down_{e_k}(silu(gate x) * up x)."""
        ids, wts = self.ids[:1], self.wts[:1]
        torch.ops.aq.moe_route(logits.reshape(1, -1), ids, wts, self.K)
        torch.ops.aq.moe_gate_up_q4(self.gu_q, self.gu_s, self.E, ids.reshape(-1), x, self.a1, self.G)
        torch.ops.aq.moe_down_q4(self.dn_q, self.dn_s, self.E, ids.reshape(-1), wts.reshape(-1), self.a1, out, self.G,
                                 add)
