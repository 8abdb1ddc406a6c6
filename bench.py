"""Benchmark of the weight-quantized matmul path on one MI355X; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-cpu]
    python bench.py --profile dominant|copy|decode|heads|gemvs|moe   # short runs for rocprofv3 passes

Workload (BASELINE.json metric "int4 GEMV GB/s (% of 8 TB/s) at M=1; prefill GEMM TFLOP/s; MoE layer ms"):
  value     C1 int4 prefill GEMM TFLOP/s: one step = one Llama-3.2-1B layer's projections at M = 431 fp16 tokens
            (fused q|k|v 3072 x 2048, o 2048 x 2048, fused gate|up 16384 x 2048, down 2048 x 8192; G = 32), the
            layer's weights rotating over 16 distinct layers (547 MB, more than the 256 MB Infinity Cache). FLOPs
            count the true M (2 * 431 * 60.8 M weights = 52.4 GFLOP a step).
  roofline  the dominant kernel, k_gemm_x16 on C1's gate|up (431 x 16384 x 2048, 28.9 GFLOP a launch), timed as a
            graph burst of 48 launches with HIP events on its stream; traffic = HBM bytes a launch from the committed
            rocprofv3 FETCH_SIZE / WRITE_SIZE passes (profiles/), scaled by a plain copy's counter reading.
  gemv_c0   C0 int4 decode GEMV (8192 x 2048, G = 32, fp32 x/y) GB/s over a rotating pool of >= 512 MB of distinct
            weight copies: graph burst (time per launch) and single cold launch.
  decode_c4 C4 Llama-3.2-1B decode step at context 512 (int4 linears incl. lm_head, fp16 KV cache): tokens/s of
            graph-replayed steps, and GB/s over the 711.9 MB a step must read.
  heads     output heads with their device argmax (LFM2.5 Q6_K 128000 x 2048, Bonsai ternary 248320 x 2048,
            Llama int4 128256 x 2048): microseconds and GB/s over weight copies rotating past the Infinity Cache.
The K timed steps are replayed from hipGraphs.
Inputs are synthetic (seeded), resident in HBM before the timed region. ``--gpus N`` with N > 1 exits: this build
measures one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

T_START = time.perf_counter()
ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "mojo-adreno_amd"))

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0


def _dev(a, dev):
    import numpy as np
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a).to(dev)


def _gemv_bytes(n, k, group, tokens=1):
    return n * k // 2 + n * (k // group) * 2 + tokens * k * 4 + tokens * n * 4


class GraphTimer:
    """Capture a list of launches into one hipGraph; time replays with events on the replay stream."""

    def __init__(self, launches):
        import torch
        self.stream = torch.cuda.Stream()
        self.graph = torch.cuda.CUDAGraph()
        for fn in launches:  # run once eagerly (sets kernel attributes outside capture)
            fn()
        torch.cuda.synchronize()
        with torch.cuda.graph(self.graph, stream=self.stream):
            for fn in launches:
                fn()
        torch.cuda.synchronize()

    def time(self, replays: int) -> float:
        """Seconds per replay (the stream is pre-filled with a sleep so host submission is not timed)."""
        import torch
        with torch.cuda.stream(self.stream):
            self.graph.replay()
            torch.cuda.synchronize()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda._sleep(2_000_000)
            start.record()
            for _ in range(replays):
                self.graph.replay()
            end.record()
            end.synchronize()
        return start.elapsed_time(end) / 1e3 / replays


class ReadCeiling:
    """The streaming-read ceiling of a matrix-vector launch: aq_stream_read over the same number of bytes (every 16
    bytes loaded once with the weights' streaming cache policy, nothing decoded), timed like the GEMVs (a graph burst
    over distinct slices of a pool larger than the 256 MB Infinity Cache), the best of several workgroup counts."""

    BLOCKS = (0, 1024, 2048, 4096)

    def __init__(self, dev, pool_mb: int = 640):
        import torch
        from aq import ops  # noqa: F401  (registers torch.ops.aq)
        self.pool = torch.empty(pool_mb << 18, dtype=torch.int32, device=dev)  # contents are not read for meaning
        self.sink = torch.empty(4 * 8192, dtype=torch.int32, device=dev)
        self.cache = {}

    def us(self, nbytes: int) -> float:
        import torch
        n = -(-nbytes // 16) * 16
        if n in self.cache:
            return self.cache[n]
        stride = -(-n // 4096) * 4096  # distinct 4 KB-aligned slices
        copies = max(2, min(256, self.pool.numel() * 4 // stride))
        best = float("inf")
        for blocks in self.BLOCKS:
            launches = [(lambda i=i: torch.ops.aq.stream_read(self.pool[i * stride // 4:(i * stride + n) // 4],
                                                              self.sink, blocks)) for i in range(copies)]
            best = min(best, GraphTimer(launches).time(replays=3) / copies)
        self.cache[n] = round(best * 1e6, 3)
        return self.cache[n]


def bench_gemv_c0(dev, steps: int, warmup: int, pool_mb: int = 600):
    """C0 int4 GEMV: burst (graph of distinct-copy launches) and single cold launch."""
    import numpy as np
    import torch
    from aq import ops, synth
    d = synth.c0()
    n, k, g = d["n"], d["k"], d["group"]
    per = _gemv_bytes(n, k, g)
    copies = max(2, int(pool_mb * 1e6 // per))
    wq0, ws0 = _dev(d["wq"], dev), _dev(d["ws"], dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(100)
    pool = [(wq0, ws0)]
    for _ in range(copies - 1):
        wq = torch.randint(-2 ** 31, 2 ** 31 - 1, wq0.shape, dtype=torch.int32, device=dev, generator=gen)
        ws = (torch.rand(ws0.shape, device=dev, generator=gen) * 0.03 + 1e-3).to(torch.float16)
        pool.append((wq, ws))
    x = _dev(d["x"], dev)
    y = torch.empty(n, dtype=torch.float32, device=dev)
    launches = [(lambda wq=wq, ws=ws: ops.gemv_q4(wq, ws, x, y, g)) for wq, ws in pool]
    # one graph per step block: steps launches rotating over the pool
    seq = [launches[i % copies] for i in range(max(steps, 1))]
    timer = GraphTimer(seq)
    for _ in range(max(warmup, 1)):
        timer.graph.replay()
    torch.cuda.synchronize()
    t_step = timer.time(replays=1) / len(seq)
    # longer burst for a stable per-op figure
    t_burst = min(timer.time(replays=3) / len(seq), t_step)
    # single cold launches (distinct copy each time, sleep-prefilled stream)
    cold = []
    s = torch.cuda.current_stream()
    for i in range(1, min(copies, 21)):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1_000_000)
        a.record()
        launches[i]()
        b.record()
        b.synchronize()
        cold.append(a.elapsed_time(b) / 1e3)
    s.synchronize()
    t_cold = float(np.median(cold))
    return dict(bytes=per, wbytes=n * k // 2 + n * (k // g) * 2, flop=2 * n * k, t_step=t_step, t_burst=t_burst, t_cold=t_cold, pool_copies=copies,
                pool_mb=round(copies * per / 1e6, 1), steps=len(seq))


C1_LAYER = (("qkv", 3072, 2048), ("o", 2048, 2048), ("gate_up", 16384, 2048), ("down", 2048, 8192))


def bench_gemm_c1(dev, steps: int, warmup: int, layers: int = 16):
    """C1: one layer's four (fused) projection GEMMs a step, weights rotating over `layers` distinct layers."""
    import numpy as np
    import torch
    from aq import ops, synth
    m, g = synth.C1_TOKENS, 32
    rng = np.random.default_rng(1)
    gen = torch.Generator(device=dev)
    gen.manual_seed(101)
    xs = {k: _dev(rng.standard_normal((m, k), dtype=np.float32).astype(np.float16), dev) for k in (2048, 8192)}
    ys = {name: torch.empty((m, n), dtype=torch.float32, device=dev) for name, n, _ in C1_LAYER}
    weights = []
    for layer in range(layers):
        lw = {}
        for name, n, k in C1_LAYER:
            if layer == 0:
                wq, ws = synth.int4_matrix(rng, n, k, g)
                lw[name] = (_dev(wq, dev), _dev(ws, dev))
            else:
                wq = torch.randint(-2 ** 31, 2 ** 31 - 1, (n, k // 8), dtype=torch.int32, device=dev, generator=gen)
                ws = (torch.rand((n, k // g), device=dev, generator=gen) * 0.03 + 1e-3).to(torch.float16)
                lw[name] = (wq, ws)
        weights.append(lw)

    def launch(layer, name):
        k = dict((nm, kk) for nm, _, kk in C1_LAYER)[name]
        wq, ws = weights[layer][name]
        return lambda: ops.gemm_q4(xs[k], wq, ws, ys[name], g)

    flop_step = sum(2 * m * n * k for _, n, k in C1_LAYER)
    step_launches = [[launch(l, name) for name, _, _ in C1_LAYER] for l in range(layers)]
    nsteps = max(steps, 1)
    seq = [fn for i in range(nsteps) for fn in step_launches[i % layers]]
    timer = GraphTimer(seq)
    for _ in range(max(warmup, 1)):
        timer.graph.replay()
    torch.cuda.synchronize()
    t_step = timer.time(replays=1) / nsteps
    per = {}
    for name, n, k in C1_LAYER:
        tt = GraphTimer([launch(l, name) for l in range(layers)] * 2).time(replays=3) / (2 * layers)
        per[name] = dict(us=round(tt * 1e6, 3), tflops=round(2 * m * n * k / tt / 1e12, 2))
    return dict(flop=flop_step, t_step=t_step, steps=nsteps, per_gemm=per, layers=layers,
                weights_mb=round(layers * sum(n * k * 0.5625 for _, n, k in C1_LAYER) / 1e6, 1))


DOMINANT = "k_gemm_x16<0, 7, 4, false, false, 0, true>"  # the fused gate|up launch of C1 (16384 x 2048, M = 431)
DOMINANT_SHAPE = (431, 16384, 2048)


def _gate_up_launches(dev, layers: int = 16):
    """The dominant kernel's launches: C1's gate|up GEMM over `layers` distinct weight copies."""
    import torch
    from aq import ops
    m, n, k = DOMINANT_SHAPE
    gen = torch.Generator(device=dev)
    gen.manual_seed(104)
    x = torch.randn((m, k), device=dev, generator=gen).to(torch.float16)
    y = torch.empty((m, n), dtype=torch.float32, device=dev)
    ws = [(torch.randint(-2 ** 31, 2 ** 31 - 1, (n, k // 8), dtype=torch.int32, device=dev, generator=gen),
           (torch.rand((n, k // 32), device=dev, generator=gen) * 0.03 + 1e-3).to(torch.float16))
          for _ in range(layers)]
    return [(lambda wq=wq, s_=s_: ops.gemm_q4(x, wq, s_, y, 32)) for wq, s_ in ws]


def time_dominant(dev, rounds: int = 3):
    """Average duration of one dominant-kernel launch: a hipGraph of `rounds` passes over the 16 weight copies,
    replayed with HIP events recorded on the replay stream (the stream the kernels run on), divided by the launches.
    The per-launch figure includes the graph's inter-kernel gap (about 1 us), so it sits slightly above the
    kernel-trace average."""
    launches = _gate_up_launches(dev) * rounds
    t = GraphTimer(launches).time(replays=3) / len(launches)
    m, n, k = DOMINANT_SHAPE
    return dict(kernel=DOMINANT, flop=2 * m * n * k, t=t, launches=len(launches))


def profile_run(dev, what: str):
    """Short runs for rocprofv3 counter passes (see profiles/): the dominant kernel alone, or a plain copy of known
    size that calibrates FETCH_SIZE / WRITE_SIZE."""
    import torch
    if what == "dominant":
        launches = _gate_up_launches(dev)
        for fn in launches:
            fn()
    elif what == "decode":  # C4: 20 graph-replayed decode steps at context 512
        bench_decode_c4(dev, replays=20)
    elif what == "heads":  # the three output heads with their argmax (and their streaming-read ceilings)
        bench_heads(dev, ReadCeiling(dev))
    elif what == "gemvs":  # the C4 step's GEMVs one at a time (and their streaming-read ceilings)
        bench_gemv_c4(dev, ReadCeiling(dev))
    elif what == "moe":  # C3: the block at 404 tokens and one token at a time
        bench_moe_c3(dev)
    else:
        nbytes = 256 << 20
        a = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).fill_(1.0)
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        for _ in range(4):
            b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"profile": what, "done": True}), flush=True)


def load_traffic():
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes."""
    f = ROOT / "profiles" / "k_gemm_x16_c1_gate_up_traffic.json"
    if not f.exists():
        return None
    d = json.loads(f.read_text())
    return d.get("traffic_bytes") if d.get("kernel") == DOMINANT else None


def _t2_gemv_bytes(n, k):
    return (k // 16) * n * 4 + (k // 128) * n * 2 + k * 2 + n * 4


# The reference's Qwen3 MLP: gate and up fused along N into one T2W matrix "gu" (qwen3/convert.cpp:118), one
# projection over 2F outputs (qwen3/model.mojo:165 decode, :230 prefill), then down.
C2_MATS = (("gu", 24576, 4096), ("down", 4096, 12288))


def _c2_first(rng):
    """Copy 0 of the C2 weights from the seeded generator: gate and up (12288 x 4096) fused along N, then down."""
    import numpy as np
    from aq import synth
    g, u, d = (synth.ternary_matrix(rng, n, k) for n, k in ((12288, 4096), (12288, 4096), (4096, 12288)))
    return {"gu": (np.concatenate([g[0], u[0]], axis=1), np.concatenate([g[1], u[1]], axis=1)), "down": d}


def bench_ternary_c2(dev, pool_mb: int = 560):
    """C2: ternary GEMV (M=1) over a rotating pool of distinct MLP weight sets (gate|up fused, down), and ternary GEMM
    at M=412."""
    import numpy as np
    import torch
    from aq import ops, synth
    gen = torch.Generator(device=dev)
    gen.manual_seed(102)
    per_layer = sum(_t2_gemv_bytes(n, k) for _, n, k in C2_MATS)
    copies = max(2, int(pool_mb * 1e6 // per_layer))
    rng = np.random.default_rng(2)
    first = _c2_first(rng)
    mats = []
    for c in range(copies):
        trip = {}
        for name, n, k in C2_MATS:
            if c == 0:
                trip[name] = (_dev(first[name][0], dev), _dev(first[name][1], dev))
            else:  # random 2-bit codes (3 would decode to +2; timing does not depend on the values)
                w = torch.randint(-2 ** 31, 2 ** 31 - 1, (k // 16, n), dtype=torch.int32, device=dev, generator=gen)
                s_ = (torch.rand((k // 128, n), device=dev, generator=gen) * 0.02).to(torch.float16)
                trip[name] = (w, s_)
        mats.append(trip)
    xh = {k: torch.randint(0, 2 ** 14, (k // 2,), dtype=torch.int32, device=dev, generator=gen) for k in (4096, 12288)}
    ys = {name: torch.empty(n, dtype=torch.float32, device=dev) for name, n, _ in C2_MATS}
    launches = [(lambda w=m[name][0], s_=m[name][1], k=k, y=ys[name]: ops.t2_gemv(xh[k], w, s_, y))
                for m in mats for name, _, k in C2_MATS]
    t_all = GraphTimer(launches).time(replays=3)
    gemv = dict(gbs=round(copies * per_layer / t_all / 1e9, 2), us_per_layer=round(t_all / copies * 1e6, 3),
                frac_hbm=round(copies * per_layer / t_all / 1e9 / HBM_PEAK_GBS, 4), pool_mb=round(copies * per_layer / 1e6, 1))
    m = synth.C2_GEMM_TOKENS
    xs = {k: torch.randn((m, k), device=dev, generator=gen).to(torch.float16) for k in (4096, 12288)}
    yg = {name: torch.empty((m, n), dtype=torch.float32, device=dev) for name, n, _ in C2_MATS}
    gl = [(lambda w=mm[name][0], s_=mm[name][1], k=k, y=yg[name]: ops.gemm_t2(xs[k], w, s_, y))
          for mm in mats[:4] for name, _, k in C2_MATS]
    t_g = GraphTimer(gl).time(replays=3) / min(4, copies)
    flop = sum(2 * m * n * k for _, n, k in C2_MATS)
    gemm = dict(tflops=round(flop / t_g / 1e12, 2), us_per_layer=round(t_g * 1e6, 3),
                frac_mfma=round(flop / t_g / 1e12 / MFMA_F16_PEAK_TFLOPS, 4), tokens=m)
    return dict(gemv=gemv, gemm=gemm)


def bench_moe_c3(dev):
    """C3: Qwen3-30B-A3B-shaped MoE block at 404 tokens (grouped prefill) and at 1 token (decode), over two distinct
    expert weight sets (2 x 340 MB) alternating, so the 256 MB Infinity Cache cannot hold them."""
    import numpy as np
    import torch
    from aq import moe, synth
    d = synth.c3()
    sets = []
    gen = torch.Generator(device=dev)
    gen.manual_seed(103)
    for c in range(2):
        if c == 0:
            w = [_dev(d[kk], dev) for kk in ("gu_q", "gu_s", "dn_q", "dn_s")]
        else:
            w = [torch.randint(-2 ** 31, 2 ** 31 - 1, t.shape, dtype=torch.int32, device=dev, generator=gen)
                 if t.dtype == torch.int32 else (torch.rand(t.shape, device=dev, generator=gen) * 0.03 + 1e-3).half()
                 for t in sets[0]._w]
        blk = moe.MoeBlock(*w, 128, 2048, 768, 32, 8, max_tokens=404, tm=32)
        blk._w = w
        sets.append(blk)
    x = _dev(d["x"], dev)
    logits = _dev(d["logits"], dev)
    out = torch.empty((404, 2048), dtype=torch.float32, device=dev)
    t404 = GraphTimer([lambda b=b: b.forward(x, logits, out) for b in sets]).time(replays=5) / 2
    # one token at a time: 16 different tokens (so different experts, whose rows come from HBM rather than the
    # Infinity Cache) over both weight sets
    toks = [(x[i].contiguous(), logits[i].contiguous()) for i in range(16)]
    o1 = torch.empty(2048, dtype=torch.float32, device=dev)
    calls = [(lambda b=b, xt=xt, lt=lt: b.decode(xt, lt, o1)) for xt, lt in toks for b in sets]
    t1 = GraphTimer(calls).time(replays=10) / len(calls)
    wbytes = 128 * (1536 * 2048 + 2048 * 768) * 0.5625
    return dict(ms_404=round(t404 * 1e3, 4), ms_1=round(t1 * 1e3, 4),
                gbs_404_weights=round(wbytes / t404 / 1e9, 1),
                gbs_1_active=round(8 * (1536 * 2048 + 2048 * 768) * 0.5625 / t1 / 1e9, 1),
                tokens_1_rotation=len(toks))


def bench_decode_c4(dev, replays: int = 40):
    """C4: a full Llama-3.2-1B-architecture decode step (random int4 weights drawn on the device, 695 MB of linears,
    fp16 embedding table) at context 512: the KV cache holds random fp16 rows 0..510 and the step at position 511
    appends row 511 and attends over all 512. One step = 83 launches replayed from one hipGraph (the token each step
    feeds back is the previous step's device argmax; the position stays at 511)."""
    import torch
    from aq.llama import LlamaConfig, LlamaDecoder, LlamaWeights
    cfg = LlamaConfig()
    dec = LlamaDecoder(LlamaWeights.random(cfg, 4, dev))
    gen = torch.Generator(device=dev)
    gen.manual_seed(104)
    for kc, vc in zip(dec.kc, dec.vc):
        kc.normal_(generator=gen)
        vc.normal_(generator=gen)
    dec.token.fill_(128000)
    dec.pos.fill_(cfg.max_pos - 1)
    t = GraphTimer([lambda: dec.step(advance=0)]).time(replays=replays)
    nbytes = cfg.weight_bytes() + cfg.kv_bytes(cfg.max_pos)
    out = dict(tok_s=round(1 / t, 1), us_per_token=round(t * 1e6, 2), bytes_per_token=nbytes,
               gbs=round(nbytes / t / 1e9, 1), frac_hbm=round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4), context=512,
               launches_per_step=1 + 5 * cfg.layers + 2)
    del dec
    torch.cuda.empty_cache()
    return out


def bench_gemv_c4(dev, ceil: ReadCeiling, pool_mb: int = 600, names=None):
    """The C4 decode step's int4 GEMVs one at a time, each launched as the step launches it: q|k|v with the attention
    RMSNorm fused into its x staging, o combining the split-attention states while staging, gate|up with the MLP
    RMSNorm and the SwiGLU product fused, down adding into the residual, and the lm_head with the final RMSNorm and
    the device argmax (two launches). Microseconds per launch by graph burst over a rotating pool of distinct weight
    copies (more than the Infinity Cache holds), beside ReadCeiling's time for the same weight and scale bytes."""
    import torch
    from aq import ops
    from aq.llama import LlamaConfig
    cfg = LlamaConfig()
    d, f, g = cfg.dim, cfg.ffn, cfg.group
    gen = torch.Generator(device=dev)
    gen.manual_seed(106)
    x = torch.randn(d, device=dev, generator=gen)
    xf = torch.randn(f, device=dev, generator=gen)
    norm = (torch.rand(d, device=dev, generator=gen) + 0.5).half()
    splits = max(1, min(ops.ATTN_MAX_SPLITS, cfg.max_pos // 64))
    parts = torch.randn(ops.attn_parts_numel(cfg.heads, splits), device=dev, generator=gen)
    ml = parts[cfg.heads * splits * 64:].view(-1, 2)
    ml[:, 0] = 0.0
    ml[:, 1] = 1.0
    qkv = torch.empty(cfg.qkv, dtype=torch.float32, device=dev)
    act = torch.empty(f, dtype=torch.float32, device=dev)
    res = torch.zeros(d, dtype=torch.float32, device=dev)
    logits = torch.empty(cfg.vocab, dtype=torch.float32, device=dev)
    cand = torch.zeros(ops.HEAD_CANDIDATES, dtype=torch.int64, device=dev)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    hist = torch.empty(0, dtype=torch.int32, device=dev)
    a = torch.ops.aq
    shapes = {  # name: (rows, K, launch)
        "qkv": (cfg.qkv, d, lambda m: a.rmsnorm_gemv_q4(m[0], m[1], x, norm, cfg.eps, qkv, g)),
        "o": (d, cfg.heads * cfg.head_dim, lambda m: a.attn_out_q4(m[0], m[1], parts, splits, res, g)),
        "gate_up": (2 * f, d, lambda m: a.rmsnorm_gate_up_q4(m[0], m[1], x, norm, cfg.eps, act, g)),
        "down": (d, f, lambda m: a.gemv_q4(m[0], m[1], xf, res, g, True)),
        "lm_head": (cfg.vocab, d, lambda m: a.head_argmax_q4(m[0], m[1], x, norm, cfg.eps, logits, g, cand, tok, pos,
                                                             hist, 0)),
    }
    out = {}
    for name, (rows, k, launch) in shapes.items():
        if names and name not in names:
            continue
        wbytes = rows * k // 2 + rows * (k // g) * 2
        copies = max(2, int(pool_mb * 1e6 // wbytes))
        mats = [(torch.randint(-2 ** 31, 2 ** 31 - 1, (rows, k // 8), dtype=torch.int32, device=dev, generator=gen),
                 (torch.rand((rows, k // g), device=dev, generator=gen) * 0.03 + 1e-3).half()) for _ in range(copies)]
        t = GraphTimer([lambda m=m: launch(m) for m in mats]).time(replays=5) / copies
        del mats
        torch.cuda.empty_cache()
        read = ceil.us(wbytes)
        out[name] = dict(us=round(t * 1e6, 3), read_us=read, frac_of_read=round(read / (t * 1e6), 3),
                         gbs=round(wbytes / t / 1e9, 1), mb=round(wbytes / 1e6, 2), pool_copies=copies)
    return out


def _q6_bytes(rows, cols):
    return rows * (cols // 256) * 210 + cols * 4 + rows * 4


def bench_heads(dev, ceil: ReadCeiling, pool_mb: int = 640):
    """Output heads with their device argmax (head GEMV + argmax step, two launches): LFM2.5's Q6_K tied head
    (128000 x 2048), Bonsai's ternary head (248320 x 2048, X2H input) and Llama-3.2-1B's int4 lm_head (128256 x 2048,
    G = 32), each over a rotating pool of distinct weight copies larger than the 256 MB Infinity Cache. Bytes a
    launch: the weights (and their scales), x and the logits."""
    import torch
    from aq import ops, synth
    gen = torch.Generator(device=dev)
    gen.manual_seed(105)
    cand = torch.zeros(max(ops.HEAD_CANDIDATES, ops.t2_head_candidates(synth.BONSAI_HEAD["vocab"], synth.BONSAI_HEAD["hidden"])),
                       dtype=torch.int64, device=dev)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    hist = torch.empty(0, dtype=torch.int32, device=dev)
    nonorm = torch.empty(0, dtype=torch.float16, device=dev)
    out = {}

    def run(name, per, make, launch):
        copies = max(2, int(pool_mb * 1e6 // per))
        mats = [make() for _ in range(copies)]
        t = GraphTimer([lambda m=m: launch(m) for m in mats]).time(replays=5) / copies
        read = ceil.us(per)
        out[name] = dict(us=round(t * 1e6, 2), gbs=round(per / t / 1e9, 1), frac_hbm=round(per / t / 1e9 / HBM_PEAK_GBS, 4),
                         mb=round(per / 1e6, 1), pool_copies=copies, read_us=read, frac_of_read=round(read / (t * 1e6), 3))
        del mats
        torch.cuda.empty_cache()

    v, k = synth.LFM2_HEAD["vocab"], synth.LFM2_HEAD["hidden"]
    x = torch.randn(k, device=dev, generator=gen)
    lg = torch.empty(v, dtype=torch.float32, device=dev)
    run("q6_lfm2", _q6_bytes(v, k),
        lambda: (torch.randint(0, 256, (v, k // 256, 208), dtype=torch.uint8, device=dev, generator=gen),
                 (torch.rand((v, k // 256), device=dev, generator=gen) * 1e-3).half()),
        lambda m: torch.ops.aq.head_argmax_q6(m[0], m[1], x, nonorm, 1e-5, lg, cand, tok, pos, hist, 0))
    v, k = synth.BONSAI_HEAD["vocab"], synth.BONSAI_HEAD["hidden"]
    xh = torch.randint(0, 2 ** 14, (k // 2,), dtype=torch.int32, device=dev, generator=gen)
    lg = torch.empty(v, dtype=torch.float32, device=dev)
    run("t2_bonsai", _t2_gemv_bytes(v, k),
        lambda: (torch.randint(-2 ** 31, 2 ** 31 - 1, (k // 16, v), dtype=torch.int32, device=dev, generator=gen),
                 (torch.rand((k // 128, v), device=dev, generator=gen) * 0.02).half()),
        lambda m: torch.ops.aq.t2_head_argmax(xh, m[0], m[1], lg, cand, tok, pos, hist, 0))
    v, k = synth.LLAMA_1B["vocab"], synth.LLAMA_1B["hidden"]
    lg = torch.empty(v, dtype=torch.float32, device=dev)
    run("q4_llama", _gemv_bytes(v, k, 32),
        lambda: (torch.randint(-2 ** 31, 2 ** 31 - 1, (v, k // 8), dtype=torch.int32, device=dev, generator=gen),
                 (torch.rand((v, k // 32), device=dev, generator=gen) * 0.03 + 1e-3).half()),
        lambda m: torch.ops.aq.head_argmax_q4(m[0], m[1], x, nonorm, 1e-5, lg, 32, cand, tok, pos, hist, 0))
    return out


def cpu_baseline_decode():
    import numpy as np
    from aq import synth
    from aq.llama import LlamaConfig
    from oracle import cpu_baseline as cb
    cores = cb.threads()
    cfg, sample = LlamaConfig(), 2
    rng = np.random.default_rng(4)
    d, f = cfg.dim, cfg.ffn
    mats = [{name: synth.int4_matrix(rng, n, k, 32) for name, n, k in
             (("wqkv", cfg.qkv, d), ("wo", d, d), ("wgu", 2 * f, d), ("wdown", d, f))} for _ in range(sample)]
    t_layers, t_head = cb.llama_decode(mats, synth.int4_matrix(rng, cfg.vocab, d, 32), d, cfg.heads, cfg.kv_heads, f,
                                       cfg.max_pos, 32)
    per_token = t_head + t_layers * cfg.layers / sample
    return dict(value=round(1 / per_token, 2), unit="tokens/s", cores=cores, kind="port",
                sample=f"C4 decode at context 512: {sample} of 16 layers + lm_head/argmax timed (torch fp32 over "
                       f"dequantised weights, fp32 cache, median of <=5 reps on {cb.cpu_model()}), "
                       f"per token = head + 8 x the 2 layers")


def cpu_baseline_gemm():
    import numpy as np
    from aq import synth
    from oracle import cpu_baseline as cb
    cores = cb.threads()
    rng = np.random.default_rng(1)
    mats = {name: synth.int4_matrix(rng, n, k, 32) for name, n, k in C1_LAYER}
    xs = {k: rng.standard_normal((synth.C1_TOKENS, k), dtype=np.float32).astype(np.float16) for k in (2048, 8192)}
    t = cb.gemm_layer(mats, xs, 32)
    flop = sum(2 * synth.C1_TOKENS * n * k for _, n, k in C1_LAYER)
    return dict(value=round(flop / t / 1e12, 4), unit="TFLOP/s", cores=cores, kind="port",
                sample=f"C1 one layer (4 fused projections, M=431, 52.4 GFLOP): torch fp32 F.linear over dequantised "
                       f"weights, median of <=5 reps on {cb.cpu_model()}")


def cpu_baseline_gemv():
    from aq import synth
    from oracle import cpu_baseline as cb
    cores = cb.threads()
    d = synth.c0()
    t_mm, t_all = cb.gemv_q4(d["wq"], d["ws"], d["x"], d["group"])
    per = _gemv_bytes(d["n"], d["k"], d["group"])
    return dict(value=round(per / t_mm / 1e9, 2), unit="GB/s", cores=cores, kind="port",
                sample=f"C0 GEMV 8192x2048: torch fp32 mv over the dequantised matrix, median of <=20 reps on "
                       f"{cb.cpu_model()}; dequant+mv {per / t_all / 1e9:.2f} GB/s")


def cpu_baseline_ternary():
    from aq import synth
    from oracle import cpu_baseline as cb
    cores = cb.threads()
    import numpy as np
    d = synth.c2()
    g, u = d["mats"]["gate"], d["mats"]["up"]
    mats = {"gu": (np.concatenate([g[0], u[0]], axis=1), np.concatenate([g[1], u[1]], axis=1)),
            "down": d["mats"]["down"]}
    t_mv, t_mm = cb.ternary(mats, d["xv"], d["x"])
    per = sum(_t2_gemv_bytes(n, k) for _, n, k in C2_MATS)
    flop = sum(2 * d["tokens"] * n * k for _, n, k in C2_MATS)
    return dict(value=round(per / t_mv / 1e9, 2), unit="GB/s", cores=cores, kind="port",
                gemm_tflops=round(flop / t_mm / 1e12, 4),
                sample=f"C2 MLP, gate|up fused (24576x4096) and down (4096x12288): torch fp32 mv (value, over the "
                       f"layer's T2W bytes) and F.linear at M={d['tokens']} (gemm_tflops) over the dequantised "
                       f"matrices, median of <=20 / <=5 reps on {cb.cpu_model()}")


def cpu_baseline_moe():
    from aq import synth
    from oracle import cpu_baseline as cb
    cores = cb.threads()
    t = cb.moe_block(synth.c3())
    return dict(value=round(t * 1e3, 3), unit="ms", cores=cores, kind="port",
                sample=f"C3 block at 404 tokens: transformers-style fp32 torch (softmax, top-8, renormalise, loop over "
                       f"the hit experts with index_add_) over dequantised experts, median of <=5 reps on "
                       f"{cb.cpu_model()}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--profile", choices=("dominant", "copy", "decode", "heads", "gemvs", "moe"),
                    help="short run for a rocprofv3 pass: the dominant kernel, a calibration copy, C4 decode steps, "
                         "the output heads, the C4 step's GEMVs one at a time or the C3 MoE block")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every kernel runs on one GPU's share)",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    if args.profile:
        profile_run(dev, args.profile)
        return
    torch.cuda.synchronize()
    legs = {}  # wall-clock seconds of each leg (setup, warmup, timing and checks included)

    def leg(name, fn, *a):
        t = time.perf_counter()
        res = fn(*a)
        torch.cuda.synchronize()
        legs[name] = round(time.perf_counter() - t, 2)
        return res

    c1 = leg("c1", bench_gemm_c1, dev, args.steps, args.warmup)
    r = leg("c0", bench_gemv_c0, dev, 128, 10)
    c2 = leg("c2", bench_ternary_c2, dev)
    c3 = leg("c3", bench_moe_c3, dev)
    c4 = leg("c4", bench_decode_c4, dev)
    ceil = ReadCeiling(dev)
    c4["gemvs"] = leg("c4_gemvs", bench_gemv_c4, dev, ceil)
    heads = leg("heads", bench_heads, dev, ceil)
    c0_read = ceil.us(r["wbytes"])
    dom = leg("roofline", time_dominant, dev)
    value = c1["flop"] / c1["t_step"] / 1e12
    achieved = dom["flop"] / dom["t"] / 1e12
    gemv = r["bytes"] / r["t_burst"] / 1e9
    out = {
        "metric": "int4 GEMV GB/s (% of 8 TB/s) at M=1; prefill GEMM TFLOP/s; MoE layer ms",
        "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": c1["steps"], "warmup": args.warmup,
        "ms_per_step": round(c1["t_step"] * 1e3, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u4xf16->f32", "data": "synthetic",
        "config": {"workload": "C1 int4 prefill GEMM: Llama-3.2-1B layer projections (q|k|v, o, gate|up, down) at "
                               "M=431, fp16 activations, G=32, weights rotating over 16 layers",
                   "tokens": 431, "weights_mb": c1["weights_mb"]},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4), "traffic": load_traffic(),
                     "kernel": dom["kernel"], "flop_per_launch": dom["flop"],
                     "us_per_launch": round(dom["t"] * 1e6, 3)},
        "gemm_c1_per_projection": c1["per_gemm"],
        "gemv_c0": {"gbs_graph_burst": round(gemv, 2), "frac_hbm": round(gemv / HBM_PEAK_GBS, 4),
                    "gbs_single_cold": round(r["bytes"] / r["t_cold"] / 1e9, 2),
                    "us_burst": round(r["t_burst"] * 1e6, 3), "us_single_cold": round(r["t_cold"] * 1e6, 3),
                    "pool_mb": r["pool_mb"], "read_us_graph_burst": c0_read,
                    "frac_of_read": round(c0_read / (r["t_burst"] * 1e6), 3)},
        "ternary_c2": c2,
        "moe_c3": c3,
        "decode_c4": c4,
        "heads": heads,
    }
    if not args.skip_cpu:
        out["cpu_baseline"] = leg("cpu_c1", cpu_baseline_gemm)
        out["gemv_c0"]["cpu_baseline"] = leg("cpu_c0", cpu_baseline_gemv)
        out["decode_c4"]["cpu_baseline"] = leg("cpu_c4", cpu_baseline_decode)
        out["ternary_c2"]["cpu_baseline"] = leg("cpu_c2", cpu_baseline_ternary)
        out["moe_c3"]["cpu_baseline"] = leg("cpu_c3", cpu_baseline_moe)
    out["legs_s"] = legs
    out["wall_s"] = round(time.perf_counter() - T_START, 2)  # the whole run, from the first import
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
