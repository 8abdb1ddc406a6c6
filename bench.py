"""Benchmark of the weight-quantized matmul path on one MI355X; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-cpu]

Workload (BASELINE.json metric "int4 GEMV GB/s (% of 8 TB/s) at M=1; prefill GEMM TFLOP/s; MoE layer ms"):
  value   C0 int4 decode GEMV (Llama-3.2-1B FFN up, 8192 x 2048, G = 32, fp32 x/y), GB/s of algorithmic bytes.
          One step = one GEMV launch. The weights rotate over a pool of distinct copies (>= 512 MB, twice the
          256 MB Infinity Cache), so every launch streams from HBM; the K timed steps are replayed from a hipGraph.
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
    return dict(bytes=per, flop=2 * n * k, t_step=t_step, t_burst=t_burst, t_cold=t_cold, pool_copies=copies,
                pool_mb=round(copies * per / 1e6, 1), steps=len(seq))


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--skip-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (see DESIGN.md, sharding)",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    r = bench_gemv_c0(dev, args.steps, args.warmup)
    wall = time.perf_counter() - t0
    value = r["bytes"] / r["t_step"] / 1e9
    out = {
        "metric": "int4 GEMV GB/s (% of 8 TB/s) at M=1; prefill GEMM TFLOP/s; MoE layer ms",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": r["steps"], "warmup": args.warmup,
        "ms_per_step": round(r["t_step"] * 1e3, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u4xf32", "data": "synthetic",
        "config": {"workload": "C0 int4 decode GEMV, Llama-3.2-1B FFN up 8192x2048, G=32, fp32 x/y",
                   "pool_mb": r["pool_mb"], "rotating_copies": r["pool_copies"]},
        "roofline": {"bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": None},
        "gemv_c0": {"gbs_graph_burst": round(r["bytes"] / r["t_burst"] / 1e9, 2),
                    "gbs_single_cold": round(r["bytes"] / r["t_cold"] / 1e9, 2),
                    "us_burst": round(r["t_burst"] * 1e6, 3), "us_single_cold": round(r["t_cold"] * 1e6, 3)},
        "wall_s": round(wall, 2),
    }
    if not args.skip_cpu:
        out["cpu_baseline"] = cpu_baseline_gemv()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
