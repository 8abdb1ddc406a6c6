"""Llama decode step on the GPU vs the CPU oracle: the fused RMSNorm GEMVs, the embedding lookup, RoPE + KV append +
attention, the lm_head with its device argmax, and whole decode steps (eager and graph-replayed).

Bars: rel 1e-3 (inf-norm) for fp32 results; bit-exact for the embedding (fp16 -> fp32), the stored fp16 values, the
argmax index (the first maximum of the logits the GPU produced) and the token / position bookkeeping.
"""
import dataclasses

import numpy as np
import pytest

from _util import rel_inf, to_dev, to_np
from oracle import aq_oracle as orc

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _int4(rng, n, k, group=32):
    from aq import synth
    return synth.int4_matrix(rng, n, k, group)


@pytest.mark.parametrize("n,k,tokens", [(3072, 2048, 1), (2048, 8192, 1), (500, 1024, 3), (8192 + 3, 2048, 1),
                                         (9000, 4096, 1)])
def test_rmsnorm_gemv(dev, n, k, tokens):
    import torch
    rng = np.random.default_rng(n + k + tokens)
    wq, ws = _int4(rng, n, k)
    x = (rng.standard_normal((tokens, k)) * 3).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(k)).astype(np.float16)
    y = torch.empty((tokens, n), dtype=torch.float32, device=dev)
    torch.ops.aq.rmsnorm_gemv_q4(to_dev(wq, dev), to_dev(ws, dev), to_dev(x, dev), to_dev(nw, dev), 1e-5, y, 32)
    ref = np.stack([orc.gemv_q4(wq, ws, orc.rmsnorm(x[t], nw, 1e-5), 32) for t in range(tokens)])
    assert rel_inf(to_np(y), ref) < TOL


@pytest.mark.parametrize("f,k", [(8192, 2048), (4096 + 5, 2048), (5000, 4096), (768, 2048)])
def test_rmsnorm_gate_up(dev, f, k):
    """The decode gate|up with RMSNorm and SwiGLU; 4096 outputs and more take the 16-wave form (16 outputs a
    workgroup: a ragged count, and two chunks a lane at K = 4096), fewer the four-wave form."""
    import torch
    rng = np.random.default_rng(5 + f + k)
    wq, ws = _int4(rng, 2 * f, k)
    x = rng.standard_normal(k).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(k)).astype(np.float16)
    a = torch.empty(f, dtype=torch.float32, device=dev)
    torch.ops.aq.rmsnorm_gate_up_q4(to_dev(wq, dev), to_dev(ws, dev), to_dev(x, dev), to_dev(nw, dev), 1e-5, a, 32)
    ref = orc.gate_up_q4(wq, ws, orc.rmsnorm(x, nw, 1e-5), 32, f)
    assert rel_inf(to_np(a), ref) < TOL


@pytest.mark.parametrize("token", [0, 77, 999, -3, 1000])
def test_embed_exact(dev, token):
    import torch
    rng = np.random.default_rng(9)
    table = rng.standard_normal((1000, 2048)).astype(np.float16)
    x = torch.empty(2048, dtype=torch.float32, device=dev)
    tok = torch.tensor([token], dtype=torch.int32, device=dev)
    torch.ops.aq.embed_f16(to_dev(table, dev), tok, x)
    row = token if 0 <= token < 1000 else 0  # out-of-range tokens read row 0
    np.testing.assert_array_equal(to_np(x), table[row].astype(np.float32))


def _rope_np(max_pos):
    from aq.llama import LlamaConfig, rope_tables
    return rope_tables(dataclasses.replace(LlamaConfig(), max_pos=max_pos))


@pytest.mark.parametrize("heads,kv,max_pos,pos", [
    (32, 8, 512, 0), (32, 8, 512, 1), (32, 8, 512, 300), (32, 8, 512, 511), (4, 2, 64, 63), (8, 8, 128, 70),
    (16, 2, 1024, 777), (8, 1, 96, 50),
])
def test_attn_decode(dev, heads, kv, max_pos, pos):
    import torch
    rng = np.random.default_rng(heads * 7 + kv + pos)
    cos, sin = _rope_np(max_pos)
    qkv = (rng.standard_normal((heads + 2 * kv) * 64) * 2).astype(np.float32)
    kc0 = rng.standard_normal((kv, max_pos, 64)).astype(np.float16)
    vc0 = rng.standard_normal((kv, max_pos, 64)).astype(np.float16)
    kc, vc = to_dev(kc0, dev), to_dev(vc0, dev)
    out = torch.empty(heads * 64, dtype=torch.float32, device=dev)
    torch.ops.aq.attn_decode(to_dev(qkv, dev), to_dev(cos, dev), to_dev(sin, dev), kc, vc,
                             torch.tensor([pos], dtype=torch.int32, device=dev), heads, kv, out)
    kg, vg = to_np(kc).view(np.float16), to_np(vc).view(np.float16)
    # the cache: row pos is the rotated key and the value, as fp16; every other row is untouched
    k_rot = orc.rope(qkv[heads * 64:(heads + kv) * 64].reshape(kv, 64), cos[pos], sin[pos])
    v_new = qkv[(heads + kv) * 64:].reshape(kv, 64)
    np.testing.assert_array_equal(vg[:, pos], v_new.astype(np.float16))
    np.testing.assert_allclose(kg[:, pos].astype(np.float64), k_rot, rtol=1e-3, atol=1e-3)
    keep = np.ones(max_pos, bool)
    keep[pos] = False
    np.testing.assert_array_equal(kg[:, keep], kc0[:, keep])
    np.testing.assert_array_equal(vg[:, keep], vc0[:, keep])
    q = orc.rope(qkv[:heads * 64].reshape(heads, 64), cos[pos], sin[pos])
    ref = orc.attention_decode(q, kg.astype(np.float64), vg.astype(np.float64), pos + 1)
    assert rel_inf(to_np(out), ref.reshape(-1)) < TOL


@pytest.mark.parametrize("pos", [-1, 64])
def test_attn_decode_position_outside_cache(dev, pos):
    import torch
    cos, sin = _rope_np(64)
    kc = torch.ones((2, 64, 64), dtype=torch.float16, device=dev)
    vc = torch.ones((2, 64, 64), dtype=torch.float16, device=dev)
    out = torch.full((4 * 64,), 7.0, dtype=torch.float32, device=dev)
    qkv = torch.ones(8 * 64, dtype=torch.float32, device=dev)
    torch.ops.aq.attn_decode(qkv, to_dev(cos, dev), to_dev(sin, dev), kc, vc,
                             torch.tensor([pos], dtype=torch.int32, device=dev), 4, 2, out)
    assert float(out.abs().max()) == 0.0
    assert bool((kc == 1).all()) and bool((vc == 1).all())


@pytest.mark.parametrize("vocab", [128256, 1000, 7])
def test_head_argmax(dev, vocab):
    import torch
    rng = np.random.default_rng(vocab)
    k = 2048
    wq, ws = _int4(rng, vocab, k)
    x = rng.standard_normal(k).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(k)).astype(np.float16)
    logits = torch.empty(vocab, dtype=torch.float32, device=dev)
    cand = torch.zeros(4096, dtype=torch.int64, device=dev)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    pos = torch.tensor([5], dtype=torch.int32, device=dev)
    hist = torch.full((16,), -1, dtype=torch.int32, device=dev)
    torch.ops.aq.head_argmax_q4(to_dev(wq, dev), to_dev(ws, dev), to_dev(x, dev), to_dev(nw, dev), 1e-5, logits, 32,
                                cand, tok, pos, hist, 1)
    lg = to_np(logits)
    assert rel_inf(lg, orc.gemv_q4(wq, ws, orc.rmsnorm(x, nw, 1e-5), 32)) < TOL
    best = orc.argmax_first(lg)
    assert int(tok.item()) == best
    assert int(pos.item()) == 6
    h = to_np(hist)
    assert h[5] == best and (np.delete(h, 5) == -1).all()


@pytest.mark.parametrize("vocab", [37, 1000, 50000])
def test_head_argmax_one_launch_repeats(dev, vocab):
    """The head ends the greedy step in its own launch (the last workgroup to arrive picks the token, counted on a
    two-level set of arrival counters): the counters in cand's last HEAD_ARRIVAL_SLOTS slots are back at zero after
    every call, so calls in a row, eager and replayed from one graph, each give the oracle's token and advance the
    position. 37, 1000 and 50000 rows take 5 workgroups (one per counter group), 63 (groups of 3 and 4) and 1024."""
    import torch
    from aq import ops
    rng = np.random.default_rng(77)
    k = 2048
    wq, ws = _int4(rng, vocab, k)
    xs = [rng.standard_normal(k).astype(np.float32) for _ in range(3)]
    logits = torch.empty(vocab, dtype=torch.float32, device=dev)
    cand = torch.zeros(4096, dtype=torch.int64, device=dev)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    hist = torch.full((8,), -1, dtype=torch.int32, device=dev)
    nonorm = torch.empty(0, dtype=torch.float16, device=dev)
    W, S = to_dev(wq, dev), to_dev(ws, dev)
    x = torch.empty(k, dtype=torch.float32, device=dev)
    want = [orc.argmax_first(orc.gemv_q4(wq, ws, xv, 32)) for xv in xs]
    run = lambda: torch.ops.aq.head_argmax_q4(W, S, x, nonorm, 1e-5, logits, 32, cand, tok, pos, hist, 1)  # noqa
    for i, xv in enumerate(xs):  # eager
        x.copy_(to_dev(xv, dev))
        run()
        assert int(tok.item()) == want[i] and int(pos.item()) == i + 1
        assert not to_np(cand)[-ops.HEAD_ARRIVAL_SLOTS:].any()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    pos.zero_()
    for i, xv in enumerate(xs):  # replays
        x.copy_(to_dev(xv, dev))
        g.replay()
        torch.cuda.synchronize()
        assert int(tok.item()) == want[i] and int(pos.item()) == i + 1
        assert not to_np(cand)[-ops.HEAD_ARRIVAL_SLOTS:].any()
    np.testing.assert_array_equal(to_np(hist)[:3], np.array(want, np.int32))


def test_head_argmax_ties_pick_the_first(dev):
    """Rows 3, 40 and 900 are identical and give the largest logit: the token is 3 (integer-exact inputs, no norm)."""
    import torch
    vocab, k = 1000, 256
    vals = np.zeros((vocab, k), np.int64)
    rng = np.random.default_rng(1)
    vals[:] = rng.integers(-2, 3, size=(vocab, k))
    vals[[3, 40, 900]] = 7
    wq = orc.q4w_pack(vals)
    ws = np.ones((vocab, k // 32), np.float16)
    x = np.ones(k, np.float32)
    logits = torch.empty(vocab, dtype=torch.float32, device=dev)
    cand = torch.zeros(4096, dtype=torch.int64, device=dev)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    pos = torch.tensor([0], dtype=torch.int32, device=dev)
    empty = torch.empty(0, dtype=torch.int32, device=dev)
    torch.ops.aq.head_argmax_q4(to_dev(wq, dev), to_dev(ws, dev), to_dev(x, dev),
                                torch.empty(0, dtype=torch.float16, device=dev), 1e-5, logits, 32, cand, tok, pos,
                                empty, 0)
    np.testing.assert_array_equal(to_np(logits), (vals @ np.ones(k)).astype(np.float32))
    assert int(tok.item()) == 3 and int(pos.item()) == 0


def test_head_argmax_skips_nan_rows(dev):
    """A NaN logit (row 777's scales are NaN) never wins, as in the reference's `logits[i] > logits[best]` scan; an
    infinite one (row 50) does."""
    import torch
    rng = np.random.default_rng(2)
    vocab, k = 5000, 256
    wq, ws = _int4(rng, vocab, k)
    ws[777] = np.float16("nan")
    x = rng.standard_normal(k).astype(np.float32)
    logits = torch.empty(vocab, dtype=torch.float32, device=dev)
    cand = torch.zeros(4096, dtype=torch.int64, device=dev)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    empty = torch.empty(0, dtype=torch.int32, device=dev)
    nonorm = torch.empty(0, dtype=torch.float16, device=dev)
    args = (to_dev(x, dev), nonorm, 1e-5, logits, 32, cand, tok, pos, empty, 0)
    torch.ops.aq.head_argmax_q4(to_dev(wq, dev), to_dev(ws, dev), *args)
    lg = to_np(logits)
    assert np.isnan(lg[777]) and np.isfinite(np.delete(lg, 777)).all()
    assert int(tok.item()) == orc.argmax_first(np.where(np.isnan(lg), -np.inf, lg))
    ws[50] = np.float16("inf")
    wq[50] = 0xFFFFFFFF  # every value -1 * inf * x: +-inf, NaN only where x is 0
    x = np.abs(x) + 0.5
    x *= -1  # (-1) * inf * (-x) = +inf for every k
    torch.ops.aq.head_argmax_q4(to_dev(wq, dev), to_dev(ws, dev), to_dev(x, dev), *args[1:])
    lg = to_np(logits)
    assert lg[50] == np.inf and int(tok.item()) == 50


def _small_cfg(**kw):
    from aq.llama import LlamaConfig
    base = dict(dim=512, layers=2, heads=8, kv_heads=2, head_dim=64, ffn=1024, vocab=1000, max_pos=64)
    base.update(kw)
    return LlamaConfig(**base)


def _decoder(cfg, seed, dev):
    from aq import synth
    from aq.llama import LlamaDecoder, LlamaWeights, rope_tables
    arrays = synth.llama_arrays(cfg, seed)
    arrays["embed"] = (arrays["embed"].astype(np.float32) * 0.1).astype(np.float16)
    cos, sin = rope_tables(cfg)
    return LlamaDecoder(LlamaWeights.from_numpy(cfg, arrays, dev)), orc.LlamaDecodeOracle(arrays, cfg, cos, sin)


@pytest.mark.parametrize("cfg_kw", [{}, dict(dim=2048, heads=32, kv_heads=8, ffn=8192, vocab=32000, max_pos=512),
                                    dict(dim=2048, heads=32, kv_heads=8, ffn=8192, vocab=32000, max_pos=512, group=64)],
                         ids=["small", "llama1b-width-2-layers", "llama1b-width-2-layers-g64"])
def test_decode_steps_vs_oracle(dev, cfg_kw):
    """Token-by-token forward steps: logits within rel 1e-3 of the float64 oracle (same fp16 cache rounding) at every
    step, and the device argmax is the first maximum of those logits.

    A cached value that sits on an fp16 rounding boundary can round either way between the GPU's fp32 and the
    oracle's float64 arithmetic, and a small random model can amplify that: the bar is widened by twice the model's
    own sensitivity to its cache's rounding (the oracle with an fp16 cache against the oracle with a float64 one),
    which is ~1e-5 at Llama-1B width and up to a few 1e-3 for the 512-wide model."""
    cfg = _small_cfg(**cfg_kw)
    dec, oracle = _decoder(cfg, 21, dev)
    from aq import synth
    from aq.llama import rope_tables
    arrays = synth.llama_arrays(cfg, 21)
    arrays["embed"] = (arrays["embed"].astype(np.float32) * 0.1).astype(np.float16)
    exact = orc.LlamaDecodeOracle(arrays, cfg, *rope_tables(cfg), kv_dtype=None)
    tokens = [1, 500, 999, 2, 2, 300, 17, 64, 0, 777][:10]
    for pos, t in enumerate(tokens):
        lg = to_np(dec.forward(t, pos))
        ref = oracle.step(t, pos)
        sensitivity = rel_inf(ref, exact.step(t, pos))
        assert rel_inf(lg, ref) < TOL + 2 * sensitivity, (pos, sensitivity)
        if cfg.dim == 2048:
            assert rel_inf(lg, ref) < TOL, pos
        assert int(dec.token.item()) == orc.argmax_first(lg)
        assert int(dec.pos.item()) == pos + 1


def test_decode_whole_depth_end_of_context(dev):
    """All 16 layers at Llama-3.2-1B width (vocabulary cut to 32000) at the end of a 512-position context: both caches
    hold the same fp16 rows 0..506, then positions 507..511 are decoded; the logits stay within rel 1e-3 of the
    float64 oracle at every step, as the reference checks its whole-model logits (llama/run.py:186-198,295-306)."""
    from aq import synth
    from aq.llama import LlamaConfig, LlamaDecoder, LlamaWeights, rope_tables
    cfg = LlamaConfig(vocab=32000)
    assert cfg.layers == 16 and cfg.max_pos == 512
    arrays = synth.llama_arrays(cfg, 23)
    arrays["embed"] = (arrays["embed"].astype(np.float32) * 0.1).astype(np.float16)
    dec = LlamaDecoder(LlamaWeights.from_numpy(cfg, arrays, dev))
    oracle = orc.LlamaDecodeOracle(arrays, cfg, *rope_tables(cfg), weights_dtype=np.float32)
    del arrays
    rng = np.random.default_rng(5)
    p0 = 507
    for i in range(cfg.layers):
        kc = (rng.standard_normal((cfg.kv_heads, p0, cfg.head_dim)) * 3).astype(np.float16)
        vc = rng.standard_normal((cfg.kv_heads, p0, cfg.head_dim)).astype(np.float16)
        dec.kc[i][:, :p0] = to_dev(kc, dev)
        dec.vc[i][:, :p0] = to_dev(vc, dev)
        oracle.kc[i][:, :p0] = kc.astype(np.float64)
        oracle.vc[i][:, :p0] = vc.astype(np.float64)
    for pos, t in zip(range(p0, 512), [1, 500, 31999, 7, 123]):
        lg = to_np(dec.forward(t, pos))
        ref = oracle.step(t, pos)
        assert rel_inf(lg, ref) < TOL, pos
        assert int(dec.token.item()) == orc.argmax_first(lg)


def test_generate_graph_vs_oracle_greedy(dev):
    """Greedy generation by graph replay equals the oracle's greedy tokens up to the first step whose top-2 logit gap is
    within the tolerance (where either choice is correct)."""
    cfg = _small_cfg()
    dec, oracle = _decoder(cfg, 22, dev)
    prompt, max_new = [3, 14, 15, 92], 20
    got = dec.generate(prompt, max_new)
    assert len(got) == max_new
    want = []
    for pos, t in enumerate(prompt):
        lg = oracle.step(t, pos)
    for i in range(max_new):
        srt = np.sort(lg)
        if srt[-1] - srt[-2] <= 2 * TOL * np.abs(lg).max():
            break
        want.append(orc.argmax_first(lg))
        if i + 1 < max_new:
            lg = oracle.step(want[-1], len(prompt) + i)
    assert len(want) >= 5
    assert got[:len(want)] == want


def test_graph_replay_is_bitwise_eager(dev):
    """At the Llama-3.2-1B shape (random weights drawn on the device): replaying the captured step gives the same
    tokens and bit-identical logits as eager steps (every kernel is deterministic)."""
    import torch
    from aq.llama import LlamaConfig, LlamaDecoder, LlamaWeights
    cfg = LlamaConfig()
    w = LlamaWeights.random(cfg, 4, dev)
    a = LlamaDecoder(w)
    toks_a, logits_a = [], []
    a.token.fill_(128000)
    a.pos.fill_(0)
    for _ in range(6):
        a.step(advance=1)
        toks_a.append(int(a.token.item()))
        logits_a.append(a.logits.clone())
    b = LlamaDecoder(w)
    b.capture()
    b.token.fill_(128000)
    b.pos.fill_(0)
    for i in range(6):
        b.graph.replay()
        assert int(b.token.item()) == toks_a[i]
        assert torch.equal(b.logits, logits_a[i])
    assert int(b.pos.item()) == 6
    np.testing.assert_array_equal(to_np(b.hist[:6]), np.array(toks_a, np.int32))


@pytest.mark.parametrize("heads,kv,max_pos,pos,splits", [
    (32, 8, 512, 511, 8), (32, 8, 512, 0, 8), (32, 8, 512, 63, 8), (32, 8, 512, 64, 8), (32, 8, 512, 300, 3),
    (4, 2, 64, 63, 1), (16, 2, 1024, 777, 8), (8, 1, 200, 150, 7), (8, 8, 4096, 4000, 8),
])
def test_split_attention_and_combined_output_projection(dev, heads, kv, max_pos, pos, splits):
    """aq_attn_decode_split writes the cache row as aq_attn_decode does, and aq_attn_out_q4 (the spans combined while
    staging x) equals y + Wo . attention(q, cache) of the oracle."""
    import torch
    from aq import ops
    rng = np.random.default_rng(heads + kv + max_pos + pos + splits)
    cos, sin = _rope_np(max_pos)
    qkv = (rng.standard_normal((heads + 2 * kv) * 64) * 2).astype(np.float32)
    kc0 = rng.standard_normal((kv, max_pos, 64)).astype(np.float16)
    vc0 = rng.standard_normal((kv, max_pos, 64)).astype(np.float16)
    kc, vc = to_dev(kc0, dev), to_dev(vc0, dev)
    parts = torch.full((ops.attn_parts_numel(heads, splits),), float("nan"), dtype=torch.float32, device=dev)
    torch.ops.aq.attn_decode_split(to_dev(qkv, dev), to_dev(cos, dev), to_dev(sin, dev), kc, vc,
                                   torch.tensor([pos], dtype=torch.int32, device=dev), heads, kv, splits, parts)
    kg, vg = to_np(kc).view(np.float16), to_np(vc).view(np.float16)
    np.testing.assert_array_equal(vg[:, pos], qkv[(heads + kv) * 64:].reshape(kv, 64).astype(np.float16))
    keep = np.ones(max_pos, bool)
    keep[pos] = False
    np.testing.assert_array_equal(kg[:, keep], kc0[:, keep])
    q = orc.rope(qkv[:heads * 64].reshape(heads, 64), cos[pos], sin[pos])
    att = orc.attention_decode(q, kg.astype(np.float64), vg.astype(np.float64), pos + 1).reshape(-1)
    n = 700
    wq, ws = _int4(rng, n, heads * 64)
    y0 = rng.standard_normal(n).astype(np.float32)
    y = to_dev(y0, dev)
    torch.ops.aq.attn_out_q4(to_dev(wq, dev), to_dev(ws, dev), parts, splits, y, 32)
    assert rel_inf(to_np(y), orc.gemv_q4(wq, ws, att, 32, y0=y0)) < TOL
