"""Ternary (T2W) GEMV and the X2H producers on the GPU vs the oracle: packed_linear / packed_reduce / pack_half /
rmsnorm_pack / swiglu_pack."""
import numpy as np
import pytest

from _util import rel_inf, to_dev, to_np
from oracle import aq_oracle as orc

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _ops():
    from aq import ops
    return ops


def _kat(rng, n, k):
    """Integer-exact ternary inputs: codes uniform in {0,1,2}, power-of-two scales, small-integer x."""
    codes = rng.integers(0, 3, size=(n, k))
    s = np.exp2(rng.integers(-3, 2, size=(k // 128, n))).astype(np.float16)
    x = rng.integers(-3, 4, size=k).astype(np.float32)
    return codes, s, x


def _exact(codes, s, x):
    n, k = codes.shape
    s8 = (s.astype(np.float64) * 8).astype(np.int64)                 # [K/128, N] integers
    w8 = (codes.astype(np.int64) - 1) * np.repeat(s8.T, 128, axis=1)  # [N, K]
    return (w8 @ x.astype(np.int64)).astype(np.float64) / 8.0


@pytest.mark.parametrize("n,k", [(256, 512), (12288, 4096), (4096, 12288), (300, 1024), (6, 128), (1000, 2176),
                                 (37, 640), (131072, 512), (131076, 384)])
def test_t2_gemv_kat_bit_exact(dev, n, k):
    import torch
    rng = np.random.default_rng(n + k)
    codes, s, x = _kat(rng, n, k)
    y = torch.empty(n, dtype=torch.float32, device=dev)
    _ops().t2_gemv(to_dev(orc.x2h_pack(x), dev), to_dev(orc.t2w_pack(codes), dev), to_dev(s, dev), y)
    np.testing.assert_array_equal(to_np(y), _exact(codes, s, x).astype(np.float32))


@pytest.mark.parametrize("name", ["gate", "down"])
def test_c2_gemv_parity(dev, name):
    """C2: Qwen3-8B gate (12288 x 4096) and down (4096 x 12288), fp16 x."""
    import torch
    from aq import synth
    rng = np.random.default_rng(2)
    n, k = {"gate": (12288, 4096), "down": (4096, 12288)}[name]
    w, s = synth.ternary_matrix(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    xh = orc.x2h_pack(x)
    y = torch.empty(n, dtype=torch.float32, device=dev)
    _ops().t2_gemv(to_dev(xh, dev), to_dev(w, dev), to_dev(s, dev), y)
    assert rel_inf(to_np(y), orc.ternary_gemv(w, s, xh, n, k)) < TOL


def test_t2_gemv_without_workspace(dev):
    import torch
    rng = np.random.default_rng(5)
    n, k = 1024, 4096
    codes, s, x = _kat(rng, n, k)
    y = torch.empty(n, dtype=torch.float32, device=dev)
    torch.ops.aq.t2_gemv(to_dev(orc.x2h_pack(x), dev), to_dev(orc.t2w_pack(codes), dev), to_dev(s, dev), y,
                         torch.empty(8, dtype=torch.uint8, device=dev))
    np.testing.assert_array_equal(to_np(y), _exact(codes, s, x).astype(np.float32))


@pytest.mark.parametrize("n,k", [(640, 4096), (100, 2176)])
def test_packed_linear_and_reduce(dev, n, k):
    """The reference's two-kernel interface: partials [ceil(K/1024), N], then their sum."""
    import torch
    rng = np.random.default_rng(9)
    w, s = __import__("aq").synth.ternary_matrix(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    xh = orc.x2h_pack(x)
    g = (k + 1023) // 1024
    part = torch.empty((g, n), dtype=torch.float32, device=dev)
    _ops().t2_packed_linear(to_dev(xh, dev), to_dev(w, dev), to_dev(s, dev), part)
    ref = orc.ternary_partials(w, s, xh, n, k)
    assert rel_inf(to_np(part), ref) < TOL
    y = torch.empty(n, dtype=torch.float32, device=dev)
    _ops().t2_packed_reduce(part, y)
    np.testing.assert_allclose(to_np(y), to_np(part).astype(np.float64).sum(0), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("count,offset", [(4096, 0), (2006, 0), (2006, 2)])
def test_pack_half_bit_exact(dev, count, offset):
    """16-byte-aligned runs of 8 floats take the vector kernel, the ragged tail (2006 = 8 * 250 + 6) and a
    misaligned x (offset 2 floats) the scalar one; both round to nearest even."""
    import torch
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(count + offset - 2).astype(np.float32),
                        np.array([1 + 2 ** -11, 1 + 3 * 2 ** -11], np.float32)])  # ties to even
    q = torch.empty(count // 2, dtype=torch.int32, device=dev)
    _ops().pack_half(to_dev(x, dev)[offset:], q)
    np.testing.assert_array_equal(to_np(q).view(np.uint32), orc.x2h_pack(x[offset:]))


def test_rmsnorm_and_swiglu_pack(dev):
    import torch
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 4096)).astype(np.float32)
    w = rng.standard_normal(4096).astype(np.float32)
    q = torch.empty((3, 2048), dtype=torch.int32, device=dev)
    _ops().rmsnorm_pack(to_dev(x, dev), to_dev(w, dev), q)
    got = orc.x2h_unpack(to_np(q).view(np.uint32))
    ref = np.stack([orc.x2h_unpack(orc.rmsnorm_pack(x[i], w)) for i in range(3)])
    np.testing.assert_allclose(got, ref, rtol=2 ** -10, atol=1e-6)
    gu = rng.standard_normal((2, 2 * 1024)).astype(np.float32)
    q = torch.empty((2, 512), dtype=torch.int32, device=dev)
    _ops().swiglu_pack(to_dev(gu, dev), q)
    got = orc.x2h_unpack(to_np(q).view(np.uint32))
    ref = np.stack([orc.x2h_unpack(orc.swiglu_pack(gu[i], 1024)) for i in range(2)])
    np.testing.assert_allclose(got, ref, rtol=2 ** -10, atol=1e-6)


def _gemm_t2(x, w, s, dev, add_to=None):
    import torch
    m, n = x.shape[0], w.shape[1]
    y = torch.zeros((m, n), dtype=torch.float32, device=dev) if add_to is None else to_dev(add_to, dev)
    _ops().gemm_t2(to_dev(x, dev), to_dev(w, dev), to_dev(s, dev), y, add=add_to is not None)
    return to_np(y)


@pytest.mark.parametrize("m,n,k,xf32", [(16, 64, 128, False), (412, 256, 1024, False), (100, 300, 256, True),
                                        (412, 12288, 4096, False), (412, 4096, 12288, False), (1, 16, 128, False),
                                        (33, 100, 640, True), (113, 130, 128, False), (150, 200, 384, False),
                                        (412, 1024, 4096, False)])
def test_gemm_t2_kat_bit_exact(dev, m, n, k, xf32):
    """Integer-valued X and power-of-two scales: exact in fp16 MFMA with fp32 accumulation."""
    rng = np.random.default_rng(m + n + k)
    codes = rng.integers(0, 3, size=(n, k))
    s = np.exp2(rng.integers(-3, 2, size=(k // 128, n))).astype(np.float16)
    x = rng.integers(-3, 4, size=(m, k)).astype(np.float32 if xf32 else np.float16)
    got = _gemm_t2(x, orc.t2w_pack(codes), s, dev)
    s8 = (s.astype(np.float64) * 8).astype(np.int64)
    w8 = (codes.astype(np.int64) - 1) * np.repeat(s8.T, 128, axis=1)
    exact = (x.astype(np.int64) @ w8.T).astype(np.float64) / 8.0
    np.testing.assert_array_equal(got, exact.astype(np.float32))


@pytest.mark.parametrize("name", ["gate", "down"])
def test_c2_gemm_parity(dev, name):
    """C2 GEMM at M = 412, fp16 activations."""
    from aq import synth
    rng = np.random.default_rng(22)
    n, k = {"gate": (12288, 4096), "down": (4096, 12288)}[name]
    w, s = synth.ternary_matrix(rng, n, k)
    x = rng.standard_normal((412, k)).astype(np.float16)
    got = _gemm_t2(x, w, s, dev)
    assert rel_inf(got, orc.ternary_gemm(x.astype(np.float32), w, s)) < 1e-2


@pytest.mark.parametrize("m,xf32", [(64, True), (260, False)])
def test_gemm_t2_add(dev, m, xf32):
    rng = np.random.default_rng(23)
    n, k = 512, 1024
    from aq import synth
    w, s = synth.ternary_matrix(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32 if xf32 else np.float16)
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    got = _gemm_t2(x, w, s, dev, add_to=y0)
    assert rel_inf(got, orc.ternary_gemm(x.astype(np.float32), w, s) + y0) < 1e-2


def _head(dev, codes, s, x, hist_len=16, pos0=5):
    import torch
    n, k = codes.shape
    logits = torch.empty(n, dtype=torch.float32, device=dev)
    cand = torch.zeros(_ops().t2_head_candidates(n, k), dtype=torch.int64, device=dev)
    tok = torch.full((1,), -7, dtype=torch.int32, device=dev)
    pos = torch.tensor([pos0], dtype=torch.int32, device=dev)
    hist = torch.full((hist_len,), -9, dtype=torch.int32, device=dev)
    torch.ops.aq.t2_head_argmax(to_dev(orc.x2h_pack(x), dev), to_dev(orc.t2w_pack(codes), dev), to_dev(s, dev),
                                logits, cand, tok, pos, hist, 1)
    return to_np(logits), int(tok.item()), int(pos.item()), to_np(hist)


@pytest.mark.parametrize("n,k", [(151669, 256), (248320, 256), (8000, 1024), (8192, 512), (7, 128)])
def test_t2_head_argmax_kat(dev, n, k):
    """Integer-exact logits, so the token must be the first maximum of the exact products (the reference's greedy()
    over packed_head candidates)."""
    rng = np.random.default_rng(n)
    codes, s, x = _kat(rng, n, k)
    lg, tok, pos, hist = _head(dev, codes, s, x)
    exact = _exact(codes, s, x).astype(np.float32)
    np.testing.assert_array_equal(lg, exact)
    assert tok == orc.argmax_first(exact) and pos == 6
    assert hist[5] == tok and (np.delete(hist, 5) == -9).all()


@pytest.mark.parametrize("n", [248320, 151669])
def test_t2_head_argmax_one_launch_repeats(dev, n):
    """The head ends the greedy step in its own launch (the last workgroup to arrive picks the token): the arrival
    counters are back at zero after every call, so calls in a row, eager and replayed from one graph, each give the
    exact first maximum and advance the position. 248320 columns take 970 workgroups of 256 columns; 151669 take
    4740 of 32 (the last workgroup reads the keys in five passes)."""
    import torch
    ops = _ops()
    rng = np.random.default_rng(n + 2)
    k = 256
    codes, s, x0 = _kat(rng, n, k)
    xs = [x0] + [rng.integers(-3, 4, size=k).astype(np.float32) for _ in range(2)]
    want = [orc.argmax_first(_exact(codes, s, xv).astype(np.float32)) for xv in xs]
    W, S = to_dev(orc.t2w_pack(codes), dev), to_dev(s, dev)
    xh = torch.empty(k // 2, dtype=torch.int32, device=dev)
    logits = torch.empty(n, dtype=torch.float32, device=dev)
    cand = torch.zeros(ops.t2_head_candidates(n, k), dtype=torch.int64, device=dev)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    hist = torch.full((8,), -9, dtype=torch.int32, device=dev)
    run = lambda: torch.ops.aq.t2_head_argmax(xh, W, S, logits, cand, tok, pos, hist, 1)  # noqa
    for i, xv in enumerate(xs):  # eager
        xh.copy_(to_dev(orc.x2h_pack(xv), dev).view(torch.int32))
        run()
        assert int(tok.item()) == want[i] and int(pos.item()) == i + 1
        assert not to_np(cand)[-ops.HEAD_ARRIVAL_SLOTS:].any()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    pos.zero_()
    for i, xv in enumerate(xs):  # replays
        xh.copy_(to_dev(orc.x2h_pack(xv), dev).view(torch.int32))
        g.replay()
        torch.cuda.synchronize()
        assert int(tok.item()) == want[i] and int(pos.item()) == i + 1
        assert not to_np(cand)[-ops.HEAD_ARRIVAL_SLOTS:].any()
    np.testing.assert_array_equal(to_np(hist)[:3], np.array(want, np.int32))


@pytest.mark.parametrize("n", [8000, 248320])
def test_t2_head_argmax_ties_pick_the_first(dev, n):
    """Columns 3, 40, 900 and 7000 (and 140000) are all +1 codes, the largest product: the token is 3, across
    workgroups."""
    rng = np.random.default_rng(3)
    k = 256
    codes = rng.integers(0, 3, size=(n, k))
    codes[[3, 40, 900, 7000] + ([140000] if n > 140000 else [])] = 2
    s = np.ones((k // 128, n), np.float16)
    x = np.ones(k, np.float32)
    lg, tok, pos, _ = _head(dev, codes, s, x)
    np.testing.assert_array_equal(lg, (codes - 1).sum(1).astype(np.float32))
    assert tok == 3 and pos == 6


@pytest.mark.parametrize("bad", ["inf", "nan"])
@pytest.mark.parametrize("n", [8000, 131072])
def test_t2_head_argmax_nonfinite_gives_minus_one(dev, bad, n):
    """A NaN or infinite logit (here from an infinite or NaN scale of column 4321) yields token -1, where the
    reference's greedy() stops with "nonfinite logits"; the position still advances."""
    rng = np.random.default_rng(4)
    k = 256
    codes, s, x = _kat(rng, n, k)
    codes[4321] = 2
    s[:, 4321] = np.float16(bad)
    lg, tok, pos, hist = _head(dev, codes, s, x)
    assert not np.isfinite(lg[4321]) and np.isfinite(np.delete(lg, 4321)).all()
    assert tok == -1 and pos == 6 and hist[5] == -1


@pytest.mark.parametrize("wide", ["cols", "wide"])
def test_t2_head_argmax_float_logits(dev, wide):
    """Random ternary head with fp16 activations: logits vs the oracle, token = first maximum of the GPU logits."""
    import torch
    from aq import synth
    rng = np.random.default_rng(6)
    n, k = (20000, 2048) if wide == "cols" else (131072, 1024)
    w, s = synth.ternary_matrix(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    xh = orc.x2h_pack(x)
    logits = torch.empty(n, dtype=torch.float32, device=dev)
    cand = torch.zeros(_ops().t2_head_candidates(n, k), dtype=torch.int64, device=dev)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    torch.ops.aq.t2_head_argmax(to_dev(xh, dev), to_dev(w, dev), to_dev(s, dev), logits, cand, tok, pos,
                                torch.empty(0, dtype=torch.int32, device=dev), 0)
    lg = to_np(logits)
    assert rel_inf(lg, orc.ternary_gemv(w, s, xh, n, k)) < TOL
    assert int(tok.item()) == orc.argmax_first(lg) and int(pos.item()) == 0


@pytest.mark.parametrize("m,n,k,xf32", [(412, 1024, 4096, False), (412, 256, 12288, False), (100, 300, 1024, True)])
def test_gemm_t2_elementwise_error_bound(dev, m, n, k, xf32):
    """Every output within 1e-3 of its own scale, |y - ref| <= 1e-3 * (|X| . |W|^T) elementwise, against float64: the
    ternary weights times their fp16 scales are exact in fp16, so only fp32 accumulation (and, for fp32 X, its rounding
    to fp16) contribute. X spans four decades."""
    from aq import synth
    rng = np.random.default_rng(m + n + k + (3 if xf32 else 0))
    w, s = synth.ternary_matrix(rng, n, k)
    x = (rng.standard_normal((m, k)) * 10.0 ** rng.uniform(-2, 2, size=(m, k))).astype(
        np.float32 if xf32 else np.float16)
    got = _gemm_t2(x, w, s, dev).astype(np.float64)
    wd = orc.t2w_dequant(w, s).astype(np.float64)
    xd = x.astype(np.float64)
    ref = xd @ wd.T
    scale = np.abs(xd) @ np.abs(wd).T
    worst = float(np.max(np.abs(got - ref) / scale))
    assert worst <= 1e-3, worst
