"""The Q6_K tied head (GEMV, GEMV + device argmax) and embedding on the GPU vs the oracle.

Integer-exact inputs (power-of-two d, small scales, small-integer x) make the head's products exact in fp32, so the
GPU logits must equal the integer matmul bit for bit; the embedding rows must equal the oracle's (d * sc) * (q - 32)
bit for bit, the arithmetic the reference's converter ("h6", compiled from lfm2/convert.c) is pinned to."""
import numpy as np
import pytest

from _util import rel_inf, to_dev, to_np
from oracle import aq_oracle as orc

pytestmark = pytest.mark.gpu

TOL = 1e-5  # fp32 arithmetic throughout: normwise relative error against float64


def _kat(rng, rows, cols):
    """Q6W with d = 2^-e, scales in [-8, 7] and x in [-3, 3] integers: every partial sum is an exact fp32 integer
    multiple of d."""
    q = rng.integers(0, 256, size=(rows, cols // 256, 208), dtype=np.uint8)
    q[:, :, 192:] = rng.integers(-8, 8, size=(rows, cols // 256, 16), dtype=np.int8).view(np.uint8)
    d = np.exp2(-rng.integers(0, 6, size=(rows, cols // 256))).astype(np.float16)
    x = rng.integers(-3, 4, size=cols).astype(np.float32)
    return q, d, x


def _exact(q, d, x):
    vals, ds = orc.q6w_values(q, d)
    return (vals * np.repeat(ds, 16, axis=1).astype(np.float64)) @ x.astype(np.float64)


# cols 256 .. 4096: 4 .. 64 lanes a row (3072: 48 units in 64 lanes); 5120, 8192: the LDS path. Rows not a multiple of
# the rows per wave step, and more rows than one pass of the waves.
@pytest.mark.parametrize("rows,cols", [(1001, 256), (77, 512), (3000, 1024), (5003, 2048), (4100, 4096),
                                       (999, 3072), (1500, 5120), (300, 8192), (7, 2048)])
def test_gemv_q6_kat_bit_exact(dev, rows, cols):
    import torch
    rng = np.random.default_rng(rows + cols)
    q, d, x = _kat(rng, rows, cols)
    y = torch.empty(rows, dtype=torch.float32, device=dev)
    torch.ops.aq.gemv_q6(to_dev(q, dev), to_dev(d, dev), to_dev(x, dev), y)
    np.testing.assert_array_equal(to_np(y), _exact(q, d, x).astype(np.float32))


@pytest.mark.parametrize("rows,cols", [(16384, 2048), (2000, 3072), (1000, 5120)])
def test_gemv_q6_vs_oracle(dev, rows, cols):
    import torch
    from aq import synth
    rng = np.random.default_rng(cols)
    q, d = synth.q6_matrix(rng, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    y = torch.empty(rows, dtype=torch.float32, device=dev)
    torch.ops.aq.gemv_q6(to_dev(q, dev), to_dev(d, dev), to_dev(x, dev), y)
    assert rel_inf(to_np(y), orc.gemv_q6(q, d, x)) < TOL


def _head(dev, q, d, x, nw=None, eps=1e-5, pos0=3):
    import torch
    from aq import ops
    rows, cols = q.shape[0], q.shape[1] * 256
    logits = torch.empty(rows, dtype=torch.float32, device=dev)
    cand = torch.zeros(ops.HEAD_CANDIDATES, dtype=torch.int64, device=dev)
    tok = torch.full((1,), -7, dtype=torch.int32, device=dev)
    pos = torch.tensor([pos0], dtype=torch.int32, device=dev)
    hist = torch.full((8,), -9, dtype=torch.int32, device=dev)
    norm = to_dev(nw, dev) if nw is not None else torch.empty(0, dtype=torch.float16, device=dev)
    torch.ops.aq.head_argmax_q6(to_dev(q, dev), to_dev(d, dev), to_dev(x, dev), norm, eps, logits, cand, tok, pos,
                                hist, 1)
    return to_np(logits), int(tok.item()), int(pos.item()), to_np(hist)


@pytest.mark.parametrize("rows,cols", [(65536, 2048), (3000, 5120)])
def test_head_argmax_q6_kat(dev, rows, cols):
    """LFM2's head shape (65536 x 2048) and the LDS path: exact logits, token = their first maximum."""
    rng = np.random.default_rng(rows)
    q, d, x = _kat(rng, rows, cols)
    lg, tok, pos, hist = _head(dev, q, d, x)
    exact = _exact(q, d, x).astype(np.float32)
    np.testing.assert_array_equal(lg, exact)
    assert tok == orc.argmax_first(exact) and pos == 4
    assert hist[3] == tok and (np.delete(hist, 3) == -9).all()


@pytest.mark.parametrize("rows,cols", [(65536, 2048), (3000, 5120)])
def test_head_argmax_q6_one_launch_repeats(dev, rows, cols):
    """The head ends the greedy step in its own launch (the last workgroup to arrive picks the token): the arrival
    counters in cand's last HEAD_ARRIVAL_SLOTS slots are back at zero after every call, so calls in a row, eager and
    replayed from one graph, each give the exact first maximum and advance the position (768 and 750 workgroups)."""
    import torch
    from aq import ops
    rng = np.random.default_rng(rows + 1)
    q, d, x0 = _kat(rng, rows, cols)
    xs = [x0] + [rng.integers(-3, 4, size=cols).astype(np.float32) for _ in range(2)]
    want = [orc.argmax_first(_exact(q, d, xv).astype(np.float32)) for xv in xs]
    Q, D = to_dev(q, dev), to_dev(d, dev)
    x = torch.empty(cols, dtype=torch.float32, device=dev)
    logits = torch.empty(rows, dtype=torch.float32, device=dev)
    cand = torch.zeros(ops.head_q6_candidates(rows, cols), dtype=torch.int64, device=dev)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    hist = torch.full((8,), -1, dtype=torch.int32, device=dev)
    nonorm = torch.empty(0, dtype=torch.float16, device=dev)
    run = lambda: torch.ops.aq.head_argmax_q6(Q, D, x, nonorm, 1e-5, logits, cand, tok, pos, hist, 1)  # noqa
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


def test_head_argmax_q6_ties_pick_the_first(dev):
    """Rows 5, 2000 and 40000 are copies of the largest row: the token is 5 (the rows sit in different waves)."""
    rng = np.random.default_rng(8)
    rows, cols = 65536, 2048
    q, d, x = _kat(rng, rows, cols)
    exact = _exact(q, d, x)
    top = int(np.argmax(exact))
    for r in (5, 2000, 40000):
        q[r], d[r] = q[top], d[top]
    lg, tok, _, _ = _head(dev, q, d, x)
    assert lg[5] == lg[2000] == lg[40000] == lg.max()
    assert tok == orc.argmax_first(lg) and tok <= 5  # 5 unless an earlier row ties exactly


def test_head_argmax_q6_fused_norm(dev):
    """Final RMSNorm fused into the head, against rmsnorm then the dequantized matrix in float64."""
    from aq import synth
    rng = np.random.default_rng(9)
    rows, cols = 65536, 2048
    q, d = synth.q6_matrix(rng, rows, cols)
    x = (3 * rng.standard_normal(cols)).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float16)
    lg, tok, _, _ = _head(dev, q, d, x, nw=nw, eps=1e-5)
    assert rel_inf(lg, orc.gemv_q6(q, d, orc.rmsnorm(x, nw, 1e-5))) < TOL
    assert tok == orc.argmax_first(lg)


@pytest.mark.parametrize("cols", [2048, 5120])
def test_embed_q6_bit_exact(dev, cols):
    """Rows of several tokens, one out of range (reads row 0), equal to the oracle's dequantisation bit for bit."""
    import torch
    from aq import synth
    rng = np.random.default_rng(cols)
    rows = 3000
    q, d = synth.q6_matrix(rng, rows, cols)
    d[17, 0] = np.float16(3e-7)  # an fp16-subnormal d
    ids = np.array([17, 0, 2999, -5, 3000, 1234], np.int32)
    x = torch.empty((len(ids), cols), dtype=torch.float32, device=dev)
    torch.ops.aq.embed_q6(to_dev(q, dev), to_dev(d, dev), to_dev(ids, dev), x)
    deq = orc.q6w_dequant(q, d)
    want = deq[np.where((ids >= 0) & (ids < rows), ids, 0)]
    np.testing.assert_array_equal(to_np(x), want)
