"""int4 (Q4W) GEMV on the GPU vs the CPU oracle: gemv_q4 / gemv_add_q4 / lk.gemv_q4 / t_gemv_q4 / gate_up_q4."""
import numpy as np
import pytest

from _util import exact_int4_product, kat_int4, rel_inf, to_dev, to_np
from oracle import aq_oracle as orc

pytestmark = pytest.mark.gpu

TOL_FP32 = 1e-3  # rel (inf-norm) bar for fp32 activations


def _ops():
    from aq import ops
    return ops


def test_c0_shape_parity(dev):
    """C0: Llama-3.2-1B FFN-up 8192 x 2048, G = 32, fp32 x/y."""
    import torch
    from aq import synth
    d = synth.c0()
    y = torch.empty(d["n"], dtype=torch.float32, device=dev)
    _ops().gemv_q4(to_dev(d["wq"], dev), to_dev(d["ws"], dev), to_dev(d["x"], dev), y, d["group"])
    ref = orc.gemv_q4(d["wq"], d["ws"], d["x"], d["group"])
    assert rel_inf(to_np(y), ref) < TOL_FP32


@pytest.mark.parametrize("n,k,group,tokens", [
    (64, 2048, 32, 1), (300, 2048, 64, 1), (129, 768, 128, 1), (77, 8192, 32, 1), (5, 32, 32, 1),
    (33, 4096 + 32, 32, 1), (40, 256, 256, 1), (17, 512, 16, 1), (19, 1024, 8, 1), (23, 96, 24, 1),
    (70, 2048, 32, 2), (70, 2048, 64, 3), (65, 1024, 32, 5), (31, 2048, 128, 8), (9, 4096, 32, 8),
    (40, 2048, 32, 9), (33, 1024, 64, 12), (17, 2048, 32, 16), (21, 512, 16, 13),
    # the long-K form (K split over the waves of a workgroup): 2 or 4 slices, one or two chunks a lane
    (2048, 8192, 32, 1), (100, 8192, 64, 1), (4096, 4096, 128, 1), (7, 16384, 32, 1), (9, 12288 + 32, 32, 1),
    # the 16-wave form without a K split (32 outputs a workgroup): C0's shape, a ragged row count, two chunks a lane
    (8192, 2048, 32, 1), (12000 + 3, 4096, 64, 1), (32768, 1024, 32, 1),
])
def test_kat_bit_exact(dev, n, k, group, tokens):
    """Integer-exact inputs: the GPU result must equal the exact product bit for bit, whatever the sum order."""
    import torch
    rng = np.random.default_rng(n * 1000 + k + group + tokens)
    vals, ws, x = kat_int4(rng, n, k, group, tokens)
    wq = orc.q4w_pack(vals)
    y = torch.empty((tokens, n), dtype=torch.float32, device=dev)
    _ops().gemv_q4(to_dev(wq, dev), to_dev(ws, dev), to_dev(x, dev), y, group)
    np.testing.assert_array_equal(to_np(y), exact_int4_product(vals, ws, x, group).astype(np.float32))


@pytest.mark.parametrize("n,k,group,tokens", [(8192, 2048, 32, 1), (4096, 2048, 64, 1), (2048, 8192, 32, 1),
                                                (3000, 2048, 128, 1), (1000, 2048, 32, 4), (700, 1024, 32, 13)])
def test_elementwise_error_bound(dev, n, k, group, tokens):
    """Every output, not only the largest, within 1e-3 of its own scale: |y - ref| <= 1e-3 * (|W| . |x|) elementwise.
    The power-of-two-group path rounds each 32-wide chunk of x to 22-bit fixed point against the chunk's largest
    value, so x spans seven decades within and across chunks (a small x beside a large one keeps only the bits above
    2^-22 of the chunk's maximum). The bound is relative to |W| . |x|, not to |y|, so it also holds the rows whose sums
    nearly cancel."""
    import torch
    from aq import synth
    rng = np.random.default_rng(n + k + group + tokens)
    wq, ws = synth.int4_matrix(rng, n, k, group)
    x = (rng.standard_normal((tokens, k)) * 10.0 ** rng.uniform(-4, 3, size=(tokens, k))).astype(np.float32)
    y = torch.empty((tokens, n), dtype=torch.float32, device=dev)
    _ops().gemv_q4(to_dev(wq, dev), to_dev(ws, dev), to_dev(x, dev), y, group)
    w = orc.q4w_dequant(wq, ws, group).astype(np.float64)
    ref = x.astype(np.float64) @ w.T
    scale = np.abs(x.astype(np.float64)) @ np.abs(w).T
    err = np.abs(to_np(y).astype(np.float64) - ref)
    worst = float(np.max(err / scale))
    assert worst <= 1e-3, worst


@pytest.mark.parametrize("tokens,k", [(1, 2048), (4, 2048), (1, 8192)])
def test_add_residual(dev, tokens, k):
    """gemv_add_q4: y += W x (llama/kernels/gemv_add_q4.mojo:30); K = 8192 is the decode down projection's form."""
    import torch
    rng = np.random.default_rng(7 + k)
    n, g = 1000, 64
    wq, ws = rng.integers(0, 2 ** 32, (n, k // 8), dtype=np.uint32), \
        (np.abs(rng.standard_normal((n, k // g))) * 0.02 + 1e-3).astype(np.float16)
    x = rng.standard_normal((tokens, k)).astype(np.float32)
    y0 = rng.standard_normal((tokens, n)).astype(np.float32)
    y = to_dev(y0, dev)
    _ops().gemv_q4(to_dev(wq, dev), to_dev(ws, dev), to_dev(x, dev), y, g, add=True)
    ref = orc.gemm_q4(wq, ws, x, g, y0=y0)
    assert rel_inf(to_np(y), ref) < TOL_FP32


@pytest.mark.parametrize("tokens,f", [(1, 768), (3, 768), (1, 8192), (1, 4096 + 16 + 7)])
def test_gate_up(dev, tokens, f):
    import torch
    rng = np.random.default_rng(11 + f)
    k, g = 2048, 32
    wq = rng.integers(0, 2 ** 32, (2 * f, k // 8), dtype=np.uint32)
    ws = (np.abs(rng.standard_normal((2 * f, k // g))) * 0.02 + 1e-3).astype(np.float16)
    x = rng.standard_normal((tokens, k)).astype(np.float32)
    a = torch.empty((tokens, f), dtype=torch.float32, device=dev)
    _ops().gate_up_q4(to_dev(wq, dev), to_dev(ws, dev), to_dev(x, dev), a, g)
    ref = np.stack([orc.gate_up_q4(wq, ws, x[t], g, f) for t in range(tokens)])
    assert rel_inf(to_np(a), ref) < TOL_FP32


def test_llama_lm_head_shape(dev):
    """The largest decode GEMV of C4: lm_head 128256 x 2048 (exercises the persistent row loop)."""
    import torch
    from aq import synth
    rng = np.random.default_rng(4)
    wq, ws = synth.int4_matrix(rng, 128256, 2048, 32)
    x = rng.standard_normal(2048).astype(np.float32)
    y = torch.empty(128256, dtype=torch.float32, device=dev)
    _ops().gemv_q4(to_dev(wq, dev), to_dev(ws, dev), to_dev(x, dev), y, 32)
    assert rel_inf(to_np(y), orc.gemv_q4(wq, ws, x, 32)) < TOL_FP32


def test_error_paths(dev):
    import torch
    from aq import AqError
    wq = torch.zeros((8, 64), dtype=torch.int32, device=dev)  # K = 512
    ws = torch.zeros((8, 16), dtype=torch.float16, device=dev)
    x = torch.zeros(513, dtype=torch.float32, device=dev)
    y = torch.zeros(8, dtype=torch.float32, device=dev)
    with pytest.raises(AqError, match="misaligned"):
        _ops().gemv_q4(wq, ws, x[1:], y, 32)
    with pytest.raises(ValueError):
        _ops().gemv_q4(wq, ws, x[:512], y, 48)  # 512 % 48 != 0


@pytest.mark.parametrize("tokens,k", [(10, 2048), (12, 2048), (16, 1024)])
def test_few_rows_vs_oracle(dev, tokens, k):
    """Few-row products (rows_q4, lfm2/kernels/dsk.mojo:97-119: up to 12 rows for speculative verify; here up to 16):
    every weight row read once for all rows, rel 1e-3."""
    import torch
    from aq import synth
    rng = np.random.default_rng(tokens * 100 + k)
    n = 21504 if k == 2048 else 3000
    wq, ws = synth.int4_matrix(rng, n, k, 32)
    x = rng.standard_normal((tokens, k)).astype(np.float32)
    y0 = rng.standard_normal((tokens, n)).astype(np.float32)
    y = to_dev(y0, dev)
    _ops().gemv_q4(to_dev(wq, dev), to_dev(ws, dev), to_dev(x, dev), y, 32, add=True)
    assert rel_inf(to_np(y), orc.gemm_q4(wq, ws, x, 32, y0=y0)) < TOL_FP32


@pytest.mark.parametrize("k,n", [(2048, 300), (8192, 2048)])
def test_non_finite_x_gives_nan(dev, k, n):
    """A NaN in x makes every output NaN, as the reference's fp32 sums do (0 * NaN included); the other tokens'
    outputs stay finite and correct."""
    import torch
    rng = np.random.default_rng(k + n)
    wq = rng.integers(0, 2 ** 32, (n, k // 8), dtype=np.uint32)
    ws = (np.abs(rng.standard_normal((n, k // 32))) * 0.02 + 1e-3).astype(np.float16)
    x = rng.standard_normal((2, k)).astype(np.float32)
    x[0, k // 3] = np.nan
    y = torch.empty((2, n), dtype=torch.float32, device=dev)
    for t in range(2):  # one token at a time: the decode forms
        yt = y[t]
        _ops().gemv_q4(to_dev(wq, dev), to_dev(ws, dev), to_dev(x[t], dev), yt, 32)
    got = to_np(y)
    assert np.isnan(got[0]).all()
    assert rel_inf(got[1], orc.gemv_q4(wq, ws, x[1], 32)) < TOL_FP32
