"""int4 (Q4W) GEMM on MFMA vs the oracle: p_gemm_q4 / lk.gemm_q4 (fp16 MFMA, fp32 accumulation)."""
import numpy as np
import pytest

from _util import exact_int4_product, kat_int4, rel_inf, rel_l2, to_dev, to_np
from oracle import aq_oracle as orc

pytestmark = pytest.mark.gpu

TOL_F16 = 1e-2  # rel (inf-norm) bar for fp16 MFMA with fp32 accumulation


def _gemm(x, wq, ws, group, dev, add_to=None):
    import torch
    from aq import ops
    m, n = x.shape[0], wq.shape[0]
    y = torch.zeros((m, n), dtype=torch.float32, device=dev) if add_to is None else to_dev(add_to, dev)
    ops.gemm_q4(to_dev(x, dev), to_dev(wq, dev), to_dev(ws, dev), y, group, add=add_to is not None)
    return to_np(y)


@pytest.mark.parametrize("m,n,k,group,xf32", [
    (16, 64, 128, 32, False), (431, 256, 2048, 32, False), (144, 512, 256, 32, False), (37, 300, 160, 32, False),
    (1, 16, 32, 32, False), (431, 3072, 2048, 64, True), (288, 256, 512, 128, False), (64, 192, 256, 16, False),
    (50, 80, 96, 8, True), (500, 1024, 1024, 32, False),
    # fp16 X with one, two or four scales per 128 k (one aligned scale load per row and super-step)
    (431, 512, 2048, 64, False), (200, 768, 1024, 128, False), (64, 256, 2048, 256, False),
    # scale rows that are not aligned for that load (K / group = 65, 33) take the general kernel
    (100, 256, 2080, 32, False), (90, 128, 2112, 64, False),
    # tall tiles (M > 112, 128 columns): one row past a whole block, ragged columns, one super-step, three row tiles
    (113, 130, 128, 32, False), (150, 200, 512, 32, False), (240, 1000, 384, 64, False), (700, 384, 256, 32, False),
    # narrow 128-column tiles in the eight-wave form (>= 16 super-steps a workgroup): the fused q|k|v of C1
    (431, 3072, 2048, 32, False),
    # one pass that would leave CUs idle takes shorter tiles (2 x 81 tiles of 7 blocks -> 3 x 81 of 5)
    (200, 20736, 128, 32, False),
    # more than 256 workgroups with 16 super-steps each: the four-wave form, two workgroups a CU
    (16, 65792, 2048, 32, False),
])
def test_kat_bit_exact(dev, m, n, k, group, xf32):
    """Integer-valued X, power-of-two scales: exact in fp16 and in fp32 accumulation, so the MFMA result must equal
    the exact product bit for bit. Pins the fragment layouts, the k permutation and the tile edges."""
    rng = np.random.default_rng(m * 7 + n + k + group)
    vals, ws, x = kat_int4(rng, n, k, group, tokens=m)
    x = x.astype(np.float32 if xf32 else np.float16)
    got = _gemm(x, orc.q4w_pack(vals), ws, group, dev)
    np.testing.assert_array_equal(got, exact_int4_product(vals, ws, x.astype(np.float32), group).astype(np.float32))


@pytest.mark.parametrize("name", ["q", "k", "o", "gate", "down"])
def test_c1_projection_parity(dev, name):
    """C1: Llama-3.2-1B projections at M = 431, fp16 activations, G = 32."""
    from aq import synth
    proj = {p[0]: p for p in synth.C1_PROJECTIONS}[name]
    d = synth.c1(projections=(proj,))
    wq, ws = d["mats"][name]
    x = d["x"][proj[2]]
    got = _gemm(x, wq, ws, 32, dev)
    ref = orc.gemm_q4(wq, ws, x.astype(np.float32), 32)
    assert rel_inf(got, ref) < TOL_F16
    assert rel_l2(got, ref) < 2e-3


def test_tall_tile_add(dev):
    """The residual form on tall tiles (fp16 X, M > 112), with and without a split of K."""
    rng = np.random.default_rng(31)
    for m, n, k in ((300, 384, 1024), (431, 640, 8192)):
        vals, ws, x = kat_int4(rng, n, k, 32, tokens=m)
        x = x.astype(np.float16)
        y0 = rng.integers(-4, 4, size=(m, n)).astype(np.float32)
        got = _gemm(x, orc.q4w_pack(vals), ws, 32, dev, add_to=y0)
        np.testing.assert_array_equal(got, (exact_int4_product(vals, ws, x.astype(np.float32), 32) + y0)
                                      .astype(np.float32))


def test_fp32_input_and_add(dev):
    """The reference's own p_gemm_q4 interface: fp32 X; plus the residual form."""
    rng = np.random.default_rng(3)
    m, n, k, g = 200, 512, 1024, 64
    wq = rng.integers(0, 2 ** 32, (n, k // 8), dtype=np.uint32)
    ws = (np.abs(rng.standard_normal((n, k // g))) * 0.02 + 1e-3).astype(np.float16)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    got = _gemm(x, wq, ws, g, dev, add_to=y0)
    ref = orc.gemm_q4(wq, ws, x, g, y0=y0)
    assert rel_inf(got, ref) < TOL_F16


@pytest.mark.parametrize("m,n,k", [(431, 512, 8192), (431, 2048, 2048), (64, 256, 4096), (100, 96, 1024)])
def test_split_k_kat(dev, m, n, k):
    """Shapes the planner splits along K (few tiles): partials in the workspace, reduced in split order."""
    from aq import _lib
    assert _lib.lib().aq_gemm_q4_workspace_bytes(m, n, k) > 0
    rng = np.random.default_rng(m + n + k)
    vals, ws, x = kat_int4(rng, n, k, 32, tokens=m)
    x = x.astype(np.float16)
    got = _gemm(x, orc.q4w_pack(vals), ws, 32, dev)
    np.testing.assert_array_equal(got, exact_int4_product(vals, ws, x.astype(np.float32), 32).astype(np.float32))
    y0 = rng.integers(-4, 4, size=(m, n)).astype(np.float32)
    got = _gemm(x, orc.q4w_pack(vals), ws, 32, dev, add_to=y0)
    np.testing.assert_array_equal(got, (exact_int4_product(vals, ws, x.astype(np.float32), 32) + y0)
                                  .astype(np.float32))


def test_split_k_leftover_workspace_and_graph(dev):
    """Split-K over a workspace the caller never clears: a workspace full of leftover bytes, calls in a row over it
    (the second adding onto Y), and replays of one captured call with new X each give the exact product."""
    import torch
    from aq import _lib
    m, n, k = 431, 512, 8192
    need = _lib.lib().aq_gemm_q4_workspace_bytes(m, n, k)
    assert need > 0
    rng = np.random.default_rng(77)
    vals, ws, x = kat_int4(rng, n, k, 32, tokens=m)
    x = x.astype(np.float16)
    want = exact_int4_product(vals, ws, x.astype(np.float32), 32)
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    wsp = torch.randint(0, 256, (need,), dtype=torch.uint8, device=dev, generator=gen)
    X, W, S = to_dev(x, dev), to_dev(orc.q4w_pack(vals), dev), to_dev(ws, dev)
    y = torch.empty((m, n), dtype=torch.float32, device=dev)
    torch.ops.aq.gemm_q4(X, W, S, y, 32, False, wsp)
    np.testing.assert_array_equal(to_np(y), want.astype(np.float32))
    y0 = rng.integers(-4, 4, size=(m, n)).astype(np.float32)
    y.copy_(to_dev(y0, dev))
    torch.ops.aq.gemm_q4(X, W, S, y, 32, True, wsp)
    np.testing.assert_array_equal(to_np(y), (want + y0).astype(np.float32))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        torch.ops.aq.gemm_q4(X, W, S, y, 32, False, wsp)
    for i in range(3):
        xi = rng.integers(-3, 4, size=(m, k)).astype(np.float16)
        X.copy_(to_dev(xi, dev))
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_np(y), exact_int4_product(vals, ws, xi.astype(np.float32), 32)
                                      .astype(np.float32), err_msg=f"replay {i}")


def test_no_workspace_single_pass(dev):
    """A workspace smaller than asked for falls back to one pass over K, with the same result."""
    import torch
    rng = np.random.default_rng(12)
    m, n, k = 431, 512, 4096
    vals, ws, x = kat_int4(rng, n, k, 32, tokens=m)
    x = x.astype(np.float16)
    y = torch.zeros((m, n), dtype=torch.float32, device=dev)
    tiny = torch.empty(16, dtype=torch.uint8, device=dev)
    torch.ops.aq.gemm_q4(to_dev(x, dev), to_dev(orc.q4w_pack(vals), dev), to_dev(ws, dev), y, 32, False, tiny)
    np.testing.assert_array_equal(to_np(y), exact_int4_product(vals, ws, x.astype(np.float32), 32)
                                  .astype(np.float32))


@pytest.mark.parametrize("m,n,k,group,xf32", [
    (431, 512, 2048, 32, False),   # fp16 X, the direct-to-LDS kernel in its eight-wave form
    (431, 2048, 8192, 32, False),  # K split: fp32 partials summed in split order
    (200, 384, 1024, 64, True),    # fp32 X (the reference's p_gemm_q4 interface), rounded to fp16 when staged
    (128, 256, 2048, 128, False),
    (90, 128, 2112, 64, False),    # K % 128 != 0: the general kernel
])
def test_elementwise_error_bound(dev, m, n, k, group, xf32):
    """Every output, not only the largest, within 1e-3 of its own scale: |y - ref| <= 1e-3 * (|X| . |W|^T)
    elementwise, against float64 over the exact dequantised weights. The error sources bound it: each dequantised
    weight rounded to fp16 (2^-11 relative), fp32 X rounded to fp16 (2^-11), fp32 accumulation. X spans four decades,
    and the bound is relative to |X| . |W|^T rather than |y|, so it also holds the outputs whose sums nearly cancel."""
    from aq import synth
    rng = np.random.default_rng(m + n + k + group + (7 if xf32 else 0))
    wq, ws = synth.int4_matrix(rng, n, k, group)
    x = (rng.standard_normal((m, k)) * 10.0 ** rng.uniform(-2, 2, size=(m, k))).astype(
        np.float32 if xf32 else np.float16)
    got = _gemm(x, wq, ws, group, dev).astype(np.float64)
    w = orc.q4w_dequant(wq, ws, group).astype(np.float64)
    xd = x.astype(np.float64)
    ref = xd @ w.T
    scale = np.abs(xd) @ np.abs(w).T
    worst = float(np.max(np.abs(got - ref) / scale))
    assert worst <= 1e-3, worst
