"""Pins the oracle's ternary (T2W) and fp16-pair (X2H) arithmetic."""
import math

import numpy as np
import pytest

from oracle import aq_oracle as orc


def test_t2w_known_word_and_index_map():
    # codes of k = 0..15 for one output column: 0,1,2,0,1,2,... -> bits 2k
    codes = np.array([[i % 3 for i in range(16)]], np.uint8)
    w = orc.t2w_pack(codes)
    expect = sum((i % 3) << (2 * i) for i in range(16))
    assert w.shape == (1, 1) and int(w[0, 0]) == expect
    # word (k/16, n) of a 2-column, 32-k matrix: brute-force index map of prefill.mojo:228-230
    rng = np.random.default_rng(0)
    c = rng.integers(0, 3, size=(2, 32))
    w = orc.t2w_pack(c)
    assert w.shape == (2, 2)
    for n in range(2):
        for k in range(32):
            assert (int(w[k // 16, n]) >> (2 * (k % 16))) & 3 == c[n, k]
    np.testing.assert_array_equal(orc.t2w_codes(w), c)


def test_t2w_dequant_brute_force():
    rng = np.random.default_rng(1)
    n, k = 3, 256
    c = rng.integers(0, 3, size=(n, k))
    s = (np.abs(rng.standard_normal((k // 128, n))) * 0.02).astype(np.float16)
    got = orc.t2w_dequant(orc.t2w_pack(c), s)
    for r in range(n):
        for kk in range(k):
            assert float(got[r, kk]) == (c[r, kk] - 1) * float(s[kk // 128, r])


def test_x2h_known_bits_and_rounding():
    w = orc.x2h_pack(np.array([1.0, -2.0], np.float32))
    assert int(w[0]) == 0xC0003C00  # fp16 1.0 = 0x3C00 in the low half (even k), -2.0 = 0xC000 high
    # round to nearest even: 1 + 2^-11 is halfway between 1 and 1 + 2^-10 -> 1.0; 1 + 3*2^-11 -> 1 + 2^-9
    w = orc.x2h_pack(np.array([1 + 2 ** -11, 1 + 3 * 2 ** -11], np.float32))
    assert int(w[0]) & 0xFFFF == 0x3C00 and int(w[0]) >> 16 == 0x3C02
    x = np.array([0.5, 3.25, -7.0, 1e-3], np.float32)
    np.testing.assert_array_equal(orc.x2h_unpack(orc.x2h_pack(x)), x.astype(np.float16).astype(np.float32))


def test_ternary_gemv_partials_and_gemm_brute_force():
    rng = np.random.default_rng(2)
    n, k = 5, 2048 + 128
    c = rng.integers(0, 3, size=(n, k))
    s = (np.abs(rng.standard_normal((k // 128, n))) * 0.02).astype(np.float16)
    w = orc.t2w_pack(c)
    x = rng.standard_normal(k).astype(np.float32)
    xh = orc.x2h_pack(x)
    xv = x.astype(np.float16).astype(np.float64)
    y = orc.ternary_gemv(w, s, xh, n, k)
    parts = orc.ternary_partials(w, s, xh, n, k)
    assert parts.shape == (3, n)  # ceil(2176 / 1024) partial rows
    np.testing.assert_allclose(parts.sum(0), y, rtol=1e-12, atol=1e-12)
    for r in range(n):
        ref = math.fsum((c[r, kk] - 1) * float(s[kk // 128, r]) * xv[kk] for kk in range(k))
        assert y[r] == pytest.approx(ref, rel=1e-12, abs=1e-12)
    X = rng.standard_normal((2, k)).astype(np.float32)
    Y = orc.ternary_gemm(X, w, s)
    for i in range(2):
        for r in range(n):
            ref = math.fsum((c[r, kk] - 1) * float(s[kk // 128, r]) * float(X[i, kk]) for kk in range(k))
            assert Y[i, r] == pytest.approx(ref, rel=1e-12, abs=1e-12)


def test_rmsnorm_and_swiglu_pack():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(256).astype(np.float32)
    w = rng.standard_normal(256).astype(np.float32)
    r = 1 / math.sqrt(sum(float(v) ** 2 for v in x) / 256 + 1e-6)
    ref = np.array([float(x[i]) * r * float(w[i]) for i in range(256)])
    got = orc.x2h_unpack(orc.rmsnorm_pack(x, w))
    np.testing.assert_allclose(got, ref, rtol=2 ** -10, atol=1e-6)
    gu = rng.standard_normal(2 * 64).astype(np.float32)
    got = orc.x2h_unpack(orc.swiglu_pack(gu, 64))
    ref = [float(gu[i]) / (1 + math.exp(-float(gu[i]))) * float(gu[64 + i]) for i in range(64)]
    np.testing.assert_allclose(got, ref, rtol=2 ** -10, atol=1e-6)
