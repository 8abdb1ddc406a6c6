"""Pins the oracle's int4 (Q4W) arithmetic against known answers, textbook two's complement and brute force."""
import math

import numpy as np
import pytest

from _util import exact_int4_product, kat_int4
from oracle import aq_oracle as orc


def _brute_values(word: int):
    """Textbook 4-bit two's complement, nibble j at bits 4j (written independently of the oracle's XOR form)."""
    out = []
    for j in range(8):
        nib = (word >> (4 * j)) & 0xF
        out.append(nib - 16 if nib >= 8 else nib)
    return out


@pytest.mark.parametrize("word,vals", [
    (0x76543210, [0, 1, 2, 3, 4, 5, 6, 7]),
    (0xFEDCBA98, [-8, -7, -6, -5, -4, -3, -2, -1]),
    (0x00000000, [0] * 8),
    (0xFFFFFFFF, [-1] * 8),
    (0x8000000F, [-1, 0, 0, 0, 0, 0, 0, -8]),
])
def test_known_words(word, vals):
    assert orc.q4w_values(np.array([[word]], np.uint32))[0].tolist() == vals


def test_values_match_brute_force():
    rng = np.random.default_rng(0)
    words = rng.integers(0, 2 ** 32, size=(7, 5), dtype=np.uint32)
    got = orc.q4w_values(words)
    for r in range(7):
        ref = sum((_brute_values(int(w)) for w in words[r]), [])
        assert got[r].tolist() == ref


def test_pack_roundtrip_and_layout():
    rng = np.random.default_rng(1)
    q = rng.integers(-8, 8, size=(6, 40))
    wq = orc.q4w_pack(q)
    assert wq.shape == (6, 5) and wq.dtype == np.uint32
    np.testing.assert_array_equal(orc.q4w_values(wq), q)
    # element k of a row sits in word k // 8 at bits 4 * (k % 8), low nibble first
    assert int(orc.q4w_pack(np.array([[1, 0, 0, 0, 0, 0, 0, 0]]))[0, 0]) == 0x1
    assert int(orc.q4w_pack(np.array([[0, 0, 0, 0, 0, 0, 0, -8]]))[0, 0]) == 0x80000000
    with pytest.raises(ValueError):
        orc.q4w_pack(np.array([[8] * 8]))


def test_dequant_exact_and_scale_index():
    rng = np.random.default_rng(2)
    n, k, g = 3, 96, 32
    q = rng.integers(-8, 8, size=(n, k))
    ws = rng.standard_normal((n, k // g)).astype(np.float16)
    got = orc.q4w_dequant(orc.q4w_pack(q), ws, g)
    for r in range(n):
        for c in range(k):
            assert float(got[r, c]) == q[r, c] * float(ws[r, c // g])  # exact: small int x fp16 fits fp32


@pytest.mark.parametrize("n,k,g", [(3, 64, 32), (5, 48, 16), (2, 128, 64), (4, 24, 8)])
def test_gemv_brute_force(n, k, g):
    rng = np.random.default_rng(n + k + g)
    q = rng.integers(-8, 8, size=(n, k))
    ws = (rng.standard_normal((n, k // g)) * 0.05).astype(np.float16)
    x = rng.standard_normal(k).astype(np.float32)
    y0 = rng.standard_normal(n).astype(np.float32)
    got = orc.gemv_q4(orc.q4w_pack(q), ws, x, g)
    got_add = orc.gemv_q4(orc.q4w_pack(q), ws, x, g, y0=y0)
    for r in range(n):
        ref = math.fsum(q[r, c] * float(ws[r, c // g]) * float(x[c]) for c in range(k))
        assert got[r] == pytest.approx(ref, rel=1e-12, abs=1e-12)
        assert got_add[r] == pytest.approx(ref + float(y0[r]), rel=1e-12, abs=1e-12)


def test_gemm_brute_force_nonsquare():
    rng = np.random.default_rng(5)
    m, n, k, g = 3, 5, 64, 32
    q = rng.integers(-8, 8, size=(n, k))
    ws = (rng.standard_normal((n, k // g)) * 0.05).astype(np.float16)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got = orc.gemm_q4(orc.q4w_pack(q), ws, x, g)
    assert got.shape == (m, n)
    for i in range(m):
        for r in range(n):
            ref = math.fsum(q[r, c] * float(ws[r, c // g]) * float(x[i, c]) for c in range(k))
            assert got[i, r] == pytest.approx(ref, rel=1e-12, abs=1e-12)


def test_gemv_integer_kat_exact():
    rng = np.random.default_rng(9)
    vals, ws, x = kat_int4(rng, 17, 256, 32, tokens=2)
    got = orc.gemm_q4(orc.q4w_pack(vals), ws, x, 32)
    np.testing.assert_array_equal(got, exact_int4_product(vals, ws, x, 32))


def test_gate_up_brute_force():
    rng = np.random.default_rng(4)
    f, k, g = 3, 64, 32
    q = rng.integers(-8, 8, size=(2 * f, k))
    ws = (rng.standard_normal((2 * f, k // g)) * 0.1).astype(np.float16)
    x = rng.standard_normal(k).astype(np.float32)
    got = orc.gate_up_q4(orc.q4w_pack(q), ws, x, g, f)
    for j in range(f):
        dot = [math.fsum(q[r, c] * float(ws[r, c // g]) * float(x[c]) for c in range(k)) for r in (j, f + j)]
        ref = dot[0] / (1 + math.exp(-dot[0])) * dot[1]
        assert got[j] == pytest.approx(ref, rel=1e-12, abs=1e-14)
