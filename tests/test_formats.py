"""libaq's weight-format converters (host code, CPU) vs the reference's own converters and the oracle. Bit-exact.

The golden fixtures come from llama/st2bin.c, qwen3moe/convert.c and lfm2/convert.c compiled from the reference's
sources (tests/golden/make_ref_vectors.py); random inputs are checked against the oracle's numpy restatements, whose
fp16 rounding is numpy's own (an independent implementation of the conversion the library does by hand).
"""
import ctypes
from pathlib import Path

import numpy as np
import pytest

from oracle import aq_oracle as orc

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def fmt():
    from aq import formats
    return formats


def _u16(a):
    return np.asarray(a).view(np.uint16)


def test_quantize_q4_bf16_vs_st2bin(fmt):
    d = np.load(GOLDEN / "ref_st2bin_q4.npz")
    wq, ws = fmt.quantize_q4(d["src_bf16"], 64, bf16=True)
    np.testing.assert_array_equal(wq, d["words"])
    np.testing.assert_array_equal(_u16(ws), _u16(d["scales"]))


@pytest.mark.parametrize("group", [32, 64, 128])
def test_quantize_q4_searched_vs_qwen3moe(fmt, group):
    d = np.load(GOLDEN / "ref_qwen3moe_q4.npz")
    wq, ws = fmt.quantize_q4_searched(d[f"src_bf16_g{group}"], group)
    np.testing.assert_array_equal(wq, d[f"words_g{group}"])
    np.testing.assert_array_equal(_u16(ws), _u16(d[f"scales_g{group}"]))


def test_gguf_q4_0_vs_lfm2(fmt):
    d = np.load(GOLDEN / "ref_lfm2_q4.npz")
    raw = d["raw"]
    rows, cols = raw.shape[0], raw.shape[1] // 18 * 32
    wq, ws = fmt.gguf_q4_0_to_q4w(raw, rows, cols)
    np.testing.assert_array_equal(wq, d["words"])
    np.testing.assert_array_equal(_u16(ws), _u16(d["scales"]))
    np.testing.assert_array_equal(_u16(fmt.gguf_q4_0_to_f16(raw, rows, cols)), _u16(d["h4"]))


@pytest.mark.parametrize("group", [8, 32, 64, 128])
def test_quantize_q4_fp16_vs_oracle_across_exponents(fmt, group):
    """Weights spread over fp16's whole exponent range (incl. subnormal scales) exercise every rounding path of the
    library's float -> fp16 conversion against numpy's."""
    rng = np.random.default_rng(group)
    rows, cols = 64, 256
    mag = 2.0 ** rng.uniform(-24, 15, size=(rows, cols // group, 1))
    w = (rng.standard_normal((rows, cols // group, group)) * mag).reshape(rows, cols)
    w = np.clip(w, -60000, 60000).astype(np.float16)
    w[0, :group] = 0
    q_ref, s_ref, _ = orc.quantize4(w, group)
    q, s = fmt.quantize_q4(w, group)
    np.testing.assert_array_equal(_u16(s), _u16(s_ref))
    np.testing.assert_array_equal(q, q_ref)


@pytest.mark.parametrize("group", [16, 32, 256])
def test_quantize_q4_searched_vs_oracle(fmt, group):
    rng = np.random.default_rng(100 + group)
    w = (rng.standard_normal((32, 512)) * 2.0 ** rng.uniform(-20, 8, size=(32, 1))).astype(np.float32)
    bits = (w.view(np.uint32) >> 16).astype(np.uint16)  # truncated to bf16: any bf16 pattern will do
    q_ref, s_ref = orc.quantize4_searched((bits.astype(np.uint32) << 16).view(np.float32), group)
    q, s = fmt.quantize_q4_searched(bits, group)
    np.testing.assert_array_equal(_u16(s), _u16(s_ref))
    np.testing.assert_array_equal(q, q_ref)


def test_gguf_q6_k_vs_lfm2(fmt):
    d = np.load(GOLDEN / "ref_lfm2_q6.npz")
    raw = d["raw"]
    rows, cols = raw.shape[0], raw.shape[1] // 210 * 256
    q, dd = fmt.gguf_q6_k_to_q6w(raw, rows, cols)
    np.testing.assert_array_equal(q, d["q"])
    np.testing.assert_array_equal(_u16(dd), _u16(d["d"]))
    np.testing.assert_array_equal(_u16(fmt.gguf_q6_k_to_f16(raw, rows, cols)), _u16(d["h6"]))


def test_gguf_q6_k_vs_oracle_random(fmt):
    rng = np.random.default_rng(9)
    rows, cols = 5, 1024
    raw = rng.integers(0, 256, size=rows * cols // 256 * 210, dtype=np.uint8)
    d = (rng.standard_normal(rows * cols // 256) * 0.01).astype(np.float16)
    raw.reshape(-1, 210)[:, 208:] = d.view(np.uint8).reshape(-1, 2)
    q_ref, d_ref = orc.gguf_q6_k_to_q6w(raw, rows, cols)
    q, dd = fmt.gguf_q6_k_to_q6w(raw, rows, cols)
    np.testing.assert_array_equal(q, q_ref)
    np.testing.assert_array_equal(_u16(dd), _u16(d_ref))
    h = fmt.gguf_q6_k_to_f16(raw, rows, cols)
    np.testing.assert_array_equal(_u16(h), _u16(orc.q6w_dequant(q_ref, d_ref).astype(np.float16)))
    with pytest.raises(ValueError):
        fmt.gguf_q6_k_to_q6w(raw, rows, 1000)


def test_gguf_vs_oracle_random(fmt):
    rng = np.random.default_rng(7)
    rows, cols = 10, 320
    raw = rng.integers(0, 256, size=rows * cols // 32 * 18, dtype=np.uint8)
    d = (np.abs(rng.standard_normal(rows * cols // 32)) * 0.05).astype(np.float16)
    raw.reshape(-1, 18)[:, :2] = d.view(np.uint8).reshape(-1, 2)
    q_ref, s_ref = orc.gguf_q4_0_to_q4w(raw, rows, cols)
    q, s = fmt.gguf_q4_0_to_q4w(raw, rows, cols)
    np.testing.assert_array_equal(q, q_ref)
    np.testing.assert_array_equal(_u16(s), _u16(s_ref))
    h = fmt.gguf_q4_0_to_f16(raw, rows, cols)
    np.testing.assert_array_equal(_u16(h), _u16(orc.gguf_q4_0_dequant(raw, rows, cols).astype(np.float16)))


def test_t2w_from_mlx_vs_oracle(fmt):
    rng = np.random.default_rng(8)
    k = 512
    parts = []
    for n in (40, 24, 64):
        codes = rng.integers(0, 2 ** 32, size=(n, k // 16), dtype=np.uint32)
        sc = (np.abs(rng.standard_normal((n, k // 128))) * 0.02).astype(np.float16)
        parts.append((codes, sc, (-sc.astype(np.float32)).astype(np.float16)))
    w, s = fmt.t2w_from_mlx(parts, k)
    w_ref, s_ref = orc.mlx_to_t2w(parts, k)
    np.testing.assert_array_equal(w, w_ref)
    np.testing.assert_array_equal(_u16(s), _u16(s_ref))


def _mlx_affine_dequant(codes, scales, biases, k):
    """MLX's published 2-bit affine format (mlx.core.quantize with bits = 2, group_size = 128, the quantisation
    qwen3/export.py:41 asserts): element k of row n is bits 2 (k % 16) of word k / 16 (16 codes per uint32, lowest
    bits first) and its value is code * scales[n, k/128] + biases[n, k/128]. A pure-Python bit walk in float64,
    independent of both converters."""
    n = codes.shape[0]
    out = np.zeros((n, k))
    for r in range(n):
        for kk in range(k):
            code = (int(codes[r, kk // 16]) >> (2 * (kk % 16))) & 3
            out[r, kk] = code * float(scales[r, kk // 128]) + float(biases[r, kk // 128])
    return out


def test_t2w_from_mlx_closed_form(fmt):
    """Pins the MLX -> T2W converter (qwen3/convert.cpp:39-74) to MLX's own dequantisation: the fused T2W matrix,
    dequantised as T2W ((code - 1) * s), equals every part's MLX value code * scale + bias stacked along N, for the
    library's C++ and the oracle alike. Codes cover 0..3 (3 is 2 * scale when bias = -scale). A planted swap of two
    parts and an untransposed word layout both fail the same check."""
    rng = np.random.default_rng(13)
    k = 256
    parts, mlx = [], []
    for n in (24, 8, 40):
        codes = rng.integers(0, 2 ** 32, size=(n, k // 16), dtype=np.uint32)
        sc = (np.abs(rng.standard_normal((n, k // 128))) * 0.02).astype(np.float16)
        bi = (-sc.astype(np.float32)).astype(np.float16)
        parts.append((codes, sc, bi))
        mlx.append(_mlx_affine_dequant(codes, sc, bi, k))
    want = np.concatenate(mlx, axis=0)  # [sum n, K]

    def matches(w, s):
        return w.shape == (k // 16, want.shape[0]) and np.array_equal(orc.t2w_dequant(w, s).astype(np.float64), want)

    assert matches(*fmt.t2w_from_mlx(parts, k))
    assert matches(*orc.mlx_to_t2w(parts, k))
    # planted mistakes the check must catch
    assert not matches(*orc.mlx_to_t2w([parts[1], parts[0], parts[2]], k))     # parts in the wrong order
    w, s = orc.mlx_to_t2w(parts, k)
    flat = np.concatenate([c for c, _, _ in parts], axis=0)                     # codes left [N, K/16] row-major
    assert not matches(np.ascontiguousarray(flat.reshape(k // 16, -1)), s)      # ... read as if transposed


def test_t2w_from_mlx_rejects_non_ternary(fmt):
    from aq import AqError
    k = 256
    codes = np.zeros((4, k // 16), np.uint32)
    sc = np.full((4, k // 128), 0.5, np.float16)
    bi = (-sc.astype(np.float32)).astype(np.float16)
    bi[2, 1] = np.float16(-0.25)
    with pytest.raises(AqError, match="invalid argument|status 7"):
        fmt.t2w_from_mlx([(codes, sc, bi)], k)
    with pytest.raises(ValueError):
        orc.mlx_to_t2w([(codes, sc, bi)], k)


def test_converter_errors(fmt):
    from aq import AqError, _lib
    with pytest.raises(AqError):
        fmt.quantize_q4(np.zeros((2, 96), np.float16), 64)  # cols % group
    with pytest.raises(AqError):
        fmt.quantize_q4_searched(np.zeros((2, 1024), np.uint16), 512)  # group > 256
    assert _lib.lib().aq_gguf_q4_0_to_q4w(None, 1, 32, None, None) == 5  # AQ_ERR_NULL
    assert _lib.lib().aq_gguf_q4_0_to_f16(ctypes.c_void_p(8), 1, 33, ctypes.c_void_p(8)) == 1  # AQ_ERR_SHAPE


def test_t2w_scales_from_bonsai_pairs(fmt):
    """bonsai/convert.cpp's fp32 (scale, bias) pairs of a ternary matrix give back its fp16 scales exactly; a
    non-ternary group, or a scale fp16 cannot hold, is refused and nothing is written."""
    from aq import AqError
    rng = np.random.default_rng(11)
    s16 = (np.abs(rng.standard_normal((16, 300))) * 0.02).astype(np.float16)
    s16[0, 0] = np.float16(6e-8)   # fp16 subnormal
    s16[1, 1] = np.float16(0.0)
    pairs = np.stack([s16.astype(np.float32), -s16.astype(np.float32)], axis=-1)
    got = fmt.t2w_scales_from_pairs(pairs)
    np.testing.assert_array_equal(_u16(got), _u16(s16))
    np.testing.assert_array_equal(_u16(got), _u16(orc.bonsai_pairs_to_t2w_scales(pairs)))
    bad = pairs.copy()
    bad[3, 7, 1] += 1e-3           # bias != -scale: an affine 2-bit group
    with pytest.raises(AqError):
        fmt.t2w_scales_from_pairs(bad)
    with pytest.raises(ValueError):
        orc.bonsai_pairs_to_t2w_scales(bad)
    bad = pairs.copy()
    bad[2, 2] = [0.1, -0.1]        # 0.1 is not an fp16 value
    with pytest.raises(AqError):
        fmt.t2w_scales_from_pairs(bad)
