"""The oracle's weight-format functions against the reference's own C converters (CPU).

Fixtures: tests/golden/ref_*.npz, written by tests/golden/make_ref_vectors.py from llama/st2bin.c,
qwen3moe/convert.c and lfm2/convert.c, compiled from the reference's sources by oracle/Makefile. When oracle/_ref
holds those binaries, the same checks also run on fresh random inputs. Bit-exact throughout.
"""
import importlib.util
from pathlib import Path

import numpy as np
import pytest

from oracle import aq_oracle as orc

GOLDEN = Path(__file__).resolve().parent / "golden"
REF = Path(__file__).resolve().parent.parent / "oracle" / "_ref"


def _gen():
    spec = importlib.util.spec_from_file_location("make_ref_vectors", GOLDEN / "make_ref_vectors.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _check_st2bin(src, words, scales):
    w16 = _gen().bf16_to_f32(src).astype(np.float16)  # st2bin rounds each bf16 weight to fp16 first
    q, s, _ = orc.quantize4(w16, 64)
    np.testing.assert_array_equal(s.view(np.uint16), scales.view(np.uint16))
    np.testing.assert_array_equal(q, words)


def _check_qwen3moe(src, group, words, scales):
    q, s = orc.quantize4_searched(_gen().bf16_to_f32(src), group)
    np.testing.assert_array_equal(s.view(np.uint16), scales.view(np.uint16))
    np.testing.assert_array_equal(q, words)


def _check_lfm2(raw, rows, cols, words, scales, h4):
    q, s = orc.gguf_q4_0_to_q4w(raw, rows, cols)
    np.testing.assert_array_equal(q, words)
    np.testing.assert_array_equal(s.view(np.uint16), scales.view(np.uint16))
    h = orc.gguf_q4_0_dequant(raw, rows, cols).astype(np.float16)
    np.testing.assert_array_equal(h.view(np.uint16), h4.view(np.uint16))


def _check_lfm2_q6(raw, rows, cols, q6, d6, h6):
    q, d = orc.gguf_q6_k_to_q6w(raw, rows, cols)
    np.testing.assert_array_equal(q, q6)
    np.testing.assert_array_equal(d.view(np.uint16), d6.view(np.uint16))
    h = orc.q6w_dequant(q, d).astype(np.float16)
    np.testing.assert_array_equal(h.view(np.uint16), h6.view(np.uint16))


def test_quantize4_vs_st2bin_fixture():
    d = np.load(GOLDEN / "ref_st2bin_q4.npz")
    _check_st2bin(d["src_bf16"], d["words"], d["scales"])
    assert (d["scales"][0, 0] == 0) and np.all(d["words"][0, :8] == 0)  # the planted all-zero group


@pytest.mark.parametrize("group", [32, 64, 128])
def test_quantize4_searched_vs_qwen3moe_fixture(group):
    d = np.load(GOLDEN / "ref_qwen3moe_q4.npz")
    _check_qwen3moe(d[f"src_bf16_g{group}"], group, d[f"words_g{group}"], d[f"scales_g{group}"])


def test_gguf_q4_0_vs_lfm2_fixture():
    d = np.load(GOLDEN / "ref_lfm2_q4.npz")
    raw = d["raw"]
    rows, cols = raw.shape[0], raw.shape[1] // 18 * 32
    _check_lfm2(raw, rows, cols, d["words"], d["scales"], d["h4"])


def test_gguf_q6_k_vs_lfm2_fixture():
    d = np.load(GOLDEN / "ref_lfm2_q6.npz")
    raw = d["raw"]
    rows, cols = raw.shape[0], raw.shape[1] // 210 * 256
    _check_lfm2_q6(raw, rows, cols, d["q"], d["d"], d["h6"])
    sc = d["q"][0, 0, 192:208].view(np.int8)
    assert tuple(sc[:3]) == (-128, 0, 127) and float(d["d"][0, 0]) == 0.0  # the planted extremes


def test_q6_values_vs_pointer_walk():
    """The vectorised Q6_K unpacking against a scalar walk in the reference's own loop shape (two 128-weight halves,
    four quarter outputs per l, then ql += 64, qh += 32, sc += 8): every element's position, bits and scale."""
    rng = np.random.default_rng(3)
    blk = rng.integers(0, 256, 208, dtype=np.uint8)
    d = np.array([[1.0]], np.float16)
    vals, ds = orc.q6w_values(blk.reshape(1, 1, 208), d)
    want_v, want_s = np.zeros(256, int), np.zeros(256)
    ql, qh, sc = 0, 128, 192
    for n in (0, 128):
        for l in range(32):
            for j, (b, shift, hs) in enumerate([(ql + l, 0, 0), (ql + l + 32, 0, 2), (ql + l, 4, 4),
                                                (ql + l + 32, 4, 6)]):
                want_v[n + l + 32 * j] = (((int(blk[b]) >> shift) & 15) | (((int(blk[qh + l]) >> hs) & 3) << 4)) - 32
                want_s[n + l + 32 * j] = np.int8(blk[sc + l // 16 + 2 * j])
        ql, qh, sc = ql + 64, qh + 32, sc + 8
    np.testing.assert_array_equal(vals[0], want_v)
    np.testing.assert_array_equal(np.repeat(ds[0], 16), want_s)
    assert vals.min() >= -32 and vals.max() <= 31


def test_fixture_plants_rounding_ties():
    """Row 2 of each fixture holds exact .5 quotients: the reference rounded them to even, as the oracle must."""
    d = np.load(GOLDEN / "ref_st2bin_q4.npz")
    codes = orc.q4w_values(d["words"])[2, :8]
    # values 7, .5, 1.5, 2.5, -.5, -1.5, -2.5, 3.5 with s = 1 -> 7, 0, 2, 2, 0, -2, -2, 4
    assert list(codes) == [7, 0, 2, 2, 0, -2, -2, 4]


_HAVE_REF = all((REF / b).exists() for b in ("llama_st2bin", "qwen3moe_convert", "lfm2_convert"))


@pytest.mark.skipif(not _HAVE_REF, reason="oracle/_ref not built (make -C oracle needs /root/reference)")
@pytest.mark.parametrize("seed", [1, 2])
def test_live_reference_binaries(seed):
    g = _gen()
    rng = np.random.default_rng(1000 + seed)
    src = g.bf16_matrix(rng, 8, 256, 64)
    _check_st2bin(src, *g.st2bin_q4(src))
    for group in (32, 128):
        src = g.bf16_matrix(rng, 8, 256, group)
        _check_qwen3moe(src, group, *g.qwen3moe_q4(src, group))
    raw = g.q4_0_blocks(rng, 6, 128)
    _check_lfm2(raw, 6, 128, *g.lfm2_q4(raw, 6, 128))
    raw = g.q6_k_blocks(rng, 3, 768)
    _check_lfm2_q6(raw, 3, 768, *g.lfm2_q6(raw, 3, 768))
