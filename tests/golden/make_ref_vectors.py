"""Golden vectors from the reference's own C weight converters, built from their sources by oracle/Makefile.

    make -C oracle                      # builds oracle/_ref/{llama_st2bin, qwen3moe_convert, lfm2_convert}
    python tests/golden/make_ref_vectors.py         # every fixture; `... make_ref_vectors.py q6` the Q6_K one only

Each converter reads raw input bytes at the offsets its recipe names (no real checkpoint is needed), so this script
writes seeded synthetic inputs, runs the converter on a recipe, reads the output bytes back and stores inputs and
outputs as small .npz fixtures beside this file:

  ref_st2bin_q4.npz    llama/st2bin.c "q4" (quantize4: s = fp16(max|w| / 7), G = 64) on bf16 rows
  ref_qwen3moe_q4.npz  qwen3moe/convert.c "q4" (least-squared-error scale over d = 6.5 .. 9) for G = 32, 64, 128
  ref_lfm2_q4.npz      lfm2/convert.c "q4" (GGUF Q4_0 -> Q4W words + scales) and "h4" (Q4_0 -> fp16)
  ref_lfm2_q6.npz      lfm2/convert.c "q6" (GGUF Q6_K -> 208-byte super-blocks + d) and "h6" (Q6_K -> fp16)

The inputs include the cases the quantizers branch on: an all-zero group (scale 0), exact .5 quotients (rintf ties
to even), fp16-subnormal magnitudes and groups whose max is negative. tests/test_oracle_golden.py checks the oracle
against these fixtures bit for bit, and against fresh runs of the binaries when oracle/_ref is present.
"""
from __future__ import annotations

import subprocess
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REF = HERE.parent.parent / "oracle" / "_ref"


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (the inputs are then exactly representable)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_matrix(rng: np.random.Generator, rows: int, cols: int, group: int) -> np.ndarray:
    """bf16 bits [rows, cols] with the quantizers' edge cases planted in the first groups."""
    w = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    w[0, :group] = 0.0                                   # all-zero group: scale 0, codes 0
    w[1, :group] = -np.abs(w[1, :group])                 # max |w| taken by a negative value
    w[1, 0] = -0.7
    # exact .5 quotients under s = max/7: max 7, values k + 0.5 -> rintf ties to even
    w[2, :group] = np.resize(np.array([7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5], np.float32), group)
    w[3, :group] = np.float32(3e-6) * rng.standard_normal(group).astype(np.float32)  # fp16 subnormals
    w[4, :group] = np.float32(1000.0) * rng.standard_normal(group).astype(np.float32)  # large magnitudes
    return bf16_bits(w).reshape(rows, cols)


def run(binary: str, args: list[str]):
    exe = REF / binary
    if not exe.exists():
        raise SystemExit(f"{exe} missing: run `make -C oracle` first")
    subprocess.run([str(exe), *args], check=True, capture_output=True)


def st2bin_q4(src_bits: np.ndarray):
    """llama/st2bin.c recipe line `q4 <out q> <out s> <src> <rows> <cols>` (G = 64)."""
    rows, cols = src_bits.shape
    with tempfile.TemporaryDirectory() as d:
        d = Path(d)
        (d / "in.bin").write_bytes(src_bits.tobytes())
        qbytes, sbytes = rows * cols // 2, rows * cols // 64 * 2
        (d / "recipe.txt").write_text(f"size {qbytes + sbytes}\nq4 0 {qbytes} 0 {rows} {cols}\n")
        run("llama_st2bin", [str(d / "in.bin"), str(d / "recipe.txt"), str(d), str(d / "out.bin")])
        out = (d / "out.bin").read_bytes()
    words = np.frombuffer(out[:qbytes], np.uint32).reshape(rows, cols // 8)
    scales = np.frombuffer(out[qbytes:qbytes + sbytes], np.float16).reshape(rows, cols // 64)
    return words.copy(), scales.copy()


def qwen3moe_q4(src_bits: np.ndarray, group: int):
    """qwen3moe/convert.c recipe lines `src <shard>` + `q4 <out q> <out s> <src> <rows> <cols> <group>`."""
    rows, cols = src_bits.shape
    with tempfile.TemporaryDirectory() as d:
        d = Path(d)
        (d / "shard.bin").write_bytes(src_bits.tobytes())
        qbytes, sbytes = rows * cols // 2, rows * cols // group * 2
        (d / "recipe.txt").write_text(f"size {qbytes + sbytes}\nsrc shard.bin\nq4 0 {qbytes} 0 {rows} {cols} {group}\n")
        run("qwen3moe_convert", [str(d), str(d / "recipe.txt"), str(d / "out.bin")])
        out = (d / "out.bin").read_bytes()
    words = np.frombuffer(out[:qbytes], np.uint32).reshape(rows, cols // 8)
    scales = np.frombuffer(out[qbytes:qbytes + sbytes], np.float16).reshape(rows, cols // group)
    return words.copy(), scales.copy()


def q4_0_blocks(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    """Random GGUF Q4_0 rows: per 32 weights an fp16 d (incl. 0, negative, subnormal) and 16 nibble bytes."""
    nb = rows * cols // 32
    d = (np.abs(rng.standard_normal(nb)) * 0.02).astype(np.float16)
    d[0] = 0.0
    d[1] = -d[1]
    d[2] = np.float16(3e-7)
    b = np.zeros((nb, 18), np.uint8)
    b[:, :2] = d.view(np.uint8).reshape(nb, 2)
    b[:, 2:] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
    return b.reshape(rows, cols // 32 * 18)


def lfm2_q4(raw: np.ndarray, rows: int, cols: int):
    """lfm2/convert.c recipe lines `q4 <src> <rows> <cols> <out q> <out s>` and `h4 <src> <rows> <cols> <out>`."""
    with tempfile.TemporaryDirectory() as d:
        d = Path(d)
        (d / "model.gguf").write_bytes(raw.tobytes())
        qbytes, sbytes, hbytes = rows * cols // 2, rows * cols // 32 * 2, rows * cols * 2
        (d / "recipe.txt").write_text(f"size {qbytes + sbytes + hbytes}\nq4 0 {rows} {cols} 0 {qbytes}\n"
                                      f"h4 0 {rows} {cols} {qbytes + sbytes}\n")
        run("lfm2_convert", [str(d / "model.gguf"), str(d / "recipe.txt"), str(d / "out.bin")])
        out = (d / "out.bin").read_bytes()
    words = np.frombuffer(out[:qbytes], np.uint32).reshape(rows, cols // 8)
    scales = np.frombuffer(out[qbytes:qbytes + sbytes], np.float16).reshape(rows, cols // 32)
    h = np.frombuffer(out[qbytes + sbytes:qbytes + sbytes + hbytes], np.float16).reshape(rows, cols)
    return words.copy(), scales.copy(), h.copy()


def q6_k_blocks(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    """Random GGUF Q6_K rows: per 256 weights ql[128], qh[64] random bytes, int8 scales[16] over the whole range
    (incl. -128, 0, 127) and an fp16 d (incl. 0, negative, subnormal)."""
    nb = rows * cols // 256
    b = rng.integers(0, 256, (nb, 210), dtype=np.uint8)
    sc = b[:, 192:208].view(np.int8)
    sc[0, :3] = (-128, 0, 127)
    d = (np.abs(rng.standard_normal(nb)) * 0.002).astype(np.float16)
    d[0] = 0.0
    d[1] = -d[1]
    d[2] = np.float16(3e-7)
    b[:, 208:] = d.view(np.uint8).reshape(nb, 2)
    return b.reshape(rows, cols // 256 * 210)


def lfm2_q6(raw: np.ndarray, rows: int, cols: int):
    """lfm2/convert.c recipe lines `q6 <src> <rows> <cols> <out q> <out d>` and `h6 <src> <rows> <cols> <out>`."""
    with tempfile.TemporaryDirectory() as d:
        d = Path(d)
        (d / "model.gguf").write_bytes(raw.tobytes())
        nb = rows * cols // 256
        qbytes, dbytes, hbytes = nb * 208, nb * 2, rows * cols * 2
        (d / "recipe.txt").write_text(f"size {qbytes + dbytes + hbytes}\nq6 0 {rows} {cols} 0 {qbytes}\n"
                                      f"h6 0 {rows} {cols} {qbytes + dbytes}\n")
        run("lfm2_convert", [str(d / "model.gguf"), str(d / "recipe.txt"), str(d / "out.bin")])
        out = (d / "out.bin").read_bytes()
    q = np.frombuffer(out[:qbytes], np.uint8).reshape(rows, cols // 256, 208)
    dd = np.frombuffer(out[qbytes:qbytes + dbytes], np.float16).reshape(rows, cols // 256)
    h = np.frombuffer(out[qbytes + dbytes:qbytes + dbytes + hbytes], np.float16).reshape(rows, cols)
    return q.copy(), dd.copy(), h.copy()


def main(only: str | None = None):
    if only == "q6":  # the Q6_K fixture alone, from its own seed: the other fixtures stay byte for byte
        raw = q6_k_blocks(np.random.default_rng(2025), 6, 512)
        q, d, h = lfm2_q6(raw, 6, 512)
        np.savez_compressed(HERE / "ref_lfm2_q6.npz", raw=raw, q=q, d=d, h6=h)
        return 0

    rng = np.random.default_rng(2024)
    src = bf16_matrix(rng, 24, 512, 64)
    w, s = st2bin_q4(src)
    np.savez_compressed(HERE / "ref_st2bin_q4.npz", src_bf16=src, words=w, scales=s)

    out = {}
    for g in (32, 64, 128):
        src = bf16_matrix(rng, 16, 512, g)
        w, s = qwen3moe_q4(src, g)
        out[f"src_bf16_g{g}"], out[f"words_g{g}"], out[f"scales_g{g}"] = src, w, s
    np.savez_compressed(HERE / "ref_qwen3moe_q4.npz", **out)

    raw = q4_0_blocks(rng, 12, 256)
    w, s, h = lfm2_q4(raw, 12, 256)
    np.savez_compressed(HERE / "ref_lfm2_q4.npz", raw=raw, words=w, scales=s, h4=h)
    main("q6")
    for f in sorted(HERE.glob("ref_*.npz")):
        print(f.name, f.stat().st_size, "bytes")


if __name__ == "__main__":
    sys.exit(main(sys.argv[1] if len(sys.argv) > 1 else None))
