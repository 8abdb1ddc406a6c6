"""Weight-format converters on host arrays: the producers of the Q4W and T2W layouts the kernels consume.

Thin numpy wrappers over libaq's host entry points (include/aq.h, csrc/aq_convert.cpp), which write the reference
converters' bytes:

  quantize_q4           llama/run.py:56-70 quantize4 (fp16 weights) / llama/st2bin.c "q4" (bf16 weights)
  quantize_q4_searched  qwen3moe/convert.c:120-159 "q4" (least-squared-error scale over d = 6.5 .. 9)
  gguf_q4_0_to_q4w      lfm2/convert.c:59-71 (GGUF Q4_0 -> Q4W words + fp16 scales, G = 32)
  gguf_q4_0_to_f16      lfm2/convert.c:73-80 "h4" (GGUF Q4_0 -> fp16)
  gguf_q6_k_to_q6w      lfm2/convert.c:148-155 "q6" (GGUF Q6_K -> 208-byte super-blocks + fp16 d apart)
  gguf_q6_k_to_f16      lfm2/convert.c:82-103 "h6" (GGUF Q6_K -> fp16)
  t2w_scales_from_pairs bonsai/convert.cpp:44-61 emitPacked ((scale, bias) fp32 pairs -> T2W fp16 scales)
  t2w_from_mlx          qwen3/convert.cpp:39-74 addPacked (MLX 2-bit projections -> one transposed T2W matrix)

Inputs are numpy arrays; bf16 weights are passed as their uint16 bit patterns (numpy has no bf16 type).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib


def _ptr(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)


def quantize_q4(w: np.ndarray, group: int = 64, bf16: bool = False):
    """Q4W words [rows, cols/8] and fp16 scales [rows, cols/group] of fp16 weights, or of bf16 bit patterns
    (uint16, ``bf16=True``) each rounded to fp16 first as llama/st2bin.c does."""
    if bf16:
        src = np.ascontiguousarray(w, dtype=np.uint16)
    else:
        src = np.ascontiguousarray(np.asarray(w, dtype=np.float16)).view(np.uint16)
    rows, cols = src.shape
    wq = np.empty((rows, cols // 8), np.uint32)
    ws = np.empty((rows, cols // group), np.float16)
    _lib.call("aq_quantize_q4", _ptr(src), int(bf16), rows, cols, group, _ptr(wq), _ptr(ws))
    return wq, ws


def quantize_q4_searched(w_bf16: np.ndarray, group: int):
    """Q4W words and fp16 scales of bf16 weights (uint16 bit patterns) with the searched scale."""
    src = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    rows, cols = src.shape
    wq = np.empty((rows, cols // 8), np.uint32)
    ws = np.empty((rows, cols // group), np.float16)
    _lib.call("aq_quantize_q4_searched", _ptr(src), rows, cols, group, _ptr(wq), _ptr(ws))
    return wq, ws


def gguf_q4_0_to_q4w(blocks, rows: int, cols: int):
    """GGUF Q4_0 rows (rows * cols / 32 blocks of 18 bytes) -> Q4W words [rows, cols/8], fp16 scales [rows, cols/32]."""
    src = np.ascontiguousarray(np.frombuffer(bytes(blocks), np.uint8) if not isinstance(blocks, np.ndarray)
                               else blocks.view(np.uint8).reshape(-1))
    if src.size != rows * cols // 32 * 18:
        raise ValueError("Q4_0 data size does not match rows x cols")
    wq = np.empty((rows, cols // 8), np.uint32)
    ws = np.empty((rows, cols // 32), np.float16)
    _lib.call("aq_gguf_q4_0_to_q4w", _ptr(src), rows, cols, _ptr(wq), _ptr(ws))
    return wq, ws


def gguf_q4_0_to_f16(blocks, rows: int, cols: int) -> np.ndarray:
    """GGUF Q4_0 rows -> fp16 [rows, cols] ((nib - 8) * d in fp32, rounded)."""
    src = np.ascontiguousarray(np.frombuffer(bytes(blocks), np.uint8) if not isinstance(blocks, np.ndarray)
                               else blocks.view(np.uint8).reshape(-1))
    if src.size != rows * cols // 32 * 18:
        raise ValueError("Q4_0 data size does not match rows x cols")
    out = np.empty((rows, cols), np.float16)
    _lib.call("aq_gguf_q4_0_to_f16", _ptr(src), rows, cols, _ptr(out))
    return out


def _q6_k_src(blocks, rows: int, cols: int) -> np.ndarray:
    src = np.ascontiguousarray(np.frombuffer(bytes(blocks), np.uint8) if not isinstance(blocks, np.ndarray)
                               else blocks.view(np.uint8).reshape(-1))
    if cols % 256 or src.size != rows * cols // 256 * 210:
        raise ValueError("Q6_K data size does not match rows x cols (cols % 256 == 0, 210 bytes per 256 weights)")
    return src


def gguf_q6_k_to_q6w(blocks, rows: int, cols: int):
    """GGUF Q6_K rows (rows * cols / 256 super-blocks of 210 bytes) -> Q6W: q uint8 [rows, cols/256, 208] and
    d fp16 [rows, cols/256]."""
    src = _q6_k_src(blocks, rows, cols)
    q = np.empty((rows, cols // 256, 208), np.uint8)
    d = np.empty((rows, cols // 256), np.float16)
    _lib.call("aq_gguf_q6_k_to_q6w", _ptr(src), rows, cols, _ptr(q), _ptr(d))
    return q, d


def gguf_q6_k_to_f16(blocks, rows: int, cols: int) -> np.ndarray:
    """GGUF Q6_K rows -> fp16 [rows, cols] ((d * sc) * (q - 32) in fp32, rounded)."""
    src = _q6_k_src(blocks, rows, cols)
    out = np.empty((rows, cols), np.float16)
    _lib.call("aq_gguf_q6_k_to_f16", _ptr(src), rows, cols, _ptr(out))
    return out


def t2w_scales_from_pairs(params: np.ndarray) -> np.ndarray:
    """bonsai/convert.cpp's (scale, bias) pairs fp32 [K/128, N, 2] -> T2W scales fp16 [K/128, N]. Raises AqError if a
    group is not ternary (bias != -scale) or a scale is not exact in fp16."""
    src = np.ascontiguousarray(params, np.float32)
    if src.ndim != 3 or src.shape[2] != 2:
        raise ValueError("params must be [K/128, N, 2]")
    out = np.empty(src.shape[:2], np.float16)
    _lib.call("aq_t2w_scales_from_pairs", _ptr(src), src.shape[0], src.shape[1], _ptr(out))
    return out


def t2w_from_mlx(parts, k: int):
    """MLX 2-bit projections [(codes uint32 [n_i, K/16], scales fp16 [n_i, K/128], biases fp16 [n_i, K/128]), ...]
    -> (w uint32 [K/16, sum n_i], s fp16 [K/128, sum n_i]). Raises AqError if a group is not ternary."""
    arrs = [(np.ascontiguousarray(c, np.uint32), np.ascontiguousarray(np.asarray(s, np.float16)).view(np.uint16),
             np.ascontiguousarray(np.asarray(b, np.float16)).view(np.uint16)) for c, s, b in parts]
    n = len(arrs)
    rows = np.array([a[0].shape[0] for a in arrs], np.int64)
    codes = (ctypes.c_void_p * n)(*[a[0].ctypes.data for a in arrs])
    scales = (ctypes.c_void_p * n)(*[a[1].ctypes.data for a in arrs])
    biases = (ctypes.c_void_p * n)(*[a[2].ctypes.data for a in arrs])
    total = int(rows.sum())
    w = np.empty((k // 16, total), np.uint32)
    s = np.empty((k // 128, total), np.float16)
    _lib.call("aq_t2w_from_mlx", ctypes.cast(codes, ctypes.c_void_p), ctypes.cast(scales, ctypes.c_void_p),
              ctypes.cast(biases, ctypes.c_void_p), _ptr(rows), n, k, _ptr(w), _ptr(s))
    return w, s
