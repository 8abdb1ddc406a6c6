"""ctypes binding of libaq.so, the C ABI declared in include/aq.h.

The library is built in-tree (``mojo-adreno_amd/build.py``) and loaded from this directory. There is no fallback: if
it is missing, every op raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

_HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("AQ_LIB", _HERE / "libaq.so"))

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64

# name -> argument types (all return int status). Kept in the order of include/aq.h.
SIGNATURES: dict[str, list] = {
    "aq_version": [],
    "aq_gemv_q4": [_p, _p, _p, _p, _i64, _i64, _i32, _i32, _i32, _p],
    "aq_gate_up_q4": [_p, _p, _p, _p, _i64, _i64, _i32, _i32, _p],
    "aq_gemm_q4": [_p, _i32, _p, _p, _p, _i64, _i64, _i64, _i32, _i32, _p, _i64, _p],
    "aq_gemm_q4_workspace_bytes": [_i64, _i64, _i64],
    "aq_gemm_q4_noalloc": [_p, _i32, _p, _p, _p, _i64, _i64, _i64, _i32, _i32, _p],
    "aq_gemm_t2": [_p, _i32, _p, _p, _p, _i64, _i64, _i64, _i32, _p, _i64, _p],
    "aq_gemm_t2_workspace_bytes": [_i64, _i64, _i64],
    "aq_moe_gemm_q4": [_p, _i32, _i64, _p, _p, _p, _i64, _i64, _i64, _i32, _p, _p, _i32, _i32, _i64, _i32, _p, _p],
    "aq_moe_route": [_p, _p, _p, _i64, _i32, _i32, _p],
    "aq_moe_route_pack": [_p, _p, _p, _i64, _i32, _i32, _p, _p, _i64, _p],
    "aq_moe_group": [_p, _i64, _i32, _i32, _i32, _p, _p, _p, _p, _i64, _p, _i32, _p, _p],
    "aq_moe_group_max_rows": [_i64, _i32, _i32, _i32],
    "aq_moe_group_max_tiles": [_i64, _i32, _i32, _i32],
    "aq_moe_expert_lists": [_p, _i64, _i32, _i32, _i32, _p, _p, _i32, _p, _i32, _p, _p, _i64, _p],
    "aq_moe_combine": [_p, _i64, _p, _p, _p, _i64, _i64, _i32, _i32, _p],
    "aq_moe_gate_up_q4": [_p, _p, _i64, _p, _p, _p, _i64, _i64, _i32, _i32, _p],
    "aq_moe_down_q4": [_p, _p, _i64, _p, _p, _p, _p, _i64, _i64, _i32, _i32, _i32, _p],
    "aq_gemv_f32": [_p, _p, _p, _i64, _i64, _i32, _p],
    "aq_t2_gemv": [_p, _p, _p, _p, _i64, _i64, _p, _i64, _p],
    "aq_t2_gemv_workspace_bytes": [_i64, _i64],
    "aq_t2_head_argmax": [_p, _p, _p, _p, _i64, _i64, _p, _i64, _p, _p, _p, _i32, _i32, _p],
    "aq_t2_head_candidates": [_i64, _i64],
    "aq_gemv_q6": [_p, _p, _p, _p, _i64, _i64, _p],
    "aq_head_argmax_q6": [_p, _p, _p, _p, ctypes.c_float, _p, _i64, _i64, _p, _i64, _p, _p, _p, _i32, _i32, _p],
    "aq_head_q6_candidates": [_i64, _i64],
    "aq_embed_q6": [_p, _p, _i64, _i64, _p, _i32, _p, _p],
    "aq_stream_read": [_p, _i64, _i32, _p, _p],
    "aq_t2_packed_linear": [_p, _p, _p, _p, _i64, _i64, _p],
    "aq_t2_packed_reduce": [_p, _p, _i64, _i32, _p],
    "aq_pack_half": [_p, _p, _i64, _p],
    "aq_rmsnorm_pack": [_p, _p, _p, _i64, _i64, ctypes.c_float, _p],
    "aq_swiglu_pack": [_p, _p, _i64, _i64, _p],
    "aq_rmsnorm_gemv_q4": [_p, _p, _p, _p, ctypes.c_float, _p, _i64, _i64, _i32, _i32, _p],
    "aq_rmsnorm_gate_up_q4": [_p, _p, _p, _p, ctypes.c_float, _p, _i64, _i64, _i32, _i32, _p],
    "aq_embed_f16": [_p, _i64, _i64, _p, _p, _p],
    "aq_attn_decode": [_p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _p, _p],
    "aq_attn_decode_split": [_p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _p, _p],
    "aq_attn_out_q4": [_p, _p, _p, _i32, _p, _i64, _i64, _i32, _p],
    "aq_head_argmax_q4": [_p, _p, _p, _p, ctypes.c_float, _p, _i64, _i64, _i32, _p, _i64, _p, _p, _p, _i32, _i32,
                          _p],
    "aq_quantize_q4": [_p, _i32, _i64, _i64, _i32, _p, _p],
    "aq_quantize_q4_searched": [_p, _i64, _i64, _i32, _p, _p],
    "aq_gguf_q4_0_to_q4w": [_p, _i64, _i64, _p, _p],
    "aq_gguf_q4_0_to_f16": [_p, _i64, _i64, _p],
    "aq_gguf_q6_k_to_q6w": [_p, _i64, _i64, _p, _p],
    "aq_t2w_scales_from_pairs": [_p, _i64, _i64, _p],
    "aq_gguf_q6_k_to_f16": [_p, _i64, _i64, _p],
    "aq_t2w_from_mlx": [_p, _p, _p, _p, _i32, _i64, _p, _p],
}
RESTYPES = {"aq_gemm_q4_workspace_bytes": ctypes.c_int64, "aq_t2_gemv_workspace_bytes": ctypes.c_int64,
            "aq_t2_head_candidates": ctypes.c_int64, "aq_head_q6_candidates": ctypes.c_int64,
            "aq_gemm_t2_workspace_bytes": ctypes.c_int64, "aq_moe_group_max_rows": ctypes.c_int64,
            "aq_moe_group_max_tiles": ctypes.c_int32}

_lib = None


class AqError(RuntimeError):
    """A non-zero aq_status from the C ABI."""

    def __init__(self, fn: str, status: int):
        self.status = status
        super().__init__(f"{fn}: {status_string(status)} (status {status})")


def lib() -> ctypes.CDLL:
    """Load libaq.so once (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python mojo-adreno_amd/build.py`")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, args in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = RESTYPES.get(name, ctypes.c_int)
        handle.aq_status_string.argtypes = [ctypes.c_int]
        handle.aq_status_string.restype = ctypes.c_char_p
        _lib = handle
    return _lib


def status_string(status: int) -> str:
    return lib().aq_status_string(int(status)).decode()


def call(name: str, *args) -> None:
    """Call an entry point and raise AqError on a non-zero status."""
    st = getattr(lib(), name)(*args)
    if st != 0:
        raise AqError(name, st)
