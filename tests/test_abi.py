"""The C ABI library loads on a CPU-only host, exports every symbol include/aq.h declares, and rejects bad
arguments before touching the GPU (no compute calls here)."""
import ctypes
import re

import pytest

from conftest import ROOT


def _declared():
    text = (ROOT / "include" / "aq.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+char\s*\*|int)\s+(aq_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    import aq
    lib = aq.lib()
    names = _declared()
    assert "aq_gemv_q4" in names and len(names) >= 4
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared in include/aq.h but not exported: {missing}"


def test_bindings_cover_every_declared_symbol():
    from aq import _lib
    names = set(_declared()) - {"aq_status_string"}
    assert names <= set(_lib.SIGNATURES), f"no ctypes signature for {sorted(names - set(_lib.SIGNATURES))}"


def test_status_strings():
    from aq import _lib
    assert _lib.status_string(0) == "ok"
    assert "misaligned" in _lib.status_string(3)
    assert "unknown" in _lib.status_string(999)


def test_version():
    import aq
    assert aq.lib().aq_version() >= 100


@pytest.mark.parametrize("args,status", [
    ((None, None, None, None, 8, 512, 32, 1, 0, None), 5),  # NULL pointers
])
def test_gemv_rejects_null(args, status):
    import aq
    assert aq.lib().aq_gemv_q4(*args) == status


def test_gemv_rejects_bad_shapes_before_launch():
    import aq
    lib = aq.lib()
    buf = ctypes.create_string_buffer(4096 + 16)
    p = (ctypes.addressof(buf) + 15) & ~15  # host memory: never dereferenced, every call must fail first
    assert lib.aq_gemv_q4(p, p, p, p, 8, 500, 32, 1, 0, None) == 1      # K % 32 != 0
    assert lib.aq_gemv_q4(p, p, p, p, 8, 512, 12, 1, 0, None) == 2      # group % 8 != 0
    assert lib.aq_gemv_q4(p, p, p, p, 8, 512, 48, 1, 0, None) == 2      # K % group != 0
    assert lib.aq_gemv_q4(p, p, p, p, 8, 512, 32, 17, 0, None) == 1     # tokens > 16
    assert lib.aq_gemv_q4(p, p, p, p, 8, 4096, 32, 9, 0, None) == 6     # 16 rows of x staging exceed LDS
    assert lib.aq_gate_up_q4(p, p, p, p, 8, 512, 32, 9, None) == 1      # gate|up: at most 8 tokens
    assert lib.aq_gemv_q4(p, p, p, p, 0, 512, 32, 1, 0, None) == 1      # N == 0
    assert lib.aq_gemv_q4(p, p, p, p, 8, 32768, 32, 2, 0, None) == 6    # x staging exceeds LDS
    assert lib.aq_gemv_q4(p + 4, p, p, p, 8, 512, 32, 1, 0, None) == 3  # misaligned words
    assert lib.aq_gate_up_q4(p, p, p, p, 8, 500, 32, 1, None) == 1


def test_torch_ops_registered():
    import torch
    from aq import ops  # noqa: F401
    for name in ("gemv_q4", "gate_up_q4"):
        assert hasattr(torch.ops.aq, name)


def test_ops_reject_host_tensors():
    """No CPU fallback: host tensors are refused before any kernel call."""
    import torch
    from aq import ops
    wq = torch.zeros((8, 64), dtype=torch.int32)
    with pytest.raises((ValueError, NotImplementedError, RuntimeError)):
        ops.gemv_q4(wq, torch.zeros((8, 16), dtype=torch.float16), torch.zeros(512), torch.zeros(8), 32)


def test_decode_entries_reject_bad_arguments_before_launch():
    import aq
    lib = aq.lib()
    buf = ctypes.create_string_buffer(4096 + 16)
    p = (ctypes.addressof(buf) + 15) & ~15  # host memory: never dereferenced, every call must fail first
    f = ctypes.c_float(1e-5)
    assert lib.aq_rmsnorm_gemv_q4(p, p, p, None, f, p, 8, 512, 32, 1, None) == 5        # no norm weights
    assert lib.aq_rmsnorm_gemv_q4(p, p, p, p + 2, f, p, 8, 512, 32, 1, None) == 3       # misaligned norm weights
    assert lib.aq_rmsnorm_gate_up_q4(p, p, p, p, f, p, 8, 500, 32, 1, None) == 1        # K % 32
    assert lib.aq_embed_f16(p, 100, 12, p, p, None) == 1                                 # d % 8
    assert lib.aq_embed_f16(None, 100, 16, p, p, None) == 5
    assert lib.aq_attn_decode(p, p, p, p, p, p, 32, 8, 128, 512, p, None) == 1          # head_dim != 64
    assert lib.aq_attn_decode(p, p, p, p, p, p, 32, 6, 64, 512, p, None) == 1           # heads % kv_heads
    assert lib.aq_attn_decode(p, p, p, p, p, p, 48, 3, 64, 512, p, None) == 1           # 16 heads per KV head
    assert lib.aq_attn_decode(p, p, p, p, p, p, 32, 4, 64, 8192, p, None) == 6          # scores exceed LDS
    assert lib.aq_attn_decode(p, p, p, None, p, p, 32, 8, 64, 512, p, None) == 5
    # lm_head: 128256 rows need 4 * 1024 argmax candidates; the position pointer is required
    assert lib.aq_head_argmax_q4(p, p, p, None, f, p, 128256, 2048, 32, p, 1000, p, p, None, 0, 1, None) == 6
    assert lib.aq_head_argmax_q4(p, p, p, None, f, p, 1000, 2048, 32, p, 4096, p, None, None, 0, 1, None) == 5
    assert lib.aq_head_argmax_q4(p, p, p, None, f, p, 1000, 2048, 32, p + 4, 4096, p, p, None, 0, 1, None) == 3


def test_decode_ops_registered():
    import torch
    from aq import ops  # noqa: F401
    for name in ("rmsnorm_gemv_q4", "rmsnorm_gate_up_q4", "embed_f16", "attn_decode", "head_argmax_q4"):
        assert hasattr(torch.ops.aq, name)


def test_t2_head_argmax_validation():
    import aq
    lib = aq.lib()
    buf = ctypes.create_string_buffer(4096 + 16)
    p = (ctypes.addressof(buf) + 15) & ~15  # host memory: never dereferenced, every call must fail first
    # one argmax key per workgroup: 256 columns each when N % 4 == 0 gives >= 512 workgroups (K <= 16384), else 32
    # once that gives >= 256 workgroups, else 16
    assert lib.aq_t2_head_candidates(248320, 2048) == 970
    assert lib.aq_t2_head_candidates(248320, 32768) == 7760
    assert lib.aq_t2_head_candidates(151669, 2048) == 4740
    assert lib.aq_t2_head_candidates(8000, 1024) == 500
    assert lib.aq_t2_head_candidates(8192, 512) == 256
    assert lib.aq_t2_head_candidates(7, 128) == 1
    assert lib.aq_t2_head_candidates(0, 128) == 0
    assert lib.aq_t2_head_argmax(p, p, p, p, 8000, 1024, p, 499, p, p, None, 0, 1, None) == 6   # too few keys
    assert lib.aq_t2_head_argmax(p, p, p, p, 8000, 1024, p, 500, p, None, None, 0, 1, None) == 5  # no pos
    assert lib.aq_t2_head_argmax(p, p, p, p, 8000, 1024, p + 4, 500, p, p, None, 0, 1, None) == 3  # misaligned keys
    assert lib.aq_t2_head_argmax(p, p, p, p, 8000, 1000, p, 500, p, p, None, 0, 1, None) == 1     # K % 128
    assert lib.aq_t2_head_argmax(p, p, p, None, 8000, 1024, p, 500, p, p, None, 0, 1, None) == 5  # no logits


def test_q6_validation():
    import aq
    lib = aq.lib()
    buf = ctypes.create_string_buffer(4096 + 16)
    p = (ctypes.addressof(buf) + 15) & ~15  # host memory: never dereferenced, every call must fail first
    f = ctypes.c_float(1e-5)
    # one argmax key per wave, at most 3072 waves: 65536 rows x 2048 (2 rows a wave step) -> 3072; 7 rows x 256
    # (16 a step) -> 4
    assert lib.aq_head_q6_candidates(65536, 2048) == 3072
    assert lib.aq_head_q6_candidates(7, 256) == 4
    assert lib.aq_head_q6_candidates(1000, 5120) == 1000
    assert lib.aq_head_q6_candidates(10, 100) == 0
    assert lib.aq_gemv_q6(p, p, p, p, 100, 1000, None) == 1              # cols % 256
    assert lib.aq_gemv_q6(p + 8, p, p, p, 100, 2048, None) == 3          # q not 16-byte aligned
    assert lib.aq_gemv_q6(p, p, None, p, 100, 2048, None) == 5
    assert lib.aq_gemv_q6(p, p, p, p, 1 << 24, 2048, None) == 6          # q beyond 2 GiB
    assert lib.aq_head_argmax_q6(p, p, p, None, f, p, 65536, 2048, p, 3071, p, p, None, 0, 1, None) == 6
    assert lib.aq_head_argmax_q6(p, p, p, None, f, p, 65536, 2048, p + 4, 4096, p, p, None, 0, 1, None) == 3
    assert lib.aq_head_argmax_q6(p, p, p, None, f, p, 65536, 2048, p, 4096, p, None, None, 0, 1, None) == 5
    assert lib.aq_embed_q6(p, p, 100, 2048, p, 0, p, None) == 1            # no tokens
    assert lib.aq_embed_q6(p, p, 100, 2048, None, 1, p, None) == 5


def test_moe_route_pack_validation():
    import aq
    lib = aq.lib()
    buf = ctypes.create_string_buffer(4096 + 16)
    p = (ctypes.addressof(buf) + 15) & ~15  # host memory: never dereferenced, every call must fail first
    assert lib.aq_moe_route_pack(p, p, p, 4, 128, 8, None, p, 2048, None) == 5    # no x
    assert lib.aq_moe_route_pack(p, p, p, 4, 128, 8, p, p, 2044, None) == 1       # d % 8
    assert lib.aq_moe_route_pack(p, p, p, 4, 300, 8, p, p, 2048, None) == 1       # experts > 256
    assert lib.aq_moe_route_pack(p, p, p, 4, 128, 8, p + 4, p, 2048, None) == 3   # x not 16-byte aligned
