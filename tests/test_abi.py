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


def test_python_constants_match_the_header():
    """The limits aq.ops mirrors are the header's #defines."""
    from aq import ops
    text = (ROOT / "include" / "aq.h").read_text()
    defs = dict(re.findall(r"^#define AQ_(\w+) (\d+)\s*$", text, flags=re.M))
    for name in ("HEAD_CANDIDATES", "HEAD_ARRIVAL_SLOTS", "ATTN_MAX_SPLITS", "STREAM_READ_MAX_BLOCKS"):
        assert int(defs[name]) == getattr(ops, name), name


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
    # lm_head: 128256 rows take 1024 workgroups, so 1024 argmax keys and the arrival counters' 17 slots; the position
    # pointer is required
    assert lib.aq_head_argmax_q4(p, p, p, None, f, p, 128256, 2048, 32, p, 1000, p, p, None, 0, 1, None) == 6
    assert lib.aq_head_argmax_q4(p, p, p, None, f, p, 128256, 2048, 32, p, 1024 + 16, p, p, None, 0, 1, None) == 6
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
    # one argmax key per workgroup (256 columns each when N % 4 == 0 gives >= 512 workgroups (K <= 16384), else 32
    # once that gives >= 256 workgroups, else 16), then 17 arrival counter slots
    assert lib.aq_t2_head_candidates(248320, 2048) == 970 + 17
    assert lib.aq_t2_head_candidates(248320, 32768) == 7760 + 17
    assert lib.aq_t2_head_candidates(151669, 2048) == 4740 + 17
    assert lib.aq_t2_head_candidates(8000, 1024) == 500 + 17
    assert lib.aq_t2_head_candidates(8192, 512) == 256 + 17
    assert lib.aq_t2_head_candidates(7, 128) == 1 + 17
    assert lib.aq_t2_head_candidates(0, 128) == 0
    assert lib.aq_t2_head_argmax(p, p, p, p, 8000, 1024, p, 516, p, p, None, 0, 1, None) == 6   # too few slots
    assert lib.aq_t2_head_argmax(p, p, p, p, 8000, 1024, p, 517, p, None, None, 0, 1, None) == 5  # no pos
    assert lib.aq_t2_head_argmax(p, p, p, p, 8000, 1024, p + 4, 517, p, p, None, 0, 1, None) == 3  # misaligned keys
    assert lib.aq_t2_head_argmax(p, p, p, p, 8000, 1000, p, 500, p, p, None, 0, 1, None) == 1     # K % 128
    assert lib.aq_t2_head_argmax(p, p, p, None, 8000, 1024, p, 500, p, p, None, 0, 1, None) == 5  # no logits


def test_q6_validation():
    import aq
    lib = aq.lib()
    buf = ctypes.create_string_buffer(4096 + 16)
    p = (ctypes.addressof(buf) + 15) & ~15  # host memory: never dereferenced, every call must fail first
    f = ctypes.c_float(1e-5)
    # one argmax key per workgroup of 4 waves, at most 3072 waves: 65536 rows x 2048 (2 rows a wave step) -> 768
    # workgroups; 7 rows x 256 (16 a step) -> 1; then 17 arrival counter slots
    assert lib.aq_head_q6_candidates(65536, 2048) == 3072 // 4 + 17
    assert lib.aq_head_q6_candidates(7, 256) == 1 + 17
    assert lib.aq_head_q6_candidates(1000, 5120) == 1000 // 4 + 17
    assert lib.aq_head_q6_candidates(10, 100) == 0
    assert lib.aq_gemv_q6(p, p, p, p, 100, 1000, None) == 1              # cols % 256
    assert lib.aq_gemv_q6(p + 8, p, p, p, 100, 2048, None) == 3          # q not 16-byte aligned
    assert lib.aq_gemv_q6(p, p, None, p, 100, 2048, None) == 5
    assert lib.aq_gemv_q6(p, p, p, p, 1 << 24, 2048, None) == 6          # q beyond 2 GiB
    assert lib.aq_head_argmax_q6(p, p, p, None, f, p, 65536, 2048, p, 768 + 16, p, p, None, 0, 1, None) == 6
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


def test_operand_size_guards():
    """Operands addressed through one 32-bit buffer range are refused (AQ_ERR_CAPACITY) at 2 GiB and above."""
    import aq
    lib = aq.lib()
    buf = ctypes.create_string_buffer(4096 + 16)
    p = (ctypes.addressof(buf) + 15) & ~15  # host memory: never dereferenced, every call must fail first
    # MoE decode gate|up: the stacked experts' rows, experts * 2f * K/2 bytes
    assert lib.aq_moe_gate_up_q4(p, p, 1024, p, p, p, 1024, 2048, 32, 8, None) == 6   # exactly 2 GiB
    assert lib.aq_moe_gate_up_q4(p, p, 1023, p, p, p, 1024, 2048, 32, 8, None) != 6   # just below (fails later)
    assert lib.aq_moe_down_q4(p, p, 1024, p, p, p, p, 2048, 2048, 32, 8, 0, None) == 6
    # dense GEMM: Y (and each split's partial slab) is M x N floats
    assert lib.aq_gemm_q4(p, 0, p, p, p, 4096, 131072, 128, 32, 0, None, 0, None) == 6
    assert lib.aq_gemm_t2(p, 0, p, p, p, 4096, 131072, 128, 0, None, 0, None) == 6
    assert lib.aq_gemm_q4(p, 0, p, p, p, 4095, 131072, 128, 32, 0, None, 0, None) != 6


def _moe_decode_tensors(experts=4, f=64, d=64, k=64, topk=2, group=32):
    import torch
    i32 = torch.int32
    return dict(
        gu_q=torch.zeros((experts * 2 * f, k // 8), dtype=i32), gu_s=torch.zeros((experts * 2 * f, k // group),
                                                                                  dtype=torch.float16),
        dn_q=torch.zeros((experts * d, f // 8), dtype=i32), dn_s=torch.zeros((experts * d, f // group),
                                                                             dtype=torch.float16),
        ids=torch.zeros(topk, dtype=i32), w=torch.zeros(topk), x=torch.zeros(k), a=torch.zeros((topk, f)),
        y=torch.zeros(d), experts=experts, group=group)


def _raises(fn, match):
    with pytest.raises(ValueError, match=match):
        fn()


def test_moe_decode_ops_validate_shapes_before_launch():
    """The MoE decode wrappers check every shape and dtype before any launch: mis-sized outputs are refused on the host
    (with host tensors the checks pass only to stop at the device check)."""
    import torch
    from aq import ops
    t = _moe_decode_tensors()
    gu = lambda **o: (lambda: ops._moe_gate_up_q4_impl(o.get("wq", t["gu_q"]), o.get("ws", t["gu_s"]), t["experts"],
                                                        o.get("ids", t["ids"]), o.get("x", t["x"]), o.get("a", t["a"]),
                                                        t["group"]))
    _raises(gu(), "device")
    _raises(gu(a=torch.zeros((2, 65))), "a must be")
    _raises(gu(a=torch.zeros((2, 64), dtype=torch.float16)), "a must be")
    _raises(gu(x=torch.zeros(63)), "x must be")
    _raises(gu(ws=torch.zeros((4 * 128, 1), dtype=torch.float16)), "ws must be")
    _raises(gu(wq=torch.zeros((4 * 128 + 2, 8), dtype=torch.int32)), "wq must be")
    _raises(gu(ids=torch.zeros(2, dtype=torch.int64)), "int32")
    dn = lambda **o: (lambda: ops._moe_down_q4_impl(o.get("wq", t["dn_q"]), o.get("ws", t["dn_s"]), t["experts"],
                                                     o.get("ids", t["ids"]), o.get("w", t["w"]), o.get("a", t["a"]),
                                                     o.get("y", t["y"]), t["group"], False))
    _raises(dn(), "device")
    _raises(dn(y=torch.zeros(65)), "y must be")
    _raises(dn(a=torch.zeros((3, 64))), "a must be")
    _raises(dn(w=torch.zeros(3)), "weights must be")
    _raises(dn(ws=torch.zeros((256, 3), dtype=torch.float16)), "ws must be")


def test_moe_combine_and_gemm_validate_shapes_before_launch():
    import torch
    from aq import ops
    yd, slot, w, y = torch.zeros((16, 32)), torch.zeros(8, dtype=torch.int32), torch.zeros((4, 2)), torch.zeros((4, 32))
    cb = lambda **o: (lambda: ops._moe_combine_impl(o.get("yd", yd), o.get("slot", slot), o.get("w", w),
                                                    o.get("y", y), False))
    _raises(cb(), "device")
    _raises(cb(y=torch.zeros((5, 32))), "y must be")
    _raises(cb(yd=torch.zeros((16, 36))), "yd must be")
    _raises(cb(slot=torch.zeros(7, dtype=torch.int32)), "slot must")
    _raises(cb(w=torch.zeros(8)), "weights must be")
    x = torch.zeros((4, 64), dtype=torch.float16)
    wq, ws = torch.zeros((2 * 32, 8), dtype=torch.int32), torch.zeros((2 * 32, 2), dtype=torch.float16)
    tiles, nt, out = torch.zeros(8, dtype=torch.int32), torch.zeros(1, dtype=torch.int32), torch.zeros((48, 32))
    gm = lambda **o: (lambda: ops._moe_gemm_q4_impl(x, torch.zeros(0, dtype=torch.int32), wq, o.get("ws", ws), 2, 32,
                                                    tiles, nt, 16, False, o.get("out", out)))
    _raises(gm(), "device")
    _raises(gm(ws=torch.zeros((64, 1), dtype=torch.float16)), "ws must be")
    _raises(gm(out=torch.zeros((48, 31))), "out must be")


def test_gemm_noalloc_refuses_partials_beyond_its_array():
    """aq_gemm_q4_noalloc keeps split-K partials in a static 32 MiB array per GPU: a shape needing more is refused with
    AQ_ERR_CAPACITY before any device call."""
    import aq
    lib = aq.lib()
    buf = ctypes.create_string_buffer(4096 + 16)
    p = (ctypes.addressof(buf) + 15) & ~15  # host memory: never dereferenced, every call must fail first
    assert lib.aq_gemm_q4_workspace_bytes(1120, 4096, 8192) > (32 << 20)
    assert lib.aq_gemm_q4_noalloc(p, 0, p, p, p, 1120, 4096, 8192, 32, 0, None) == 6
    assert lib.aq_gemm_q4_noalloc(p, 0, p, p, p, 431, 2048, 8016, 32, 0, None) == 1   # K % 32
    assert lib.aq_gemm_q4_noalloc(p + 4, 0, p, p, p, 431, 2048, 8192, 32, 0, None) == 3


def test_stream_read_rejects_bad_arguments_before_launch():
    import aq
    lib = aq.lib()
    buf = ctypes.create_string_buffer(4096 + 16)
    p = (ctypes.addressof(buf) + 15) & ~15  # host memory: never dereferenced, every call must fail first
    assert lib.aq_stream_read(None, 4096, 0, p, None) == 5
    assert lib.aq_stream_read(p, 4100, 0, p, None) == 1          # not whole 16-byte vectors
    assert lib.aq_stream_read(p, 0, 0, p, None) == 1
    assert lib.aq_stream_read(p, 1 << 31, 0, p, None) == 6      # 32-bit offsets
    assert lib.aq_stream_read(p, 4096, 8193, p, None) == 7      # beyond AQ_STREAM_READ_MAX_BLOCKS
    assert lib.aq_stream_read(p + 4, 4096, 0, p, None) == 3
