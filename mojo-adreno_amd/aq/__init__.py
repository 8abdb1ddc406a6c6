"""aq: MI355X-native weight-quantized matmul (int4 Q4W / ternary T2W GEMV and GEMM, grouped MoE) for gfx950.

The kernels are HIP, built into ``libaq.so`` next to this file and reached through its C ABI (``include/aq.h``).
Importing the package registers them as ``torch.ops.aq.*`` custom ops (``aq.ops``); ``aq.moe`` is the host plan of a
mixture-of-experts block.
"""
from . import _lib  # noqa: F401
from ._lib import AqError, LIB_PATH, lib  # noqa: F401
from . import ops  # noqa: F401  (registers torch.ops.aq.*)

__all__ = ["AqError", "LIB_PATH", "lib", "ops", "moe", "synth"]


def __getattr__(name):
    if name in ("moe", "synth", "formats"):
        import importlib
        return importlib.import_module(f"{__name__}.{name}")
    raise AttributeError(name)
