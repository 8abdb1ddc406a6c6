"""aq_gemm_q4_noalloc, the allocation-free variant of aq_gemm_q4, through the C ABI: its split-K partials live in the
library's static per-GPU array, so it takes no workspace and allocates nothing. Its output must equal aq_gemm_q4's
(given a workspace) bit for bit, call after call, including a second, smaller call right after a larger one (the
array keeps the last call's contents)."""
import ctypes

import numpy as np
import pytest

from _util import to_dev, to_np

pytestmark = pytest.mark.gpu


def _gemm_pair(dev, lib, m, n, k, group, add, x_f32, seed):
    """(noalloc output, workspace output) of one shape, both from the same inputs (and the same y when add)."""
    import torch
    from aq import synth
    rng = np.random.default_rng(seed)
    wq, ws = synth.int4_matrix(rng, n, k, group)
    x = rng.standard_normal((m, k)).astype(np.float32 if x_f32 else np.float16)
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    wq_d, ws_d, x_d = to_dev(wq, dev), to_dev(ws, dev), to_dev(x, dev)
    ya, yb = to_dev(y0, dev), to_dev(y0, dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    st = lib.aq_gemm_q4_noalloc(x_d.data_ptr(), int(x_f32), wq_d.data_ptr(), ws_d.data_ptr(), ya.data_ptr(), m, n, k,
                                group, int(add), stream)
    assert st == 0, st
    wsb = lib.aq_gemm_q4_workspace_bytes(m, n, k)
    work = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)
    st = lib.aq_gemm_q4(x_d.data_ptr(), int(x_f32), wq_d.data_ptr(), ws_d.data_ptr(), yb.data_ptr(), m, n, k, group,
                        int(add), work.data_ptr(), wsb, stream)
    assert st == 0, st
    torch.cuda.synchronize(dev)
    return to_np(ya), to_np(yb), wsb


# C1's down projection (4 K splits, 14 MB of partials), then smaller split shapes; fp32 X takes the general kernel
@pytest.mark.parametrize("first,second", [
    ((431, 2048, 8192, 32, False, False), (200, 2048, 4096, 32, False, False)),
    ((431, 2048, 8192, 32, True, False), (64, 1024, 8192, 64, True, False)),
    ((300, 1536, 8192, 32, False, True), (100, 512, 2048, 128, True, True)),
])
def test_noalloc_matches_workspace_entry(dev, first, second):
    import aq
    lib = aq.lib()
    for i, (m, n, k, g, xf, add) in enumerate((first, second)):
        got, want, wsb = _gemm_pair(dev, lib, m, n, k, g, add, xf, 100 + 10 * i + m)
        assert wsb > 0  # a split-K shape: the static array is in use
        np.testing.assert_array_equal(got, want)


def test_noalloc_refuses_partials_beyond_its_array(dev):
    import aq
    lib = aq.lib()
    m, n, k = 1120, 4096, 8192  # 160 tiles x 2 splits: 36.7 MB of partials > 32 MiB
    assert lib.aq_gemm_q4_workspace_bytes(m, n, k) > (32 << 20)
    buf = ctypes.create_string_buffer(4096 + 16)
    p = (ctypes.addressof(buf) + 15) & ~15  # refused before any memory is touched
    assert lib.aq_gemm_q4_noalloc(p, 0, p, p, p, m, n, k, 32, 0, None) == 6
