"""The streaming-read kernel (the ceiling the matrix-vector kernels are measured against) reads every byte once:
the XOR of its per-workgroup words equals the XOR of the buffer, for any workgroup count."""
import numpy as np
import pytest

from _util import to_dev, to_np

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,blocks", [(16, 0), (4096, 0), (9_465_872, 0), (9_465_872, 256), (9_465_872, 8192),
                                           (1_048_592, 3), (148_000_000, 0)])
def test_stream_read_xor(dev, nbytes, blocks):
    import torch
    from aq import ops
    rng = np.random.default_rng(nbytes + blocks)
    words = rng.integers(0, 2 ** 32, nbytes // 4, dtype=np.uint32)
    sink = torch.zeros(4 * ops.STREAM_READ_MAX_BLOCKS, dtype=torch.int32, device=dev)
    torch.ops.aq.stream_read(to_dev(words, dev), sink, blocks)
    used = 4 * (blocks if blocks else min(ops.STREAM_READ_MAX_BLOCKS, -(-(nbytes // 16) // 512)))
    got = np.bitwise_xor.reduce(to_np(sink).view(np.uint32)[:used])
    assert got == np.bitwise_xor.reduce(words)
