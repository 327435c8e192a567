"""The streaming-read calibration kernel reads every word it is given: the XOR
of its per-wave results equals the XOR of the buffer's 32-bit words (numpy)."""

import numpy as np
import pytest
import torch

from qwenforge_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("words,workgroups", [(4, 1), (4096, 3), (1 << 20, 64), (12345 * 4, 1024)])
def test_stream_read_covers_every_word(dev, words, workgroups):
    gen = np.random.default_rng(words)
    host = gen.integers(0, 2 ** 31, size=words, dtype=np.int64).astype(np.int32)
    src = torch.from_numpy(host).to(dev)
    sink = torch.zeros(4 * workgroups, device=dev, dtype=torch.int32)
    lib = _lib.load()
    rc = lib.qf_stream_read(src.data_ptr(), 4 * words, sink.data_ptr(), workgroups,
                            torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "qf_stream_read")
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    assert got == np.bitwise_xor.reduce(host.view(np.uint32))
