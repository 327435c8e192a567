"""The calibration kernels read every word they are given: the XOR of their
per-wave results equals the XOR of the buffer's 32-bit words (numpy).  The
launch probe's two-round-trip form rotates its reads by a device index
(any value, negative included, wraps into the buffer); its empty form writes
nothing."""

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


@pytest.mark.parametrize("round_trips,index", [(1, 0), (2, 0), (2, 12345), (2, -7)])
def test_launch_probe_reads_its_slice(dev, round_trips, index):
    workgroups, threads = 16, 512
    words = workgroups * threads * 4
    gen = np.random.default_rng(index + 7)
    host = gen.integers(0, 2 ** 31, size=words, dtype=np.int64).astype(np.int32)
    src = torch.from_numpy(host).to(dev)
    sink = torch.zeros(workgroups * threads // 64, device=dev, dtype=torch.int32)
    idx = torch.tensor([index], dtype=torch.int64, device=dev)
    lib = _lib.load()
    rc = lib.qf_launch_probe(src.data_ptr(), 4 * words, idx.data_ptr(), sink.data_ptr(),
                             workgroups, threads, round_trips,
                             torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "qf_launch_probe")
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    assert got == np.bitwise_xor.reduce(host.view(np.uint32))


def test_launch_probe_empty_form_touches_nothing(dev):
    sink = torch.full((64,), 7, device=dev, dtype=torch.int32)
    lib = _lib.load()
    rc = lib.qf_launch_probe(None, 0, None, sink.data_ptr(), 8, 512, 0,
                             torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "qf_launch_probe")
    torch.cuda.synchronize()
    assert (sink.cpu() == 7).all()
