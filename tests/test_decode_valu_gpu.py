"""The VALU comparison kernel (qf_decode_split_valu, include/qf_probe.h) is a
correct decode split launch: its partials, merged by the library's combine
launch, are within 2e-3 of the CPU oracle at the shapes the bench compares it
on (configs 1-3), so its timing against the MFMA kernel compares like with
like.  Arguments the kernel does not support are rejected."""

import pytest
import torch

import oracle
from qwenforge_amd import _lib, ops, workloads

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _valu(case, splits, dev, per_row):
    c = case.to(dev)
    b, kvh, g, d = c.grouped.shape
    cap = c.key_cache.shape[2]
    flash = ops.make_flash_scratch(b, kvh, g, cap, dev, splits=splits, fused=False)
    acc, m, l = flash[:3]
    kv_last = torch.tensor([n - 1 for n in case.lengths], dtype=torch.int64, device=dev)
    q, k, v = c.grouped, c.key_cache, c.value_cache
    lib = _lib.load()
    rc = lib.qf_decode_split_valu(q.data_ptr(), *q.stride()[:3], k.data_ptr(), *k.stride()[:3],
                                  v.data_ptr(), *v.stride()[:3],
                                  kv_last.data_ptr() if per_row else None, 1 if per_row else 0,
                                  acc.data_ptr(), m.data_ptr(), l.data_ptr(), splits,
                                  b, kvh, g, d, cap, d ** -0.5,
                                  torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "qf_decode_split_valu")
    out = ops.flash_decode_combine(flash)
    torch.cuda.synchronize()
    return out.float().cpu()


@pytest.mark.parametrize("name,build,splits,per_row", [
    ("config1", lambda: workloads.decode_uniform(1, 512, seed=0), 16, False),
    ("config2", lambda: workloads.decode_ragged(4, seed=0), 32, True),
    ("config3", lambda: workloads.decode_uniform(1, 32768, seed=0, heavy_frac=0.01), 128, False),
    ("ragged_tail", lambda: workloads.decode_ragged(3, lo=33, hi=700, seed=5), 7, True),
])
def test_valu_split_matches_oracle(dev, name, build, splits, per_row):
    case = build()
    print(f"[valu {name}] splits={splits}", flush=True)
    got = _valu(case, splits, dev, per_row)
    ref = torch.zeros_like(got)
    for b, n in enumerate(case.lengths):
        ref[b:b + 1] = oracle.grouped_decode_attention(case.grouped[b:b + 1],
                                                       case.key_cache[b:b + 1, :, :n],
                                                       case.value_cache[b:b + 1, :, :n])
    assert (got - ref).abs().max().item() <= TOL


def test_valu_split_rejects_unsupported_shapes(dev):
    lib = _lib.load()
    assert lib.qf_decode_split_valu(16, 0, 0, 0, 16, 0, 0, 0, 16, 0, 0, 0, None, 0,
                                    16, 16, 16, 4, 1, 2, 8, 64, 64, 0.125, None) == -2  # G != 7
    assert lib.qf_decode_split_valu(8, 0, 0, 0, 16, 0, 0, 0, 16, 0, 0, 0, None, 0,
                                    16, 16, 16, 4, 1, 2, 7, 64, 64, 0.125, None) == -1  # misaligned
