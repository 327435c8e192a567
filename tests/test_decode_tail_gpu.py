"""Regression: the decode merges never read past the split count.

A merging lane folds partials in batches: 4 subs x 4 or 8 partials in the
single-launch merge, 16 subs x 8 in the combine launch.  When the split count
is not a multiple of the batch, the last batch names partials j >= S; those
must read as zeros (and be masked), never as the memory that follows the
scratch.  Here that memory holds NaN and -inf, and the rows are ragged with
``kv_last`` per row, so some splits are empty (m = -inf, the value that turns
a zero weight into NaN).  Output must be finite and within 2e-3 of the CPU
oracle, for caller scratch in both merge modes and for the no-allocation
entry point (whose m array follows its acc array).
"""

import pytest
import torch

import oracle
from qwenforge_amd import _lib, ops, workloads

pytestmark = pytest.mark.gpu
TOL = 2e-3
POISON = 1 << 16  # floats of NaN / -inf after each scratch array (256 KiB)


def _poisoned(n: int, dev, shape):
    """A contiguous fp32 view of ``shape`` whose buffer continues with NaN / -inf."""
    buf = torch.full((n + POISON,), float("nan"), dtype=torch.float32, device=dev)
    buf[n + 1::2] = float("-inf")
    return buf[:n].view(*shape), buf


def _case(batch, splits):
    case = workloads.decode_ragged(batch, lo=64, hi=1024, seed=100 + splits)
    # The first row shorter than one 32-key tile per split: its later splits are empty.
    n0 = 40
    case.key_cache[0, :, n0:] = 0
    case.value_cache[0, :, n0:] = 0
    case.bias[0, n0:] = oracle.FP16_MIN
    case.lengths[0] = n0
    return case


def _check(case, out):
    ref = oracle.grouped_decode_attention(case.grouped, case.key_cache, case.value_cache,
                                          case.bias)
    got = out.float().cpu()
    assert torch.isfinite(got).all()
    assert (got - ref).abs().max().item() <= TOL


@pytest.mark.parametrize("fused,splits", [(True, 3), (True, 5), (True, 25), (True, 17),
                                          (False, 3), (False, 5), (False, 25), (False, 39),
                                          (False, 129)])
def test_merge_reads_no_partial_past_split_count(dev, fused, splits):
    batch = 4
    case = _case(batch, splits)
    c = case.to(dev)
    b, kvh, g, d = c.grouped.shape
    cap = c.key_cache.shape[2]
    rows = b * kvh * splits * g
    acc, _ = _poisoned(rows * d, dev, (b, kvh, splits, g, d))
    m, _ = _poisoned(rows, dev, (b, kvh, splits, g))
    l, _ = _poisoned(rows, dev, (b, kvh, splits, g))
    out = torch.full((b, kvh, g, d), float("nan"), dtype=torch.float16, device=dev)
    flash = (acc, m, l, out)
    if fused:
        flash += (torch.zeros(ops.ticket_size(b, kvh, splits), dtype=torch.int32, device=dev),)
    kv_last = torch.tensor([n - 1 for n in case.lengths], dtype=torch.int64, device=dev)
    print(f"[decode tail fused={fused} splits={splits}] cap={cap}", flush=True)
    ops.flash_decode_attention(c.grouped, c.key_cache, c.value_cache, c.bias, flash,
                               kv_last=kv_last)
    torch.cuda.synchronize()
    _check(case, out)


@pytest.mark.parametrize("splits", [3, 5, 25, 39])
def test_noalloc_merge_reads_no_partial_past_split_count(dev, splits):
    lib = _lib.load()
    case = _case(4, splits)
    c = case.to(dev)
    b, kvh, g, d = c.grouped.shape
    kv_last = torch.tensor([n - 1 for n in case.lengths], dtype=torch.int64, device=dev)
    out = torch.full((b, kvh, g, d), float("nan"), dtype=torch.float16, device=dev)
    gq, k, v = c.grouped, c.key_cache, c.value_cache
    print(f"[noalloc tail splits={splits}]", flush=True)
    rc = lib.qf_decode_attn_noalloc(gq.data_ptr(), gq.stride(0), gq.stride(1), gq.stride(2),
                                    k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
                                    v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
                                    c.bias.data_ptr(), c.bias.stride(0),
                                    kv_last.data_ptr(), 1, splits,
                                    out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
                                    b, kvh, g, d, k.shape[2], 0.125,
                                    torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "qf_decode_attn_noalloc")
    torch.cuda.synchronize()
    _check(case, out)
