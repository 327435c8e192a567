"""The split launch over the reference's capacity ranges (``qf_decode_split_capacity``).

Split s covers ``[s*split_len, min(+split_len, cap))`` with ``split_len =
ceil(cap / S)`` rounded up to 32 (SE:851) and ``kv_last`` only masks, so the
slots past it are read.  Checked against ``oracle.split_partials`` with
``upper = kv_last + 1`` (SE:32-115 restated) and, after the combine launch
(SE:117-162), against ``oracle.grouped_decode_attention`` on the cache
truncated at ``kv_last``.  NaN is planted in every K and V slot past
``kv_last``: the kernel must drop those rows, not just weight them by zero.
Tolerances as ``tests/test_decode_gpu.py``: output max-abs-err 2e-3; partials
m within 1e-3 (natural-log units), l and acc within 2e-3 relative to l.
"""

import pytest
import torch

import oracle
from qwenforge_amd import ops, workloads

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _split_len(cap, splits):
    return ((cap + splits - 1) // splits + 31) // 32 * 32


def _plant_nan(case, lasts):
    for b, last in enumerate(lasts):
        case.key_cache[b, :, last + 1:] = float("nan")
        case.value_cache[b, :, last + 1:] = float("nan")


def _split(case, dev, splits, kv_last, capacity=True):
    c = case.to(dev)
    b, kvh, g, _ = c.grouped.shape
    cap = c.key_cache.shape[2]
    flash = ops.make_flash_scratch(b, kvh, g, cap, dev, splits=splits, fused=False)
    ops.flash_decode_split(c.grouped, c.key_cache, c.value_cache, c.bias, flash,
                           kv_last=kv_last, split_capacity=capacity)
    out = ops.flash_decode_combine(flash)
    torch.cuda.synchronize()
    return [t.cpu() for t in flash[:3]], out.float().cpu()


def _check_partials(got, ref):
    acc, m, l = got
    r_acc, r_m, r_l = ref
    fin = torch.isfinite(r_m)
    assert torch.equal(fin, torch.isfinite(m))
    if fin.any():
        assert (m[fin] - r_m[fin]).abs().max().item() <= 1e-3
    # Empty splits hold exactly the empty state.
    assert torch.all(l[~fin] == 0) and torch.all(acc[~fin] == 0)
    rel_l = ((l - r_l).abs() / r_l.clamp_min(1e-6)).max().item()
    assert rel_l <= 2e-3
    assert ((acc - r_acc).abs() / r_l[..., None].clamp_min(1e-6)).max().item() <= 2e-3


@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("splits", [1, 4, 8, 33])
@pytest.mark.parametrize("last_of", ["full", "half", "early", "first"])
def test_shared_bound_partials_and_output(dev, last_of, splits, with_bias):
    """One kv_last for every row (the engine's write slot): splits before,
    across and wholly past it."""
    cap = 1152
    last = {"full": cap - 1, "half": cap // 2 + 5, "early": 37, "first": 0}[last_of]
    case = workloads.decode_uniform(2, cap, seed=splits + 7 * len(last_of), with_bias=with_bias)
    if with_bias:
        case.bias[:, 3::7] = workloads.FP16_MIN  # holes; slot 0 stays valid
    _plant_nan(case, [last] * 2)
    print(f"[decode capacity last={last} splits={splits} bias={with_bias}]", flush=True)
    kv_last = torch.tensor([last], dtype=torch.int64, device=dev)
    got, out = _split(case, dev, splits, kv_last)
    ref = oracle.split_partials(case.grouped, case.key_cache, case.value_cache, case.bias,
                                splits, split_len=_split_len(cap, splits), upper=last + 1)
    _check_partials(got, ref)
    bias = None if case.bias is None else case.bias[:, :last + 1]
    expect = oracle.grouped_decode_attention(case.grouped, case.key_cache[:, :, :last + 1],
                                             case.value_cache[:, :, :last + 1], bias)
    assert (out - expect).abs().max().item() <= TOL


def test_per_row_bounds(dev):
    """kv_last per row (stride 1), NaN past each row's bound."""
    cap = 2048
    lasts = [2047, 900, 31, 1500]
    case = workloads.decode_uniform(4, cap, seed=11)
    _plant_nan(case, lasts)
    kv_last = torch.tensor(lasts, dtype=torch.int64, device=dev)
    _, out = _split(case, dev, 16, kv_last)
    for b, last in enumerate(lasts):
        expect = oracle.grouped_decode_attention(case.grouped[b:b + 1],
                                                 case.key_cache[b:b + 1, :, :last + 1],
                                                 case.value_cache[b:b + 1, :, :last + 1], None)
        assert (out[b:b + 1] - expect).abs().max().item() <= TOL, b


@pytest.mark.parametrize("cap", [33, 100, 1152, 4095])
def test_without_bound_equals_default_split(dev, cap):
    """With no kv_last both entry points split the capacity: identical bits."""
    case = workloads.decode_uniform(1, cap, seed=cap)
    splits = min(16, cap // 8)
    got_cap, out_cap = _split(case, dev, splits, None, capacity=True)
    got_def, out_def = _split(case, dev, splits, None, capacity=False)
    for a, b in zip(got_cap, got_def):
        assert torch.equal(a, b)
    assert torch.equal(out_cap, out_def)


def test_bound_past_capacity_is_clamped(dev):
    """kv_last >= cap reads every slot, as the default entry point does."""
    cap = 640
    case = workloads.decode_uniform(1, cap, seed=4)
    kv_last = torch.tensor([cap + 500], dtype=torch.int64, device=dev)
    _, out = _split(case, dev, 8, kv_last)
    expect = oracle.grouped_decode_attention(case.grouped, case.key_cache, case.value_cache, None)
    assert (out - expect).abs().max().item() <= TOL


@pytest.mark.parametrize("groups", [1, 4, 16])
def test_group_sizes_and_kv_heads(dev, groups):
    """G query heads per kv head other than 7, three kv heads, a shared bound
    mid-row with NaN past it, split counts that leave empty splits."""
    gen = torch.Generator("cpu").manual_seed(100 + groups)
    cap, last = 700, 421
    q = torch.randn(2, 3, groups, 64, generator=gen).half()
    k = torch.randn(2, 3, cap, 64, generator=gen).half()
    v = torch.randn(2, 3, cap, 64, generator=gen).half()
    case = workloads.DecodeCase(q, k, v, None, [cap, cap])
    _plant_nan(case, [last, last])
    kv_last = torch.tensor([last], dtype=torch.int64, device=dev)
    for splits in (3, 11):
        got, out = _split(case, dev, splits, kv_last)
        ref = oracle.split_partials(case.grouped, case.key_cache, case.value_cache, None, splits,
                                    split_len=_split_len(cap, splits), upper=last + 1)
        _check_partials(got, ref)
        expect = oracle.grouped_decode_attention(case.grouped, case.key_cache[:, :, :last + 1],
                                                 case.value_cache[:, :, :last + 1], None)
        assert (out - expect).abs().max().item() <= TOL, splits
