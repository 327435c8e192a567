"""Parity of the HIP split-K decode attention against the CPU oracle.

Oracle: ``oracle.grouped_decode_attention`` (fp32 restatement of the graph
step's attention, SE:939-972) and ``oracle.split_partials`` (SE:32-115).
Tolerance: max-abs-err 2e-3 on the fp16 output.
"""

import pytest
import torch

import oracle
from qwenforge_amd import ops, workloads

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _ref(case):
    return oracle.grouped_decode_attention(case.grouped, case.key_cache, case.value_cache, case.bias)


def _run(case, dev, splits=None, fused=None, kv_last=None, reference_tuple=False):
    c = case.to(dev)
    b, kvh, g, _ = c.grouped.shape
    cap = c.key_cache.shape[2]
    if reference_tuple:
        # The reference's own scratch rule (SE:1027-1045): 4-tuple, two launches.
        splits = max(1, min(32, 272 // (b * kvh), cap // 256))
        flash = ops.make_flash_scratch(b, kvh, g, cap, dev, splits=splits, fused=False)
    else:
        flash = ops.make_flash_scratch(b, kvh, g, cap, dev, splits=splits, fused=fused)
    out = ops.flash_decode_attention(c.grouped, c.key_cache, c.value_cache, c.bias, flash,
                                     kv_last=kv_last)
    torch.cuda.synchronize()
    return out.float().cpu(), flash


def _err(a, b):
    return (a - b).abs().max().item()


@pytest.mark.parametrize("fused", [True, False])
def test_config1_b1_l512(dev, fused):
    case = workloads.decode_uniform(1, 512, seed=0)
    print(f"[decode cfg1 fused={fused}]", flush=True)
    out, _ = _run(case, dev, fused=fused)
    assert _err(out, _ref(case)) <= TOL


def test_config1_reference_scratch_tuple(dev):
    case = workloads.decode_uniform(1, 2048, seed=1, with_bias=True)
    out, _ = _run(case, dev, reference_tuple=True)
    assert _err(out, _ref(case)) <= TOL


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("splits", [1, 2, 5, 16, 17, 64, 128, 256])
def test_config3_long_heavy_keys_any_split(dev, splits, fused):
    case = workloads.decode_uniform(1, 32768, seed=0, heavy_frac=0.01)
    print(f"[decode cfg3 splits={splits} fused={fused}]", flush=True)
    out, _ = _run(case, dev, splits=splits, fused=fused)
    assert _err(out, _ref(case)) <= TOL


@pytest.mark.parametrize("use_kv_last", [False, True])
def test_config2_ragged_24_layers(dev, use_kv_last):
    layers = workloads.decode_ragged_layers(24, 4, seed=0)
    worst = 0.0
    for i, case in enumerate(layers):
        kv_last = None
        if use_kv_last:
            kv_last = torch.tensor([n - 1 for n in case.lengths], dtype=torch.int64, device=dev)
        out, _ = _run(case, dev, kv_last=kv_last)
        worst = max(worst, _err(out, _ref(case)))
    assert worst <= TOL


@pytest.mark.parametrize("batch,length", [(1, 8192), (2, 4096), (4, 8192), (8, 2048), (8, 4096),
                                          (3, 5000), (1, 2500), (8, 512), (1, 200), (4, 256), (12, 256)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_decode_plan_shapes_match_oracle(dev, batch, length, with_bias):
    """The default plan (ops.decode_plan) at the shapes where it picks split +
    combine launches with 16-128 splits (one workgroup per CU, or fewer
    64-key splits), a capped single launch, or one split for rows of at most
    256 slots; rows ragged through kv_last,
    stale NaN past each row's last slot, and optionally a bias with holes
    inside the valid range (fp16-min, as the reference masks padding)."""
    case = workloads.decode_uniform(batch, length, seed=length + batch)
    gen = torch.Generator().manual_seed(batch)
    lengths = torch.randint(length // 2, length + 1, (batch,), generator=gen).tolist()
    for b, n in enumerate(lengths):
        case.key_cache[b, :, n:] = float("nan")
        case.value_cache[b, :, n:] = float("nan")
    bias = None
    if with_bias:
        bias = torch.zeros(batch, length, dtype=torch.float16)
        bias[torch.rand(batch, length, generator=gen) < 0.1] = oracle.FP16_MIN
        for b, n in enumerate(lengths):
            bias[b, n - 1] = 0.0  # at least one valid slot per row
        case.bias = bias
    kv_last = torch.tensor([n - 1 for n in lengths], dtype=torch.int64, device=dev)
    splits, fused = ops.decode_plan(batch, 2, length)
    print(f"[decode plan B={batch} L={length} bias={with_bias}] splits={splits} fused={fused}",
          flush=True)
    out, flash = _run(case, dev, kv_last=kv_last)
    assert flash[0].shape[2] == splits and (len(flash) > 4) == fused
    worst = 0.0
    for b, n in enumerate(lengths):
        ref = oracle.grouped_decode_attention(case.grouped[b:b + 1], case.key_cache[b:b + 1, :, :n],
                                              case.value_cache[b:b + 1, :, :n],
                                              None if bias is None else bias[b:b + 1, :n])
        worst = max(worst, _err(out[b:b + 1], ref))
    assert worst <= TOL


def test_partials_match_oracle_split(dev):
    case = workloads.decode_ragged(4, seed=3)
    splits = 7
    out, flash = _run(case, dev, splits=splits, fused=False)
    acc, m, l = (t.cpu() for t in flash[:3])
    cap = case.key_cache.shape[2]
    split_len = ((cap + splits - 1) // splits + 31) // 32 * 32
    r_acc, r_m, r_l = oracle.split_partials(case.grouped, case.key_cache, case.value_cache,
                                            case.bias, splits, split_len=split_len)
    # m is in natural-log units, compared where finite.
    fin = torch.isfinite(r_m)
    assert torch.equal(fin, torch.isfinite(m))
    assert (m[fin] - r_m[fin]).abs().max().item() <= 1e-3
    rel_l = ((l - r_l).abs() / r_l.clamp_min(1e-6)).max().item()
    assert rel_l <= 2e-3
    scale = r_l[..., None].clamp_min(1e-6)
    assert ((acc - r_acc).abs() / scale).max().item() <= 2e-3


@pytest.mark.parametrize("cap", [1, 7, 33, 100, 4095])
def test_odd_capacities_and_empty_splits(dev, cap):
    case = workloads.decode_uniform(2, cap, seed=cap)
    out, _ = _run(case, dev, splits=min(64, 3 * cap))
    assert _err(out, _ref(case)) <= TOL


def test_single_valid_key_returns_its_value(dev):
    case = workloads.decode_uniform(1, 1024, seed=5, with_bias=True)
    j = 617
    case.bias.fill_(workloads.FP16_MIN)
    case.bias[:, j] = 0.0
    out, _ = _run(case, dev, splits=16)
    expect = case.value_cache[:, :, j:j + 1, :].float().expand(-1, -1, 7, -1)
    assert _err(out, expect) <= 1e-3


def test_uniform_value_rows(dev):
    case = workloads.decode_uniform(1, 3000, seed=6)
    row = torch.randn(64).half()
    case.value_cache[:] = row
    out, _ = _run(case, dev)
    assert _err(out, row.float().expand_as(out)) <= 1e-3


@pytest.mark.parametrize("splits,fused", [(None, None), (1, False), (3, True), (3, False),
                                          (8, True), (33, True), (33, False)])
def test_kv_last_shared_equals_truncated_cache(dev, splits, fused):
    """2501 valid slots: 1 to 10 tiles per wave (odd and even counts of the
    paired tile loop), with NaN in every slot past kv_last."""
    case = workloads.decode_uniform(1, 4096, seed=7)
    last = 2500
    kv_last = torch.tensor([last], dtype=torch.int64, device=dev)
    # Garbage past kv_last must never be read.
    case.key_cache[:, :, last + 1:] = float("nan")
    case.value_cache[:, :, last + 1:] = float("nan")
    print(f"[decode kv_last splits={splits} fused={fused}]", flush=True)
    out, _ = _run(case, dev, splits=splits, fused=fused, kv_last=kv_last)
    ref = oracle.grouped_decode_attention(case.grouped, case.key_cache[:, :, :last + 1],
                                          case.value_cache[:, :, :last + 1], None)
    assert _err(out, ref) <= TOL


@pytest.mark.parametrize("groups", [1, 4, 7, 16])
def test_group_sizes(dev, groups):
    gen = torch.Generator("cpu").manual_seed(groups)
    q = torch.randn(2, 3, groups, 64, generator=gen).half()
    k = torch.randn(2, 3, 700, 64, generator=gen).half()
    v = torch.randn(2, 3, 700, 64, generator=gen).half()
    case = workloads.DecodeCase(q, k, v, None, [700, 700])
    out, _ = _run(case, dev, splits=4)
    assert _err(out, _ref(case)) <= TOL


@pytest.mark.parametrize("splits", [2, 8, 64])
def test_fused_ticket_rearms_across_calls(dev, splits):
    """Seven calls on one scratch over three inputs: a partial or a ticket
    count left from an earlier call (same slot, another input) would show up
    in the output."""
    cases = [workloads.decode_uniform(1, 8192, seed=s).to(dev) for s in (8, 9, 10)]
    flash = ops.make_flash_scratch(1, 2, 7, 8192, dev, splits=splits, fused=True)
    for i in range(7):
        c = cases[i % 3]
        print(f"[decode rearm splits={splits} call {i}]", flush=True)
        out = ops.flash_decode_attention(c.grouped, c.key_cache, c.value_cache, None, flash)
        ref = oracle.grouped_decode_attention(c.grouped.cpu(), c.key_cache.cpu(), c.value_cache.cpu())
        assert _err(out.float().cpu(), ref) <= TOL, f"call {i}"
    assert int(flash[4].abs().sum()) == 0  # tickets re-armed


def test_strided_grouped_view_from_projection(dev):
    """grouped as the engine builds it: a view of the fused QKV projection (SE:917-939)."""
    gen = torch.Generator("cpu").manual_seed(11)
    b = 4
    projected = torch.randn(b, 1, 1152, generator=gen).half()
    grouped = projected[..., :896].view(b, 1, 14, 64).transpose(1, 2).reshape(b, 2, 7, 64)
    k = torch.randn(b, 2, 1152, 64, generator=gen).half()
    v = torch.randn(b, 2, 1152, 64, generator=gen).half()
    case = workloads.DecodeCase(grouped, k, v, None, [1152] * b)
    out, _ = _run(case, dev)
    assert _err(out, _ref(case)) <= TOL


def test_graph_capture_replay(dev):
    """Captured once, replayed with new cache contents and a moving kv_last."""
    case = workloads.decode_uniform(4, 2048, seed=12).to(dev)
    flash = ops.make_flash_scratch(4, 2, 7, 2048, dev)
    kv_last = torch.tensor([1000], dtype=torch.int64, device=dev)
    bias = torch.zeros(4, 2048, dtype=torch.float16, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.flash_decode_attention(case.grouped, case.key_cache, case.value_cache, bias, flash, kv_last)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.flash_decode_attention(case.grouped, case.key_cache, case.value_cache, bias, flash, kv_last)
    for step, last in enumerate([1000, 1500, 2047, 17]):
        kv_last.fill_(last)
        case.value_cache.mul_(-1 if step % 2 else 1)
        graph.replay()
        torch.cuda.synchronize()
        got = flash[3].float().cpu()
        ref = oracle.grouped_decode_attention(case.grouped.cpu(), case.key_cache[:, :, :last + 1].cpu(),
                                              case.value_cache[:, :, :last + 1].cpu())
        assert _err(got, ref) <= TOL, f"replay {step}"


def test_single_launch_64_splits_graph_replay(dev):
    """The single-launch merge past 32 splits (one workgroup folds all 64
    partials of its (b, h)): captured once, replayed with new cache contents,
    a moving kv_last and NaN past it; the tickets re-arm on every replay."""
    case = workloads.decode_uniform(2, 8192, seed=13).to(dev)
    flash = ops.make_flash_scratch(2, 2, 7, 8192, dev, splits=64, fused=True)
    kv_last = torch.tensor([4000, 7000], dtype=torch.int64, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.flash_decode_attention(case.grouped, case.key_cache, case.value_cache, None, flash, kv_last)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.flash_decode_attention(case.grouped, case.key_cache, case.value_cache, None, flash, kv_last)
    k0, v0 = case.key_cache.clone(), case.value_cache.clone()
    for step, lasts in enumerate([(4000, 7000), (8191, 31), (2047, 2048), (100, 6000), (5000, 5000)]):
        print(f"[decode 64-split replay {step}] kv_last={lasts}", flush=True)
        kv_last.copy_(torch.tensor(lasts, dtype=torch.int64))
        case.key_cache.copy_(k0)
        case.value_cache.copy_(v0 * (-1 if step % 2 else 1))
        for b, last in enumerate(lasts):
            case.key_cache[b, :, last + 1:] = float("nan")
            case.value_cache[b, :, last + 1:] = float("nan")
        graph.replay()
        torch.cuda.synchronize()
        got = flash[3].float().cpu()
        for b, last in enumerate(lasts):
            ref = oracle.grouped_decode_attention(case.grouped[b:b + 1].cpu(),
                                                  case.key_cache[b:b + 1, :, :last + 1].cpu(),
                                                  case.value_cache[b:b + 1, :, :last + 1].cpu())
            assert _err(got[b:b + 1], ref) <= TOL, f"replay {step} row {b}"
    assert int(flash[4].abs().sum()) == 0


def test_split_then_combine_equals_attn(dev):
    """The reference's two launches (SE:854-873) through the separate entry points."""
    case = workloads.decode_ragged(4, seed=21)
    c = case.to(dev)
    flash = ops.make_flash_scratch(4, 2, 7, c.key_cache.shape[2], dev, splits=12, fused=False)
    ops.flash_decode_split(c.grouped, c.key_cache, c.value_cache, c.bias, flash)
    out = ops.flash_decode_combine(flash).float().cpu()
    assert _err(out, _ref(case)) <= TOL
    full = ops.flash_decode_attention(c.grouped, c.key_cache, c.value_cache, c.bias, flash)
    assert torch.equal(full.float().cpu(), out)
