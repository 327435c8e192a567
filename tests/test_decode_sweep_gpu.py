"""Seeded sweep of decode-attention shapes against the CPU oracle.

Each case draws batch, kv heads, group size, capacity, per-row bounds,
split count, merge mode (two launches or single launch) and the bias from
one seed, so the kernels' wave-count choice, idle waves of short splits,
empty splits and the single-launch merge at many split counts all meet the
oracle (``oracle.grouped_decode_attention``, SE:939-972 semantics).
Tolerance: max-abs-err 2e-3.
"""

import pytest
import torch

import oracle
from qwenforge_amd import ops

pytestmark = pytest.mark.gpu
TOL = 2e-3
FP16_MIN = float(torch.finfo(torch.float16).min)


def _case(seed):
    gen = torch.Generator("cpu").manual_seed(seed)
    pick = lambda seq: seq[int(torch.randint(0, len(seq), (1,), generator=gen))]  # noqa: E731
    b = pick([1, 2, 3, 4, 6])
    kvh = pick([1, 2, 3])
    g = pick([1, 2, 5, 7, 8, 12, 16])
    cap = pick([33, 64, 200, 511, 1024, 1500, 3000, 5000])
    lengths = torch.randint(1, cap + 1, (b,), generator=gen).tolist()
    splits = pick([1, 2, 3, 7, 8, 16, 24, 32, 40, 64])
    splits = max(1, min(splits, (cap + 31) // 32))
    fused = pick([True, False])
    mode = pick(["bias", "kv_last", "both"])
    q = torch.randn(b, kvh, g, 64, generator=gen).half()
    k = torch.zeros(b, kvh, cap, 64, dtype=torch.float16)
    v = torch.zeros_like(k)
    for i, n in enumerate(lengths):
        k[i, :, :n] = torch.randn(kvh, n, 64, generator=gen).half()
        v[i, :, :n] = torch.randn(kvh, n, 64, generator=gen).half()
    bias = torch.full((b, cap), FP16_MIN, dtype=torch.float16)
    for i, n in enumerate(lengths):
        bias[i, :n] = 0.0
    return q, k, v, bias, lengths, splits, fused, mode


@pytest.mark.parametrize("seed", range(40))
def test_decode_random_shapes(dev, seed):
    q, k, v, bias, lengths, splits, fused, mode = _case(1000 + seed)
    b, kvh, g, _ = q.shape
    cap = k.shape[2]
    print(f"[decode sweep seed={seed}] B={b} KVH={kvh} G={g} cap={cap} splits={splits} "
          f"fused={fused} mode={mode}", flush=True)
    use_bias = mode in ("bias", "both")
    kv_last = None
    if mode in ("kv_last", "both"):
        kv_last = torch.tensor([n - 1 for n in lengths], dtype=torch.int64, device=dev)
    flash = ops.make_flash_scratch(b, kvh, g, cap, dev, splits=splits, fused=fused and splits > 1)
    out = ops.flash_decode_attention(q.to(dev), k.to(dev), v.to(dev),
                                     bias.to(dev) if use_bias else None, flash, kv_last=kv_last)
    torch.cuda.synchronize()
    # Both masking forms select the same slots [0, L_b): compare with the
    # oracle over each row's valid prefix.
    ref = torch.stack([
        oracle.grouped_decode_attention(q[i:i + 1], k[i:i + 1, :, :n], v[i:i + 1, :, :n])[0]
        for i, n in enumerate(lengths)])
    err = (out.float().cpu() - ref).abs().max().item()
    assert err <= TOL, f"max abs err {err}"
    if len(flash) > 4:
        assert int(flash[4].abs().sum()) == 0  # tickets re-armed
