"""Seeded sweep of causal-prefill shapes against the CPU oracle.

Each case draws batch, head layout (query heads per kv head), prompt length
(1 to 2100 tokens: 1 to 33 query tiles, whose two halves of waves take
their key tiles alternately, one half idle in the last step of every odd
count) and the entry point (plain op, or RoPE + cache append at an offset)
from one seed.  Oracle: ``oracle.causal_prefill`` on ``oracle.apply_rope_fp16``
rotated q/k (SE:164-251, SE:542-554).  Attention within max-abs-err 2e-3,
cache rows bit-exact.
"""

import pytest
import torch

import oracle
from qwenforge_amd import ops

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _case(seed):
    gen = torch.Generator("cpu").manual_seed(seed)
    pick = lambda seq: seq[int(torch.randint(0, len(seq), (1,), generator=gen))]  # noqa: E731
    b = pick([1, 2, 3])
    qh, kvh = pick([(14, 2), (8, 8), (4, 1), (12, 3), (16, 2)])
    s = pick([1, 5, 63, 64, 65, 300, 777, 1024, 1025, 1600, 2100])
    fused = pick([True, False])
    start = pick([0, 64, 192]) if fused else 0
    q = torch.randn(b, qh, s, 64, generator=gen).half()
    k = torch.randn(b, kvh, s, 64, generator=gen).half()
    v = torch.randn(b, kvh, s, 64, generator=gen).half()
    return q, k, v, fused, start


@pytest.mark.parametrize("seed", range(24))
def test_prefill_random_shapes(dev, seed):
    q, k, v, fused, start = _case(2000 + seed)
    b, qh, s, _ = q.shape
    kvh = k.shape[1]
    print(f"[prefill sweep seed={seed}] B={b} QH={qh} KVH={kvh} S={s} fused={fused} "
          f"start={start}", flush=True)
    if fused:
        cos, sin = oracle.rope_cos_sin(torch.arange(start, start + s), oracle.inv_freq(64, 1e6))
        cap = start + s + 37
        kc = torch.zeros(b, kvh, cap, 64, dtype=torch.float16, device=dev)
        vc = torch.zeros_like(kc)
        out = ops.gqa_flash_prefill_rope_append(q.to(dev), k.to(dev), v.to(dev), cos.to(dev),
                                                sin.to(dev), kc, vc, start)
        torch.cuda.synchronize()
        q_rot = oracle.apply_rope_fp16(q, cos, sin)
        k_rot = oracle.apply_rope_fp16(k, cos, sin)
        ref = oracle.causal_prefill(q_rot, k_rot, v)
        assert torch.equal(kc[:, :, start:start + s].cpu(), k_rot)
        assert torch.equal(vc[:, :, start:start + s].cpu(), v)
        assert int(kc[:, :, :start].abs().sum()) == 0 and int(kc[:, :, start + s:].abs().sum()) == 0
    else:
        out = torch.ops.student_qwen.gqa_flash_prefill(q.to(dev), k.to(dev), v.to(dev))
        torch.cuda.synchronize()
        ref = oracle.causal_prefill(q, k, v)
    err = (out.float().cpu() - ref).abs().max().item()
    assert err <= TOL, f"max abs err {err}"
