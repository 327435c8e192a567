"""The streaming prefill's work order at its thresholds.

With one to two workgroups per CU the kernel permutes its grid: the
first-round workgroups whose CUs get no second one take the heaviest query
tiles, and the second round runs lightest first.  These cases put the grid
(query tiles x 16 heads, B=1) exactly at one workgroup per CU, one past it,
exactly at two and one past two, with a ragged last tile.  Every (query
tile, head) item must still be computed once, so each case is checked against
the oracle (``oracle.causal_prefill`` on ``oracle.apply_rope_fp16``-rotated
q/k, SE:164-251 / SE:542-554) within 2e-3, with the cache bit-exact.
"""

import pytest
import torch

import oracle
from qwenforge_amd import ops

pytestmark = pytest.mark.gpu
TOL = 2e-3
QH, KVH = 16, 2


@pytest.mark.parametrize("extra_tiles", [0, 1])
@pytest.mark.parametrize("rounds", [1, 2])
def test_work_order_thresholds(dev, rounds, extra_tiles):
    cus = ops.num_cus(dev)
    if cus % QH:
        pytest.skip(f"{cus} CUs is not a multiple of {QH} heads")
    tiles = rounds * cus // QH + extra_tiles
    seq = 64 * tiles - 5  # ragged last query tile
    print(f"[prefill order cus={cus} tiles={tiles} items={tiles * QH} S={seq}]", flush=True)
    gen = torch.Generator("cpu").manual_seed(tiles)
    q = torch.randn(1, QH, seq, 64, generator=gen).half()
    k = torch.randn(1, KVH, seq, 64, generator=gen).half()
    v = torch.randn(1, KVH, seq, 64, generator=gen).half()
    cos, sin = oracle.rope_cos_sin(torch.arange(seq), oracle.inv_freq(64, 1e6))
    kc = torch.zeros(1, KVH, seq, 64, dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    out = ops.gqa_flash_prefill_rope_append(q.to(dev), k.to(dev), v.to(dev), cos.to(dev),
                                            sin.to(dev), kc, vc, 0)
    torch.cuda.synchronize()
    q_rot = oracle.apply_rope_fp16(q, cos, sin)
    k_rot = oracle.apply_rope_fp16(k, cos, sin)
    ref = oracle.causal_prefill(q_rot, k_rot, v)
    assert (out.float().cpu() - ref).abs().max().item() <= TOL
    assert torch.equal(kc.cpu(), k_rot)
    assert torch.equal(vc.cpu(), v)
