"""Seeded sweep of paged decode attention (include/qf_paged.h).

Each case draws the page size, rows, row lengths, split count, merge mode and
bias (with holes inside the valid range, as the engine's right-padded rows
have) from one seed.  The paged call must equal the dense call bit for bit
(same values, same summation order) and stay within 2e-3 of the CPU oracle
(``oracle.grouped_decode_attention`` over each row's valid prefix).  Pool
slots that hold no valid row, and dense slots past each row's length, are
NaN, so a read through a wrong page or past kv_last shows in the output.
"""

import pytest
import torch

import oracle
from qwenforge_amd import ops, paged

pytestmark = pytest.mark.gpu
TOL = 2e-3
KVH, G, D = 2, 7, 64


def _case(seed):
    gen = torch.Generator().manual_seed(seed)
    pick = lambda seq: seq[int(torch.randint(0, len(seq), (1,), generator=gen))]  # noqa: E731
    page = pick([64, 128, 256, 512])
    b = pick([1, 2, 3, 5])
    lengths = torch.randint(1, 3001, (b,), generator=gen).tolist()
    splits = pick([1, 2, 3, 8, 16, 32, 40, 64])
    fused = bool(pick([False, True])) and splits > 1
    use_bias = bool(pick([False, True]))
    return gen, page, lengths, splits, fused, use_bias


def _pool(dense, table, lengths, n_pages, page):
    pool = oracle.dense_to_pages(dense, table, lengths, n_pages, page)
    written = torch.zeros(n_pages, page, dtype=torch.bool)
    for r, n in enumerate(lengths):
        s = torch.arange(n)
        written[table[r, s // page].long(), s % page] = True
    pool[~written[:, None, :, None].expand_as(pool)] = float("nan")
    return pool


@pytest.mark.parametrize("seed", range(20))
def test_paged_decode_random(dev, seed):
    gen, page, lengths, splits, fused, use_bias = _case(500 + seed)
    b = len(lengths)
    ppr = (max(lengths) + page - 1) // page
    cap = ppr * page
    n_pages = b * ppr + 5
    print(f"[paged sweep seed={seed}] page={page} lengths={lengths} splits={splits} "
          f"fused={fused} bias={use_bias}", flush=True)
    kd = torch.randn(b, KVH, cap, D, generator=gen).half()
    vd = torch.randn(b, KVH, cap, D, generator=gen).half()
    table = torch.randperm(n_pages, generator=gen)[: b * ppr].to(torch.int32).view(b, ppr).clone()
    kp = _pool(kd, table, lengths, n_pages, page)
    vp = _pool(vd, table, lengths, n_pages, page)
    for r, n in enumerate(lengths):
        kd[r, :, n:] = float("nan")
        vd[r, :, n:] = float("nan")
    q = torch.randn(b, KVH, G, D, generator=gen).half()
    bias = None
    if use_bias:
        bias = torch.zeros(b, cap, dtype=torch.float16)
        holes = torch.rand(b, cap, generator=gen) < 0.05
        bias[holes] = oracle.FP16_MIN
        for r, n in enumerate(lengths):
            bias[r, n:] = oracle.FP16_MIN
            bias[r, n - 1] = 0.0  # at least one valid slot per row
    last = torch.tensor([n - 1 for n in lengths], dtype=torch.int64, device=dev)
    flash_p = ops.make_flash_scratch(b, KVH, G, cap, dev, splits=splits, fused=fused)
    flash_d = ops.make_flash_scratch(b, KVH, G, cap, dev, splits=splits, fused=fused)
    bias_dev = None if bias is None else bias.to(dev)
    got = paged.flash_decode_attention_paged(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev),
                                             bias_dev, flash_p, kv_last=last)
    want = ops.flash_decode_attention(q.to(dev), kd.to(dev), vd.to(dev), bias_dev, flash_d,
                                      kv_last=last)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), want.cpu())
    worst = 0.0
    for r, n in enumerate(lengths):
        ref = oracle.grouped_decode_attention(q[r:r + 1], kd[r:r + 1, :, :n], vd[r:r + 1, :, :n],
                                              None if bias is None else bias[r:r + 1, :n])
        worst = max(worst, (got[r:r + 1].float().cpu() - ref).abs().max().item())
    assert worst <= TOL, f"max abs err {worst}"
