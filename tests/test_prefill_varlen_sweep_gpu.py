"""Seeded sweep of the packed ragged prefill, dense and paged caches.

Each case draws rows (1-5, each 1-1500 tokens, tile multiples and their
neighbours included), the head layout, RoPE on or off, the append offset
start_pos and the page size from one seed.  Checks (SE:1162-1204
semantics: each row a causal prefill over its own tokens, token i written to
slot start_pos + i of its row):
- attention of every row within max-abs-err 2e-3 of ``oracle.causal_prefill``
  on ``oracle.apply_rope_fp16``-rotated q/k;
- appended K (rotated) and V rows bit-exact, every other cache slot
  untouched (the caches start as random data, not zeros);
- the paged call equal to the dense one bit for bit, and its pool, gathered
  through the block table (``oracle.pages_to_dense``), equal to the dense
  cache.
"""

import pytest
import torch

import oracle
from qwenforge_amd import ops, paged

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _case(seed):
    gen = torch.Generator("cpu").manual_seed(seed)
    pick = lambda seq: seq[int(torch.randint(0, len(seq), (1,), generator=gen))]  # noqa: E731
    b = pick([1, 2, 3, 5])
    qh, kvh = pick([(14, 2), (8, 8), (4, 1), (12, 3), (16, 2)])
    lengths = [pick([1, 7, 63, 64, 65, 200, 511, 777, 1025, 1500]) for _ in range(b)]
    rope = bool(pick([True, False]))
    start = pick([0, 64, 128])
    page = pick([64, 128, 256])
    return gen, qh, kvh, lengths, rope, start, page


@pytest.mark.parametrize("seed", range(16))
def test_prefill_varlen_random(dev, seed):
    gen, qh, kvh, lengths, rope, start, page = _case(3000 + seed)
    b, total = len(lengths), sum(lengths)
    print(f"[varlen sweep seed={seed}] QH={qh} KVH={kvh} lengths={lengths} rope={rope} "
          f"start={start} page={page}", flush=True)
    q = torch.randn(total, qh, 64, generator=gen).half()
    k = torch.randn(total, kvh, 64, generator=gen).half()
    v = torch.randn(total, kvh, 64, generator=gen).half()
    starts = [0]
    for n in lengths:
        starts.append(starts[-1] + n)
    cos = sin = None
    if rope:
        pos = torch.cat([torch.arange(start, start + n) for n in lengths])
        cos, sin = oracle.rope_cos_sin(pos, oracle.inv_freq(64, 1e6))
    ppr = (start + max(lengths) + page - 1) // page
    cap = ppr * page
    n_pages = b * ppr + 2
    kc0 = torch.randn(b, kvh, cap, 64, generator=gen).half()
    vc0 = torch.randn(b, kvh, cap, 64, generator=gen).half()
    table = torch.randperm(n_pages, generator=gen)[: b * ppr].to(torch.int32).view(b, ppr).clone()
    full = [cap] * b
    kp0 = oracle.dense_to_pages(kc0, table, full, n_pages, page)
    vp0 = oracle.dense_to_pages(vc0, table, full, n_pages, page)
    cu = torch.tensor(starts, dtype=torch.int32, device=dev)
    dev_cs = (None, None) if cos is None else (cos.to(dev), sin.to(dev))
    kc, vc = kc0.to(dev), vc0.to(dev)
    kp, vp = kp0.to(dev), vp0.to(dev)
    out_d = ops.prefill_varlen(q.to(dev), k.to(dev), v.to(dev), cu, max(lengths), *dev_cs, kc, vc,
                               start, lengths=lengths)
    out_p = paged.prefill_varlen_paged(q.to(dev), k.to(dev), v.to(dev), cu, max(lengths), *dev_cs,
                                       kp, vp, table.to(dev), start, lengths=lengths)
    torch.cuda.synchronize()
    assert torch.equal(out_d.cpu(), out_p.cpu())
    out, kc, vc = out_d.cpu(), kc.cpu(), vc.cpu()
    kc_want, vc_want = kc0.clone(), vc0.clone()
    for i, n in enumerate(lengths):
        sl = slice(starts[i], starts[i + 1])
        qi, ki, vi = q[sl].transpose(0, 1), k[sl].transpose(0, 1), v[sl].transpose(0, 1)
        if rope:
            qi = oracle.apply_rope_fp16(qi, cos[sl], sin[sl])
            ki = oracle.apply_rope_fp16(ki, cos[sl], sin[sl])
        ref = oracle.causal_prefill(qi[None], ki[None], vi[None])[0]
        err = (out[sl].transpose(0, 1).float() - ref).abs().max().item()
        assert err <= TOL, f"row {i}: max abs err {err}"
        kc_want[i, :, start:start + n] = ki
        vc_want[i, :, start:start + n] = vi
    assert torch.equal(kc, kc_want) and torch.equal(vc, vc_want)
    assert torch.equal(oracle.pages_to_dense(kp.cpu(), table, full, cap), kc_want)
    assert torch.equal(oracle.pages_to_dense(vp.cpu(), table, full, cap), vc_want)
