"""Paged-cache generation and continuous batching (``paged_engine``).

* Teacher-forced parity with the CPU oracle (``oracle.model``): each row is
  an independent sequence -- its own prefill (SE:679-737) and its own decode
  steps appending at its own next slot (SE:876-982 with a per-row slot, no
  padding holes) -- so the paged step must match the oracle row by row.
* Continuous batching: requests admitted into rows freed by finished
  requests must produce exactly the tokens they produce when served alone in
  the same step shape (every kernel of the step is row-independent), and
  every page must be back in the pool at the end.
"""

import pytest
import torch

import oracle.model as om
from qwenforge_amd.model import Qwen2Config, init_weights, weights_to
from qwenforge_amd.paged_engine import PagedDecodeEngine

pytestmark = pytest.mark.gpu
LOGIT_TOL = 3e-2  # fp16 engine vs fp32 oracle, logits std ~0.6 (as the dense engine tests)


@pytest.mark.parametrize("page", [64, 128])
def test_paged_prefill_and_decode_match_oracle(dev, page):
    cfg = Qwen2Config(layers=2)
    w_cpu = init_weights(cfg, "cpu", seed=6)
    eng = PagedDecodeEngine(cfg, weights_to(w_cpu, dev), dev)
    gen = torch.Generator().manual_seed(12)
    lengths = [37, 130, 64, 91]
    prompts = [torch.randint(0, cfg.vocab, (n,), generator=gen) for n in lengths]
    b, steps = len(prompts), 5
    need = [n + steps for n in lengths]
    ppr = -(-max(need) // page)
    kv = eng.new_paged_cache(b, b * ppr + 2, page, ppr)
    # Map rows in reverse so physical pages are not in row order.
    for r in reversed(range(b)):
        kv.map_row(r, need[r])
    logits = eng.prefill_paged([p.to(dev) for p in prompts], kv, range(b)).float().cpu()
    ref_logits, ref_caches = [], []
    for p in prompts:
        lg, rc = om.prefill(w_cpu, cfg, p.view(1, -1), ppr * page)
        ref_logits.append(lg[0])
        ref_caches.append(rc)
    ref_logits = torch.stack(ref_logits)
    err = (logits - ref_logits).abs().max().item()
    print(f"[paged engine] page={page} prefill max|dlogit| {err:.3e}", flush=True)
    assert err <= LOGIT_TOL
    for r, n in enumerate(lengths):
        for layer in range(cfg.layers):
            k, v = kv.gather(layer, r, n)
            assert (k.float().cpu() - ref_caches[r][layer][0][0, :, :n]).abs().max().item() <= 2e-2
            assert (v.float().cpu() - ref_caches[r][layer][1][0, :, :n]).abs().max().item() <= 2e-2
    ctx = eng.make_paged_context(kv, b, steps + 1)
    eng.capture_paged(ctx)
    ctx["pos"].copy_(torch.tensor(lengths, device=dev))
    ctx["step"].fill_(1)
    teacher = ref_logits.argmax(-1)
    for t in range(steps):
        ctx["token"].copy_(teacher.to(dev))
        ctx["graph"].replay()
        torch.cuda.synchronize()
        got = ctx["logits"].float().cpu()
        ref = torch.stack([
            om.decode_step(w_cpu, cfg, teacher[r:r + 1], torch.tensor([lengths[r] + t]),
                           ref_caches[r], lengths[r] + t)[0]
            for r in range(b)])
        err = (got - ref).abs().max().item()
        print(f"[paged engine] step {t} max|dlogit| {err:.3e}", flush=True)
        assert err <= LOGIT_TOL, f"step {t}"
        teacher = ref.argmax(-1)
    assert ctx["pos"].cpu().tolist() == [n + steps for n in lengths]


@pytest.mark.parametrize("max_batch", [2, 5])
def test_continuous_batching_matches_isolated_requests(dev, max_batch):
    """Five requests through 2 rows (fused step) or 5 rows (torch-projection
    step): rows are recycled as requests finish, pages return to the pool."""
    cfg = Qwen2Config(layers=2)
    eng = PagedDecodeEngine(cfg, init_weights(cfg, dev, seed=7), dev)
    gen = torch.Generator().manual_seed(3)
    lengths = [40, 100, 7, 64, 130]
    news = [6, 3, 8, 1, 5]
    prompts = [torch.randint(0, cfg.vocab, (n,), generator=gen).to(dev) for n in lengths]
    stats = {}
    print(f"[serve] max_batch={max_batch}", flush=True)
    got = eng.serve(prompts, news, max_batch=max_batch, page_size=64, stats=stats)
    kv = eng._ctx["kv"]
    assert kv.free_pages() == kv.n_pages
    assert stats["requests"] == len(prompts)
    for i, (p, n) in enumerate(zip(prompts, news)):
        alone = eng.serve([p], [n], max_batch=max_batch, page_size=64)[0]
        assert got[i].shape == (n,)
        assert torch.equal(got[i].cpu(), alone.cpu()), f"request {i}"
    if max_batch == 2:
        # Two rows: requests 0 and 1 start together; 2 takes row 1 when 1
        # finishes (after 2 replays); when 0 finishes (after 5), 3 (one token)
        # completes at its prefill and 4 takes row 0 at once; 2 and 4 both
        # finish after 9 replays.
        assert stats["replays"] == 9


def test_generate_paged_shapes_and_pages(dev):
    cfg = Qwen2Config(layers=2)
    eng = PagedDecodeEngine(cfg, init_weights(cfg, dev, seed=8), dev)
    gen = torch.Generator().manual_seed(4)
    prompts = [torch.randint(0, cfg.vocab, (n,), generator=gen).to(dev) for n in (300, 17, 1024)]
    timing = {}
    rows = eng.generate_paged(prompts, 12, timing=timing)
    assert rows.shape == (3, 12)
    # Pages: ceil((len + 11) / 64) per row.
    assert timing["pages"] == 5 + 1 + 17
