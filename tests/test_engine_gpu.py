"""Config 5: the Qwen2-shaped decode step with the HIP kernels inside a hipGraph.

Checked against the CPU oracle (``oracle.model``: fp32 restatement of
SE:679-737 and SE:876-982) per step with teacher forcing -- the oracle's
greedy token is fed to both sides -- so near-ties cannot cascade.
"""

import pytest
import torch

import oracle
import oracle.model as om
from qwenforge_amd.engine import DecodeEngine
from qwenforge_amd.model import Qwen2Config, init_weights, weights_to

pytestmark = pytest.mark.gpu
# fp16 engine vs fp32 oracle on N(0, 0.02) weights: logits have std ~0.6.
LOGIT_TOL = 3e-2


def _fp32(w):
    """fp32 copy of a weight dict (the oracle's upcasts then copy nothing)."""
    embed = w["embed"].float()
    return {"embed": embed, "final_norm": w["final_norm"].float(), "lm_head": embed,
            "layers": [{k: v.float() for k, v in layer.items()} for layer in w["layers"]]}


@pytest.mark.parametrize("batch", [1, 2, 3, 4, 6])
def test_teacher_forced_logits_match_oracle(dev, batch):
    """2 layers: the fused step at 1-4 rows (matrix-core tiles from 2), and at
    6 rows the torch projections around the same attention kernels."""
    _teacher_forced(dev, Qwen2Config(layers=2), batch, 200, 6, (200 + 6 + 63) // 64 * 64)


@pytest.mark.parametrize("batch", [1, 4])
def test_full_shape_teacher_forced_logits_match_oracle(dev, batch):
    """Config 5 at its real shape: 24 layers, vocab 151936, a 1024-token
    prefix in a cache of oracle.capacity(1024, 128) = 1152 slots (SE:1263-1273),
    8 teacher-forced graph replays of the captured step (SE:876-982)."""
    _teacher_forced(dev, Qwen2Config(), batch, 1024, 8, oracle.capacity(1024, 128))


def _teacher_forced(dev, cfg, batch, s, steps, cap):
    w_cpu = init_weights(cfg, "cpu", seed=0)
    w_ref = _fp32(w_cpu)
    eng = DecodeEngine(cfg, weights_to(w_cpu, dev), dev)
    gen = torch.Generator().manual_seed(batch)
    ids = torch.randint(0, cfg.vocab, (batch, s), generator=gen)
    caches = eng.new_caches(batch, cap)
    logits = eng.prefill(ids.to(dev), caches).float().cpu()
    ref_logits, ref_caches = om.prefill(w_ref, cfg, ids, cap)
    print(f"[engine L={cfg.layers} B={batch} S={s}] prefill max|dlogit| "
          f"{(logits - ref_logits).abs().max():.3e}", flush=True)
    assert (logits - ref_logits).abs().max().item() <= LOGIT_TOL
    for (kc, vc), (rk, rv) in zip(caches, ref_caches):
        assert (kc.float().cpu() - rk).abs().max().item() <= 2e-2
        assert (vc.float().cpu() - rv).abs().max().item() <= 2e-2
    ctx = eng.make_context(caches, batch, steps + 1)
    eng.capture(ctx)
    teacher = ref_logits.argmax(-1)
    ctx["pos"].fill_(s)
    ctx["write"].fill_(s)
    ctx["step"].fill_(1)
    for t in range(steps):
        ctx["token"].copy_(teacher.to(dev))
        ctx["graph"].replay()
        torch.cuda.synchronize()
        got = ctx["logits"].float().cpu()
        ref = om.decode_step(w_ref, cfg, teacher, torch.full((batch,), s + t), ref_caches, s + t)
        err = (got - ref).abs().max().item()
        print(f"[engine L={cfg.layers} B={batch}] step {t} max|dlogit| {err:.3e}", flush=True)
        assert err <= LOGIT_TOL, f"step {t}"
        top2 = ref.topk(2, dim=-1).values
        clear = (top2[:, 0] - top2[:, 1]) > 2 * LOGIT_TOL
        assert torch.equal(got.argmax(-1)[clear], ref.argmax(-1)[clear])
        teacher = ref.argmax(-1)


def test_graph_replay_equals_eager_step_full_shape(dev):
    """24 layers, full vocab: the captured step reproduces the eager step bit for bit."""
    cfg = Qwen2Config()
    w = init_weights(cfg, dev, seed=1)
    eng = DecodeEngine(cfg, w, dev)
    b, s = 4, 256
    ids = torch.randint(0, cfg.vocab, (b, s), generator=torch.Generator().manual_seed(0)).to(dev)
    cap = 320
    caches = eng.new_caches(b, cap)
    first = eng.prefill(ids, caches).argmax(-1)
    snap = [(k.clone(), v.clone()) for k, v in caches]
    ctx = eng.make_context(caches, b, 8)
    eng.capture(ctx)

    def reset(c):
        for (k, v), (k0, v0) in zip(c["caches"], snap):
            k.copy_(k0)
            v.copy_(v0)
        c["token"].copy_(first)
        c["pos"].fill_(s)
        c["write"].fill_(s)
        c["step"].fill_(1)

    reset(ctx)
    for _ in range(5):
        ctx["graph"].replay()
    torch.cuda.synchronize()
    graph_rows, graph_logits = ctx["rows"].clone(), ctx["logits"].clone()
    reset(ctx)
    for _ in range(5):
        eng._step(ctx)
    torch.cuda.synchronize()
    assert torch.equal(ctx["rows"][:, 1:6], graph_rows[:, 1:6])
    assert torch.equal(ctx["logits"], graph_logits)
    assert bool(torch.isfinite(graph_logits.float()).all())


@pytest.mark.parametrize("batch", [1, 4])
def test_generate_full_shape_128_tokens(dev, batch):
    """The bench's config-5 run: 1024-token prefix, 128 greedy tokens.  The
    cache capacity is the reference's rule (SE:1263-1273) and after 127
    replays the device-side bookkeeping (SE:1126-1132) stands at write slot
    1024 + 127 = 1151, positions 1151 and step 128."""
    cfg = Qwen2Config()
    eng = DecodeEngine(cfg, init_weights(cfg, dev, seed=2), dev)
    ids = torch.randint(0, cfg.vocab, (batch, 1024),
                        generator=torch.Generator().manual_seed(1)).to(dev)
    timing = {}
    rows = eng.generate(ids, 128, timing)
    ctx = eng._ctx
    assert rows.shape == (batch, 128)
    assert int(rows.min()) >= 0 and int(rows.max()) < cfg.vocab
    assert timing["decode_ms"] > 0
    assert ctx["caches"][0][0].shape[2] == oracle.capacity(1024, 128) == 1152
    assert int(ctx["write"].item()) == 1151 and int(ctx["step"].item()) == 128
    assert ctx["pos"].cpu().tolist() == [1151] * batch
    assert torch.equal(rows[:, 1:], ctx["rows"][:, 1:128])


def test_generate_ragged_full_shape_bookkeeping(dev):
    """Ragged prompts at full shape: capacity from the longest prompt, shared
    write slot p_max + 127 and per-row positions len_b + 127 after 127 replays."""
    cfg = Qwen2Config()
    eng = DecodeEngine(cfg, init_weights(cfg, dev, seed=2), dev)
    gen = torch.Generator().manual_seed(7)
    lengths = (512, 700, 896, 1024)
    prompts = [torch.randint(0, cfg.vocab, (n,), generator=gen).to(dev) for n in lengths]
    rows = eng.generate_ragged(prompts, 128)
    ctx = eng._ctx
    assert rows.shape == (4, 128)
    assert ctx["caches"][0][0].shape[2] == oracle.capacity(1024, 128)
    assert int(ctx["write"].item()) == 1024 + 127
    assert ctx["pos"].cpu().tolist() == [n + 127 for n in lengths]


def test_fused_step_matches_torch_step(dev):
    """The fused weight-streaming step and the torch-projection step agree
    (teacher-forced: both are fed the same tokens every step)."""
    cfg = Qwen2Config(layers=4)
    w = init_weights(cfg, dev, seed=3)
    b, s, steps = 2, 100, 3
    gen = torch.Generator().manual_seed(5)
    ids = torch.randint(0, cfg.vocab, (b, s), generator=gen).to(dev)
    teacher = torch.randint(0, cfg.vocab, (steps, b), generator=gen).to(dev)
    out = {}
    for fused in (True, False):
        eng = DecodeEngine(cfg, w, dev, fused_step=fused)
        caches = eng.new_caches(b, 192)
        eng.prefill(ids, caches)
        ctx = eng.make_context(caches, b, steps + 1)
        assert ctx["fused"] == fused
        ctx["pos"].fill_(s)
        ctx["write"].fill_(s)
        ctx["step"].fill_(1)
        logits = []
        for t in range(steps):
            ctx["token"].copy_(teacher[t])
            eng._step(ctx)
            logits.append(ctx["logits"].float().cpu())
        torch.cuda.synchronize()
        out[fused] = (torch.stack(logits), int(ctx["write"].item()), ctx["pos"].cpu(),
                      int(ctx["step"].item()),
                      [(k[:, :, s:s + steps].float().cpu(), v[:, :, s:s + steps].float().cpu())
                       for k, v in caches])
    (lf, wf, pf, sf, cf), (lt, wt, pt, st, ct) = out[True], out[False]
    err = (lf - lt).abs().max().item()
    print(f"[fused vs torch step] max|dlogit| {err:.3e}", flush=True)
    assert err <= LOGIT_TOL
    assert wf == wt == s + steps and sf == st == 1 + steps and torch.equal(pf, pt)
    for (kf, vf), (kt, vt) in zip(cf, ct):
        assert (kf - kt).abs().max().item() <= 2e-2
        assert (vf - vt).abs().max().item() <= 2e-2


@pytest.mark.parametrize("b", [2, 4])
def test_tile_weights_step_matches_row_weights(dev, b):
    """From 2 rows the fused step reads QKV and gate/up as matrix-core tiles;
    teacher-forced logits, appended cache rows and bookkeeping match the
    row-major (dot-product) kernels."""
    cfg = Qwen2Config(layers=3)
    w = init_weights(cfg, dev, seed=9)
    s, steps = 130, 3
    gen = torch.Generator().manual_seed(11)
    ids = torch.randint(0, cfg.vocab, (b, s), generator=gen).to(dev)
    teacher = torch.randint(0, cfg.vocab, (steps, b), generator=gen).to(dev)
    out = {}
    for tiles in (True, False):
        eng = DecodeEngine(cfg, w, dev, tile_weights=tiles)
        caches = eng.new_caches(b, 192)
        eng.prefill(ids, caches)
        ctx = eng.make_context(caches, b, steps + 1)
        assert ctx["fused"]
        ctx["pos"].fill_(s)
        ctx["write"].fill_(s)
        ctx["step"].fill_(1)
        logits = []
        for t in range(steps):
            ctx["token"].copy_(teacher[t])
            eng._step(ctx)
            logits.append(ctx["logits"].float().cpu())
        torch.cuda.synchronize()
        assert (eng._tiles is not None) == tiles
        out[tiles] = (torch.stack(logits), int(ctx["write"].item()), ctx["pos"].cpu(),
                      [k[:, :, s:s + steps].float().cpu() for k, _ in caches])
    (lt, wt, pt, ct), (lr, wr, pr, cr) = out[True], out[False]
    err = (lt - lr).abs().max().item()
    print(f"[tile vs row weights B={b}] max|dlogit| {err:.3e}", flush=True)
    assert err <= LOGIT_TOL
    assert wt == wr == s + steps and torch.equal(pt, pr)
    for kt, kr in zip(ct, cr):
        assert (kt - kr).abs().max().item() <= 2e-2


def test_ragged_prefill_and_decode_match_oracle(dev):
    """Variable-length prompts: packed prefill == per-row oracle prefill
    (SE:1186-1202), then teacher-forced decode over the bias-masked holes
    [len_b, max_len) with the shared write slot (SE:1120-1132)."""
    cfg = Qwen2Config(layers=2)
    w_cpu = init_weights(cfg, "cpu", seed=4)
    eng = DecodeEngine(cfg, weights_to(w_cpu, dev), dev)
    gen = torch.Generator().manual_seed(11)
    lengths = [37, 130, 64, 91]
    prompts = [torch.randint(0, cfg.vocab, (n,), generator=gen) for n in lengths]
    b, p_max, steps = len(prompts), max(lengths), 5
    cap = (p_max + steps + 63) // 64 * 64
    caches = eng.new_caches(b, cap)
    logits = eng.prefill_ragged([p.to(dev) for p in prompts], caches).float().cpu()
    shape = (b, cfg.kv_heads, cap, cfg.head_dim)
    ref_caches = [(torch.zeros(shape), torch.zeros(shape)) for _ in range(cfg.layers)]
    ref_logits = []
    for i, p in enumerate(prompts):
        lg, rc = om.prefill(w_cpu, cfg, p.view(1, -1), cap)
        ref_logits.append(lg[0])
        for (kk, vv), (rk, rv) in zip(ref_caches, rc):
            kk[i], vv[i] = rk[0], rv[0]
    ref_logits = torch.stack(ref_logits)
    err = (logits - ref_logits).abs().max().item()
    print(f"[ragged] prefill max|dlogit| {err:.3e}", flush=True)
    assert err <= LOGIT_TOL
    for (kc, vc), (rk, rv) in zip(caches, ref_caches):
        assert (kc.float().cpu() - rk).abs().max().item() <= 2e-2
        assert (vc.float().cpu() - rv).abs().max().item() <= 2e-2
    mask = torch.zeros(b, cap, dtype=torch.bool)
    for i, n in enumerate(lengths):
        mask[i, :n] = True
    ctx = eng.make_context(caches, b, steps + 1, bias_mask=mask.to(dev))
    eng.capture(ctx)
    ctx["pos"].copy_(torch.tensor(lengths, device=dev))
    ctx["write"].fill_(p_max)
    ctx["step"].fill_(1)
    bias = torch.full((b, cap), float(torch.finfo(torch.float16).min))
    bias[mask] = 0.0
    teacher = ref_logits.argmax(-1)
    for t in range(steps):
        ctx["token"].copy_(teacher.to(dev))
        ctx["graph"].replay()
        torch.cuda.synchronize()
        got = ctx["logits"].float().cpu()
        bias[:, p_max + t] = 0.0
        ref = om.decode_step(w_cpu, cfg, teacher, torch.tensor(lengths) + t, ref_caches, p_max + t,
                             bias=bias)
        err = (got - ref).abs().max().item()
        print(f"[ragged] step {t} max|dlogit| {err:.3e}", flush=True)
        assert err <= LOGIT_TOL, f"step {t}"
        teacher = ref.argmax(-1)


def test_generate_ragged_runs(dev):
    cfg = Qwen2Config(layers=4)
    eng = DecodeEngine(cfg, init_weights(cfg, dev, seed=5), dev)
    gen = torch.Generator().manual_seed(2)
    prompts = [torch.randint(0, cfg.vocab, (n,), generator=gen).to(dev) for n in (300, 17, 1024)]
    rows = eng.generate_ragged(prompts, 12)
    assert rows.shape == (3, 12)
    assert int(rows.min()) >= 0 and int(rows.max()) < cfg.vocab


def test_generate_reuses_the_captured_step(dev):
    """A second call of the same (batch, capacity) prefills into the stored
    caches and replays the stored graph (no capture; SE:1104-1118), and its
    tokens equal a fresh engine's for the same prompts, although the stored
    caches hold the first call's rows past the new prompt.  Another capacity
    is a second entry; coming back to the first one captures nothing."""
    cfg = Qwen2Config(layers=2)
    w = init_weights(cfg, dev, seed=4)
    eng = DecodeEngine(cfg, w, dev)
    gen = torch.Generator().manual_seed(11)
    a1 = torch.randint(0, cfg.vocab, (2, 200), generator=gen).to(dev)
    a2 = torch.randint(0, cfg.vocab, (2, 190), generator=gen).to(dev)   # same capacity, 256
    c1 = torch.randint(0, cfg.vocab, (2, 300), generator=gen).to(dev)   # capacity 320
    eng.generate(a1, 40)
    assert eng.captures == 1 and eng.graphs.keys() == [(2, 256, False)]
    got = eng.generate(a2, 24)
    assert eng.captures == 1
    want = DecodeEngine(cfg, w, dev).generate(a2, 24)
    assert torch.equal(got, want)
    eng.generate(c1, 12)
    assert eng.captures == 2 and eng.graphs.keys() == [(2, 256, False), (2, 320, False)]
    got = eng.generate(a1, 40)
    assert eng.captures == 2 and eng.graphs.keys() == [(2, 320, False), (2, 256, False)]
    assert torch.equal(got, DecodeEngine(cfg, w, dev).generate(a1, 40))


@pytest.mark.parametrize("batch", [3, 6])
def test_generate_ragged_reuses_the_captured_step(dev, batch):
    """Padded batches through the registry: the second call has other
    lengths (other holes) in the same capacity, so the stored bias is
    rebuilt from the new mask; tokens equal a fresh engine's.  Batch 6 runs
    the torch-projection step, batch 3 the fused one."""
    cfg = Qwen2Config(layers=2)
    w = init_weights(cfg, dev, seed=5)
    eng = DecodeEngine(cfg, w, dev)
    gen = torch.Generator().manual_seed(batch)
    first = [torch.randint(0, cfg.vocab, (n,), generator=gen).to(dev)
             for n in (60, 250, 130, 201, 17, 90)[:batch]]
    second = [torch.randint(0, cfg.vocab, (n,), generator=gen).to(dev)
              for n in (260, 33, 199, 120, 250, 5)[:batch]]
    eng.generate_ragged(first, 8)
    got = eng.generate_ragged(second, 8)
    assert eng.captures == 1 and eng.graphs.keys() == [(batch, 320, True)]
    assert torch.equal(got, DecodeEngine(cfg, w, dev).generate_ragged(second, 8))



def test_short_generations_run_the_step_eagerly(dev):
    """Below 8 new tokens nothing is captured or stored (SE:1274-1276): the
    step runs eagerly, and one token is the prefill's argmax alone.  The
    tokens are those of a captured run."""
    cfg = Qwen2Config(layers=2)
    w = init_weights(cfg, dev, seed=6)
    ids = torch.randint(0, cfg.vocab, (2, 200), generator=torch.Generator().manual_seed(3)).to(dev)
    eng = DecodeEngine(cfg, w, dev)
    short = eng.generate(ids, 4)
    one = eng.generate(ids, 1)
    assert eng.captures == 0 and len(eng.graphs) == 0
    full = DecodeEngine(cfg, w, dev).generate(ids, 8)
    assert torch.equal(short, full[:, :4]) and torch.equal(one, full[:, :1])


def test_registry_evicts_past_its_budget(dev):
    """With a budget below one entry's caches, each new shape evicts the
    previous one (the newest always stays, SE:1099-1103); coming back to an
    evicted shape captures again, and its tokens still equal a fresh engine's."""
    cfg = Qwen2Config(layers=2)
    w = init_weights(cfg, dev, seed=8)
    eng = DecodeEngine(cfg, w, dev)
    eng.graphs.byte_budget = 1
    gen = torch.Generator().manual_seed(9)
    a = torch.randint(0, cfg.vocab, (1, 100), generator=gen).to(dev)   # capacity 128
    c = torch.randint(0, cfg.vocab, (1, 150), generator=gen).to(dev)   # capacity 192
    eng.generate(a, 10)
    eng.generate(c, 10)
    assert eng.graphs.keys() == [(1, 192, False)] and eng.captures == 2
    got = eng.generate(a, 10)
    assert eng.graphs.keys() == [(1, 128, False)] and eng.captures == 3
    assert torch.equal(got, DecodeEngine(cfg, w, dev).generate(a, 10))
