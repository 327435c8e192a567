"""Fused decode-step kernels (include/qf_step.h) against ``oracle.step``.

Two regimes per kernel:

* integer-valued operands (|x| = 1 rows, weights in {-1, 0, 1}): every
  projection sum is an exact fp32 integer whatever the summation order, so the
  kernel must match the oracle bit for bit -- including the fp16 RoPE
  rounding, the KV-cache slot and every untouched slot;
* Qwen2-shaped random operands (N(0, 1) activations, N(0, 0.02) weights): the
  summation order differs from the oracle's, so outputs agree to within a few
  fp16 ulps (STEP_TOL, relative).
"""

import pytest
import torch

import oracle.step as ost
from oracle.rope import inv_freq, rope_cos_sin
from qwenforge_amd import step_ops

pytestmark = pytest.mark.gpu

HIDDEN, QH, KVH, D, INTER = 896, 14, 2, 64, 4864
EPS = 1e-6
STEP_TOL = 4e-3  # |got - ref| <= STEP_TOL * max(1, |ref|)


def _close(got, ref, tol=STEP_TOL):
    got, ref = got.float().cpu(), ref.float()
    err = ((got - ref).abs() / ref.abs().clamp_min(1.0)).max().item()
    return err <= tol, err


def _int_rows(b, n, gen):
    return (torch.randint(0, 2, (b, n), generator=gen) * 2 - 1).to(torch.float16)


def _int_w(n, k, gen):
    return torch.randint(-1, 2, (n, k), generator=gen).to(torch.float16)


def _rand(*shape, gen, std=1.0):
    return (torch.randn(*shape, generator=gen) * std).to(torch.float16)


def _tables(b, start, dev):
    cos, sin = rope_cos_sin(torch.arange(start, start + b), inv_freq(D, 1e6))
    return cos, sin, cos.to(dev), sin.to(dev)


@pytest.mark.parametrize("tiles", [False, True])
@pytest.mark.parametrize("batch", [1, 2, 3, 4])
@pytest.mark.parametrize("integer", [True, False])
def test_rms_qkv_rope_append(dev, batch, integer, tiles):
    gen = torch.Generator().manual_seed(10 + batch)
    width = (QH + 2 * KVH) * D
    if integer:
        x = _int_rows(batch, HIDDEN, gen)
        nw = torch.ones(HIDDEN, dtype=torch.float16)
        w = _int_w(width, HIDDEN, gen)
        bias = torch.randint(-3, 4, (width,), generator=gen).to(torch.float16)
    else:
        x = _rand(batch, HIDDEN, gen=gen)
        nw = (torch.rand(HIDDEN, generator=gen) + 0.5).to(torch.float16)
        w = _rand(width, HIDDEN, gen=gen, std=0.02)
        bias = _rand(width, gen=gen, std=0.1)
    cap, slot = 96, 37
    cos, sin, cos_d, sin_d = _tables(batch, 500, dev)
    kc0 = _rand(batch, KVH, cap, D, gen=gen)
    vc0 = _rand(batch, KVH, cap, D, gen=gen)
    kc, vc = kc0.to(dev), vc0.to(dev)
    q_out = torch.zeros(batch, QH, D, device=dev, dtype=torch.float16)
    print(f"[qkv] B={batch} integer={integer} tiles={tiles}", flush=True)
    wd = step_ops.pack_weight(w.to(dev), step_ops.PACK_ROPE) if tiles else w.to(dev)
    step_ops.rms_qkv_rope_append(x.to(dev), nw.to(dev), EPS, wd, bias.to(dev), cos_d, sin_d,
                                 kc, vc, torch.tensor([slot], device=dev), q_out)
    torch.cuda.synchronize()
    q, k, v = ost.qkv_rope16(x, nw, EPS, w, bias, cos, sin, QH, KVH, D)
    kc_ref, vc_ref = kc0.clone(), vc0.clone()
    kc_ref[:, :, slot] = k
    vc_ref[:, :, slot] = v
    if integer:
        assert torch.equal(q_out.cpu(), q)
        assert torch.equal(kc.cpu(), kc_ref)
        assert torch.equal(vc.cpu(), vc_ref)
    else:
        for name, got, ref in (("q", q_out, q), ("k", kc[:, :, slot], k), ("v", vc[:, :, slot], v)):
            ok, err = _close(got, ref)
            assert ok, f"{name}: {err:.3e}"
        other = [s for s in range(cap) if s != slot]
        assert torch.equal(kc.cpu()[:, :, other], kc0[:, :, other])
        assert torch.equal(vc.cpu()[:, :, other], vc0[:, :, other])


@pytest.mark.parametrize("tiles", [False, True])
def test_rms_qkv_gathers_embedding_rows_and_skips_out_of_range_slot(dev, tiles):
    gen = torch.Generator().manual_seed(3)
    batch, vocab = 3, 50
    width = (QH + 2 * KVH) * D
    embed = _int_rows(vocab, HIDDEN, gen)
    nw = torch.ones(HIDDEN, dtype=torch.float16)
    w = _int_w(width, HIDDEN, gen)
    token = torch.tensor([7, 0, 49])
    cos, sin, cos_d, sin_d = _tables(batch, 3, dev)
    cap = 64
    kc = torch.zeros(batch, KVH, cap, D, device=dev, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    q_out = torch.zeros(batch, QH, D, device=dev, dtype=torch.float16)
    hidden = torch.zeros(batch, HIDDEN, device=dev, dtype=torch.float16)
    wd = step_ops.pack_weight(w.to(dev), step_ops.PACK_ROPE) if tiles else w.to(dev)
    step_ops.rms_qkv_rope_append(embed.to(dev), nw.to(dev), EPS, wd, None, cos_d, sin_d,
                                 kc, vc, torch.tensor([cap], device=dev), q_out,
                                 token=token.to(dev), hidden_out=hidden)
    torch.cuda.synchronize()
    q, _, _ = ost.qkv_rope16(embed[token], nw, EPS, w, None, cos, sin, QH, KVH, D)
    assert torch.equal(q_out.cpu(), q)
    assert torch.equal(hidden.cpu(), embed[token])
    assert not bool(kc.any()) and not bool(vc.any())  # slot == cap: nothing written


@pytest.mark.parametrize("batch", [1, 2, 3, 4])
@pytest.mark.parametrize("k_dim,n", [(HIDDEN, HIDDEN), (INTER, HIDDEN), (200, 72), (6144, 96),
                                     (8192, 64), (1032, 97), (5128, 40)])
@pytest.mark.parametrize("integer", [True, False])
def test_gemv_residual(dev, batch, k_dim, n, integer):
    gen = torch.Generator().manual_seed(k_dim + n + batch)
    if integer:
        inp, w = _int_rows(batch, k_dim, gen), _int_w(n, k_dim, gen)
        res = torch.randint(-8, 9, (batch, n), generator=gen).to(torch.float16)
    else:
        inp, w, res = _rand(batch, k_dim, gen=gen), _rand(n, k_dim, gen=gen, std=0.02), _rand(batch, n, gen=gen)
    hidden = res.to(dev)
    print(f"[gemv] B={batch} K={k_dim} N={n} integer={integer}", flush=True)
    step_ops.gemv_residual(inp.to(dev), w.to(dev), hidden)
    torch.cuda.synchronize()
    ref = ost.residual16(res, inp, w)
    if integer:
        assert torch.equal(hidden.cpu(), ref)
    else:
        ok, err = _close(hidden, ref)
        assert ok, err


@pytest.mark.parametrize("tiles", [False, True])
@pytest.mark.parametrize("batch", [1, 2, 3, 4])
@pytest.mark.parametrize("integer", [True, False])
def test_rms_gate_up_swiglu(dev, batch, integer, tiles):
    gen = torch.Generator().manual_seed(20 + batch)
    if integer:
        x = _int_rows(batch, HIDDEN, gen)
        nw = torch.ones(HIDDEN, dtype=torch.float16)
        w = (_int_w(2 * INTER, HIDDEN, gen).float() / 64).to(torch.float16)  # keep silu in range
    else:
        x = _rand(batch, HIDDEN, gen=gen)
        nw = (torch.rand(HIDDEN, generator=gen) + 0.5).to(torch.float16)
        w = _rand(2 * INTER, HIDDEN, gen=gen, std=0.02)
    h = torch.zeros(batch, INTER, device=dev, dtype=torch.float16)
    print(f"[gate_up] B={batch} integer={integer} tiles={tiles}", flush=True)
    wd = step_ops.pack_weight(w.to(dev), step_ops.PACK_SWIGLU) if tiles else w.to(dev)
    step_ops.rms_gate_up_swiglu(x.to(dev), nw.to(dev), EPS, wd, h)
    torch.cuda.synchronize()
    ref = ost.swiglu16(x, nw, EPS, w)
    # silu's exp may differ in the last fp32 bit between the device and the CPU
    # library, so even exact gate/up sums allow one fp16 ulp after the product.
    ok, err = _close(h, ref, tol=2e-3 if integer else STEP_TOL)
    assert ok, err
    if integer:
        assert (h.cpu() == ref).float().mean().item() > 0.99


@pytest.mark.parametrize("batch,tiles", [(1, False), (3, False), (4, False), (1, True),
                                         (2, True), (3, True), (4, True)])
def test_rms_lm_head_and_argmax_step(dev, batch, tiles):
    """Exact integer logits and the first-maximum argmax on a planted tie, for
    the row kernel and the matrix-core kernel (packed weight)."""
    gen = torch.Generator().manual_seed(30 + batch)
    vocab = 5008 if tiles else 5003  # tiles: whole 16-row blocks; rows: not 4-row groups
    x = _int_rows(batch, HIDDEN, gen)
    nw = torch.ones(HIDDEN, dtype=torch.float16)
    w = _int_w(vocab, HIDDEN, gen)
    # Plant a tie for the maximum: rows 4000 and 1234 equal, both above the rest.
    w[1234] = torch.sign(x[0].float()).to(torch.float16)
    w[4000] = w[1234]
    logits = torch.zeros(batch, vocab, device=dev, dtype=torch.float16)
    keys = torch.zeros(batch, 96, device=dev, dtype=torch.long)
    print(f"[lm_head] B={batch} tiles={tiles}", flush=True)
    wd = w.to(dev)
    if tiles:
        wd = step_ops.pack_weight(wd, step_ops.PACK_PLAIN)
    step_ops.rms_lm_head(x.to(dev), nw.to(dev), EPS, wd, logits, keys)
    token = torch.full((batch,), -1, device=dev, dtype=torch.long)
    rows = torch.zeros(batch, 5, device=dev, dtype=torch.long)
    step = torch.tensor([2], device=dev)
    write = torch.tensor([40], device=dev)
    pos = torch.arange(batch, device=dev) + 10
    step_ops.argmax_step(keys, token, rows, step, write, pos)
    torch.cuda.synchronize()
    ref_logits, ref_idx = ost.lm_head_argmax(x, nw, EPS, w)
    assert torch.equal(logits.cpu(), ref_logits)
    assert torch.equal(token.cpu(), ref_idx)
    assert int(ref_idx[0]) == 1234
    assert torch.equal(rows.cpu()[:, 2], ref_idx)
    assert int(rows.cpu()[:, [0, 1, 3, 4]].abs().sum()) == 0
    assert int(step.item()) == 3 and int(write.item()) == 41
    assert torch.equal(pos.cpu(), torch.arange(batch) + 11)


@pytest.mark.parametrize("batch,tiles", [(2, False), (2, True), (4, True)])
def test_lm_head_random_logits_close(dev, batch, tiles):
    gen = torch.Generator().manual_seed(7)
    vocab = 151936
    x = _rand(batch, HIDDEN, gen=gen)
    nw = torch.ones(HIDDEN, dtype=torch.float16)
    w = _rand(vocab, HIDDEN, gen=gen, std=0.02)
    logits = torch.zeros(batch, vocab, device=dev, dtype=torch.float16)
    keys = torch.zeros(batch, step_ops.LM_BLOCKS, device=dev, dtype=torch.long)
    wd = w.to(dev)
    if tiles:
        wd = step_ops.pack_weight(wd, step_ops.PACK_PLAIN)
    step_ops.rms_lm_head(x.to(dev), nw.to(dev), EPS, wd, logits, keys)
    token = torch.zeros(batch, device=dev, dtype=torch.long)
    step_ops.argmax_step(keys, token)
    torch.cuda.synchronize()
    ref_logits, _ = ost.lm_head_argmax(x, nw, EPS, w)
    ok, err = _close(logits, ref_logits)
    assert ok, err
    # The device argmax is the first maximum of the device logits.
    assert torch.equal(token.cpu(), logits.float().cpu().argmax(-1))


@pytest.mark.parametrize("batch", [1, 2, 3, 4])
@pytest.mark.parametrize("splits", [1, 5, 18])
@pytest.mark.parametrize("tiles", [False, True])
def test_attn_merge_o_proj(dev, batch, splits, tiles):
    """Split-K partials merged in the o_proj prologue == oracle attention +
    o_proj, for the row kernel and the matrix-core kernel (packed weight)."""
    import oracle
    from qwenforge_amd import ops, workloads

    gen = torch.Generator().manual_seed(40 + batch + splits)
    case = workloads.decode_uniform(batch, 700, seed=splits, cap=768)
    c = case.to(dev)
    flash = ops.make_flash_scratch(batch, KVH, QH // KVH, 768, dev, splits=splits, fused=False)
    kv_last = torch.tensor([699], device=dev)
    w_o = _rand(HIDDEN, HIDDEN, gen=gen, std=0.02)
    res = _rand(batch, HIDDEN, gen=gen)
    hidden = res.to(dev)
    print(f"[merge+o_proj] B={batch} S={splits} tiles={tiles}", flush=True)
    ops.flash_decode_split(c.grouped, c.key_cache, c.value_cache, None, flash, kv_last=kv_last)
    wd = w_o.to(dev)
    step_ops.attn_merge_o_proj(flash, step_ops.pack_weight(wd, step_ops.PACK_PLAIN) if tiles else wd,
                               hidden)
    # The unfused pair: combine launch, then the plain GEMV.
    out = ops.flash_decode_combine(flash)
    hidden2 = res.to(dev)
    step_ops.gemv_residual(out.view(batch, HIDDEN), w_o.to(dev), hidden2)
    torch.cuda.synchronize()
    bias = torch.full((batch, 768), float(torch.finfo(torch.float16).min))
    bias[:, :700] = 0
    att = oracle.grouped_decode_attention(case.grouped, case.key_cache, case.value_cache, bias)
    ref = ost.residual16(res, att.to(torch.float16).reshape(batch, HIDDEN), w_o)
    ok, err = _close(hidden, ref)
    assert ok, err
    ok, err = _close(hidden, hidden2.cpu(), tol=2e-3)
    assert ok, err


@pytest.mark.parametrize("tiles", [False, True])
@pytest.mark.parametrize("batch", [1, 3, 4])
def test_rms_qkv_rope_positions_mode_equals_table_mode(dev, batch, tiles):
    """RoPE angles formed in the kernel from (pos, inv_freq) give exactly the
    outputs of the torch-built fp16 tables (SE:910-915), including far
    positions and a negative one."""
    from qwenforge_amd.rope import cos_sin, inv_freq as make_inv

    gen = torch.Generator().manual_seed(60 + batch)
    width = (QH + 2 * KVH) * D
    x = _rand(batch, HIDDEN, gen=gen).to(dev)
    nw = (torch.rand(HIDDEN, generator=gen) + 0.5).to(torch.float16).to(dev)
    w = _rand(width, HIDDEN, gen=gen, std=0.02).to(dev)
    bias = _rand(width, gen=gen, std=0.1).to(dev)
    pos = torch.tensor([0, 1023, 131071, -5][:batch], device=dev)
    inv = make_inv(D, 1e6, dev)
    cos, sin = cos_sin(pos, inv)
    cap, slot = 64, 9
    if tiles:
        w = step_ops.pack_weight(w, step_ops.PACK_ROPE)
    outs = []
    for mode in ("table", "positions"):
        kc = torch.zeros(batch, KVH, cap, D, device=dev, dtype=torch.float16)
        vc = torch.zeros_like(kc)
        q_out = torch.zeros(batch, QH, D, device=dev, dtype=torch.float16)
        if mode == "table":
            step_ops.rms_qkv_rope_append(x, nw, EPS, w, bias, cos, sin, kc, vc,
                                         torch.tensor([slot], device=dev), q_out)
        else:
            step_ops.rms_qkv_rope_append(x, nw, EPS, w, bias, None, None, kc, vc,
                                         torch.tensor([slot], device=dev), q_out,
                                         positions=(pos, inv))
        outs.append((q_out, kc, vc))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a.cpu(), b.cpu())


@pytest.mark.parametrize("layout", [0, 1, 2])
def test_pack_weight_tile_order(dev, layout):
    """Every 16-byte chunk of a packed weight is the row-major chunk the tile
    formula names (row maps plain, SwiGLU pairs, rotate-half pairs)."""
    n, k = 256, 96
    w = torch.arange(n * k, dtype=torch.float32).remainder(2039).to(torch.float16).view(n, k)
    tiles = step_ops.pack_weight(w.to(dev), layout)
    torch.cuda.synchronize()
    got = tiles.data.cpu().view(n // 16, k // 32, 64, 8)
    for rb in range(n // 16):
        for r in range(16):
            g, i = r >> 2, r & 3
            if layout == 1:
                j = 8 * rb + 2 * g + (i & 1)
                row = n // 2 + j if i & 2 else j
            elif layout == 2:
                row = 64 * (rb >> 2) + 8 * (rb & 3) + 2 * g + (i & 1) + (32 if i & 2 else 0)
            else:
                row = 16 * rb + r
            for kb in range(k // 32):
                for q in range(4):
                    want = w[row, 32 * kb + 8 * q: 32 * kb + 8 * q + 8]
                    assert torch.equal(got[rb, kb, 16 * q + r], want), (rb, r, kb, q)
