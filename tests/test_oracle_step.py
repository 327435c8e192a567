"""Pins of ``oracle.step`` (the decode-step projections with fp16 rounding points).

Each check compares the restatement with an independent evaluation: torch-CPU
half arithmetic (every half op computes in fp32 and rounds once), fp64 math,
or a hand-built case whose answer is known in closed form.
"""

import torch
import torch.nn.functional as F

import oracle.step as os_
from oracle.rope import apply_rope_fp16, inv_freq, rope_cos_sin


def _h(*shape, gen, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(torch.float16)


def test_residual16_matches_torch_half_add():
    gen = torch.Generator().manual_seed(0)
    res, inp, w = _h(3, 96, gen=gen), _h(3, 160, gen=gen), _h(96, 160, gen=gen, scale=0.05)
    lin = (inp.double() @ w.double().T).to(torch.float16)  # fp64 sum, one rounding
    want = res + lin                                       # torch half add (SE:974)
    got = os_.residual16(res, inp, w)
    # fp32 vs fp64 accumulation may move a rounding boundary by one ulp, nothing more.
    diff = (got.float() - want.float()).abs()
    ulp = torch.finfo(torch.float16).eps * want.float().abs().clamp_min(2 ** -14)
    assert bool((diff <= 2 * ulp).all())
    assert (got == want).float().mean().item() > 0.97


def test_swiglu16_matches_torch_half_ops():
    gen = torch.Generator().manual_seed(1)
    x = _h(2, 64, gen=gen)
    nw = torch.ones(64, dtype=torch.float16)
    w = _h(2 * 48, 64, gen=gen, scale=0.2)
    got = os_.swiglu16(x, nw, 1e-6, w)
    gu = os_.linear16(os_.rms_norm16(x, nw, 1e-6), w)
    g, u = gu.chunk(2, dim=-1)
    want = F.silu(g) * u  # the reference's literal ops on fp16 tensors (SE:665-666)
    assert torch.equal(got, want)


def test_rms_norm16_against_fp64_and_eager_form():
    gen = torch.Generator().manual_seed(2)
    x = _h(4, 896, gen=gen)
    w = _h(896, gen=gen).abs() + 0.5
    got = os_.rms_norm16(x, w, 1e-6).float()
    xd = x.double()
    want = xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-6) * w.double()
    assert ((got.double() - want).abs() <= want.abs() * 2 ** -10 + 1e-7).all()
    # Unit weight: equal to the eager two-rounding _rms_norm (SE:530-535).
    ones = torch.ones(896, dtype=torch.float16)
    xf = x.float()
    eager = (xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + 1e-6)).to(torch.float16) * ones
    assert torch.equal(os_.rms_norm16(x, ones, 1e-6), eager)


def test_qkv_rope16_split_order_and_rope():
    """Identity-like projection: q, k, v are slices of the normalised row."""
    qh, kvh, d = 2, 1, 64
    width = (qh + 2 * kvh) * d          # 256
    x = torch.tensor([[1.0, -1.0] * (width // 2)], dtype=torch.float16)
    nw = torch.arange(1, width + 1, dtype=torch.float32).remainder(5).add(1).to(torch.float16)
    w = torch.eye(width, dtype=torch.float16)
    bias = torch.arange(width, dtype=torch.float32).remainder(3).to(torch.float16)
    cos, sin = rope_cos_sin(torch.tensor([7]), inv_freq(d, 1e6))
    q, k, v = os_.qkv_rope16(x, nw, 1e-6, w, bias, cos, sin, qh, kvh, d)
    # |x| = 1 everywhere: rsqrt(1 + 1e-6) rounds away, so normalised = x * nw exactly.
    proj = (x.float() * nw.float() + bias.float()).to(torch.float16)
    assert torch.equal(v[0, 0], proj[0, 3 * d:4 * d])
    assert torch.equal(q[0, 1], apply_rope_fp16(proj[0, d:2 * d], cos[0], sin[0]))
    assert torch.equal(k[0, 0], apply_rope_fp16(proj[0, 2 * d:3 * d], cos[0], sin[0]))


def test_lm_head_argmax_first_maximum_on_ties():
    gen = torch.Generator().manual_seed(3)
    x = _h(3, 32, gen=gen)
    nw = torch.ones(32, dtype=torch.float16)
    w = _h(50, 32, gen=gen)
    w[17] = w[40]  # row 40 duplicates row 17: any maximum there must report 17
    w[40] *= 1
    logits, idx = os_.lm_head_argmax(x, nw, 1e-6, w)
    assert torch.equal(idx, logits.float().argmax(-1))  # torch.argmax: first maximum
    x2 = torch.zeros(2, 32, dtype=torch.float16)
    x2[:, 0] = 1
    w2 = torch.zeros(50, 32, dtype=torch.float16)
    w2[[9, 21, 33], 0] = 2.0
    _, idx2 = os_.lm_head_argmax(x2, nw, 1e-6, w2)
    assert idx2.tolist() == [9, 9]
