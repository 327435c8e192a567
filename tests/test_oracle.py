"""Pins for the CPU oracle: known answers, library routines, brute force and
invariants that a dropped term, wrong sign, wrong index or transposed operand
would break."""

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import whiteboard

GOLDEN = Path(__file__).resolve().parent / "golden"


def _rand(gen, *shape, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).half()


# ---------------------------------------------------------------- known answers

def test_whiteboard_kat_split_half_and_interleaved():
    kat = json.loads((GOLDEN / "whiteboard_kat.json").read_text())
    atol = kat["expected"]["atol"]
    last, logits = whiteboard.toy_forward(kat, "split_half")
    assert torch.allclose(logits, torch.tensor(kat["expected"]["split_half"]["logits"]), atol=atol)
    last_i, logits_i = whiteboard.toy_forward(kat, "interleaved")
    assert torch.allclose(logits_i, torch.tensor(kat["expected"]["interleaved"]["logits"]), atol=atol)
    assert torch.allclose(last_i, torch.tensor(kat["expected"]["interleaved"]["last_hidden"]), atol=atol)
    # The layouts are distinguishable, so the KAT pins rotate-half.
    assert not torch.allclose(logits, logits_i, atol=1e-2)


def test_whiteboard_kat_detects_wrong_causal_direction():
    """An anti-causal (upper-triangular) mask must miss the KAT."""
    kat = json.loads((GOLDEN / "whiteboard_kat.json").read_text())
    orig = oracle.attention.eager_attention

    def flipped(q, k, v, attention_mask=None, causal=False, acc_dtype=torch.float32):
        return orig(q.flip(-2), k.flip(-2), v.flip(-2), None, causal, acc_dtype).flip(-2)

    whiteboard.eager_attention = flipped
    try:
        _, logits = whiteboard.toy_forward(kat, "split_half")
    finally:
        whiteboard.eager_attention = orig
    assert not torch.allclose(logits, torch.tensor(kat["expected"]["split_half"]["logits"]), atol=1e-3)


# ---------------------------------------------------------------- attention

def test_eager_attention_matches_sdpa_gqa_causal():
    gen = torch.Generator().manual_seed(0)
    q = _rand(gen, 2, 14, 37, 64)
    k = _rand(gen, 2, 2, 37, 64)
    v = _rand(gen, 2, 2, 37, 64)
    got = oracle.eager_attention(q, k, v, causal=True, acc_dtype=torch.float64)
    ref = F.scaled_dot_product_attention(q.double(), k.double().repeat_interleave(7, 1),
                                         v.double().repeat_interleave(7, 1), is_causal=True)
    assert (got - ref).abs().max().item() < 1e-12


def test_eager_causal_is_bottom_right_for_decode_rows():
    gen = torch.Generator().manual_seed(1)
    q = _rand(gen, 1, 14, 3, 64)
    k = _rand(gen, 1, 2, 10, 64)
    v = _rand(gen, 1, 2, 10, 64)
    got = oracle.eager_attention(q, k, v, causal=True, acc_dtype=torch.float64)
    # Query row i (of 3) sees keys 0 .. 7 + i.
    for i in range(3):
        row = oracle.eager_attention(q[:, :, i:i + 1], k[:, :, :8 + i], v[:, :, :8 + i],
                                     acc_dtype=torch.float64)
        assert (got[:, :, i:i + 1] - row).abs().max().item() < 1e-12


def test_grouped_decode_equals_repeat_path_and_brute_force():
    gen = torch.Generator().manual_seed(2)
    b, cap = 2, 19
    grouped = _rand(gen, b, 2, 7, 64)
    kc = _rand(gen, b, 2, cap, 64)
    vc = _rand(gen, b, 2, cap, 64)
    bias = torch.zeros(b, cap, dtype=torch.float16)
    bias[0, 5:9] = oracle.FP16_MIN
    bias[1, 17:] = oracle.FP16_MIN
    got = oracle.grouped_decode_attention(grouped, kc, vc, bias, acc_dtype=torch.float64)
    # SE:636-643: the grouped form equals repeat_interleave with a key mask.
    q = grouped.reshape(b, 14, 1, 64)
    mask = (bias == 0)[:, None, None, :]
    rep = oracle.eager_attention(q, kc, vc, attention_mask=mask, acc_dtype=torch.float64)
    assert (got.reshape(b, 14, 1, 64) - rep).abs().max().item() < 1e-9
    # fp64 brute force, row by row.
    for bb in range(b):
        for h in range(2):
            rows = oracle.attention.brute_force_attention_fp64(
                grouped[bb, h].tolist(), kc[bb, h].tolist(), vc[bb, h].tolist(), 0.125,
                bias[bb].tolist())
            assert np.abs(np.array(rows) - got[bb, h].numpy()).max() < 1e-9


def test_grouped_decode_fp16_form_within_fp16_rounding_of_sdpa():
    """The reference's fp16 math form (SE:968-971): fp16 scores, fp32 softmax
    rounded to fp16, fp16 PV.  Against fp64 SDPA it is off by fp16 rounding
    only; uniform V and a single unmasked key are reproduced exactly."""
    gen = torch.Generator().manual_seed(31)
    b, kvh, g, cap = 2, 2, 7, 300
    q = _rand(gen, b, kvh, g, 64)
    k = _rand(gen, b, kvh, cap, 64)
    v = _rand(gen, b, kvh, cap, 64)
    bias = torch.zeros(b, cap, dtype=torch.float16)
    bias[1, 200:] = oracle.FP16_MIN
    got = oracle.grouped_decode_attention_fp16(q, k, v, bias)
    assert got.dtype == torch.float16
    mask = (bias == 0)[:, None, None, :].expand(b, kvh, g, cap)
    ref = F.scaled_dot_product_attention(q.double(), k.double(), v.double(), attn_mask=mask)
    err = (got.double() - ref).abs().max().item()
    assert err < 4e-3, err
    assert err > 0  # it really rounds (an fp32 path would sit near 1e-6)
    row = _rand(gen, 64)
    uni = row.expand(b, kvh, cap, 64).contiguous()
    assert torch.equal(oracle.grouped_decode_attention_fp16(q, k, uni, bias),
                       row.expand(b, kvh, g, 64))
    one = torch.full((b, cap), oracle.FP16_MIN, dtype=torch.float16)
    one[:, 17] = 0
    assert torch.equal(oracle.grouped_decode_attention_fp16(q, k, v, one),
                       v[:, :, 17:18].expand(b, kvh, g, 64))


def test_eager_prefill_fp16_form_within_fp16_rounding_of_sdpa():
    """The reference's fp16 eager prefill (SE:579-599): against fp64 causal
    SDPA with K/V repeated it is off by fp16 rounding only; the first query
    row equals V[0] of its kv head exactly and uniform V is reproduced
    exactly; a dropped causal mask or a transposed head mapping fails."""
    gen = torch.Generator().manual_seed(32)
    s = 96
    q = _rand(gen, 1, 14, s, 64)
    k = _rand(gen, 1, 2, s, 64)
    v = _rand(gen, 1, 2, s, 64)
    got = oracle.eager_attention_fp16(q, k, v)
    assert got.dtype == torch.float16
    ref = F.scaled_dot_product_attention(q.double(), k.double().repeat_interleave(7, 1),
                                         v.double().repeat_interleave(7, 1), is_causal=True)
    err = (got.double() - ref).abs().max().item()
    assert 0 < err < 4e-3, err
    assert torch.equal(got[:, :, 0], v[:, :, 0].repeat_interleave(7, 1))
    row = _rand(gen, 64)
    uni = row.expand(1, 2, s, 64).contiguous()
    assert torch.equal(oracle.eager_attention_fp16(q, k, uni), row.expand(1, 14, s, 64))
    no_mask = oracle.eager_attention_fp16(q, k, v, causal=False)
    assert (no_mask.double() - ref).abs().max().item() > 0.1
    swapped = F.scaled_dot_product_attention(q.double(), k.double().repeat(1, 7, 1, 1),
                                             v.double().repeat(1, 7, 1, 1), is_causal=True)
    assert (got.double() - swapped).abs().max().item() > 0.1


def test_grouped_decode_head_mapping_is_h_div_g():
    """Query head h of the flattened (B, 14) layout must read kv head h // 7."""
    gen = torch.Generator().manual_seed(3)
    grouped = _rand(gen, 1, 2, 7, 64)
    kc = _rand(gen, 1, 2, 11, 64)
    vc = _rand(gen, 1, 2, 11, 64)
    got = oracle.grouped_decode_attention(grouped, kc, vc, acc_dtype=torch.float64)
    q = grouped.reshape(1, 14, 1, 64)
    ref = F.scaled_dot_product_attention(q.double(), kc.double().repeat_interleave(7, 1),
                                         vc.double().repeat_interleave(7, 1))
    assert (got.reshape(1, 14, 1, 64) - ref).abs().max().item() < 1e-12


# ---------------------------------------------------------------- split-K algebra

@pytest.mark.parametrize("splits", [1, 2, 3, 7, 32, 40])
def test_split_combine_independent_of_split_count(splits):
    gen = torch.Generator().manual_seed(4)
    grouped = _rand(gen, 2, 2, 7, 64)
    kc = _rand(gen, 2, 2, 37, 64)
    vc = _rand(gen, 2, 2, 37, 64)
    bias = torch.zeros(2, 37, dtype=torch.float16)
    bias[1, 20:] = oracle.FP16_MIN
    got = oracle.flash_decode(grouped, kc, vc, bias, splits, acc_dtype=torch.float64)
    ref = oracle.grouped_decode_attention(grouped, kc, vc, bias, acc_dtype=torch.float64)
    assert (got - ref).abs().max().item() < 1e-12


def test_fully_masked_and_empty_splits_contribute_nothing():
    gen = torch.Generator().manual_seed(5)
    grouped = _rand(gen, 1, 2, 7, 64)
    kc = _rand(gen, 1, 2, 64, 64)
    vc = _rand(gen, 1, 2, 64, 64)
    bias = torch.full((1, 64), oracle.FP16_MIN, dtype=torch.float16)
    bias[0, :10] = 0
    acc, m, l = oracle.split_partials(grouped, kc, vc, bias, 8, acc_dtype=torch.float64)
    # Split 3 is fully masked: finite m near fp16-min, positive l, zero weight.
    assert bool((m[:, :, 3] < -6e4).all()) and bool((l[:, :, 3] > 0).all())
    out = oracle.combine_partials(acc, m, l)
    ref = oracle.grouped_decode_attention(grouped, kc[:, :, :10], vc[:, :, :10], None,
                                          acc_dtype=torch.float64)
    assert (out - ref).abs().max().item() < 1e-12
    # Empty splits (upper bound below the split start) have m = -inf, l = 0.
    acc2, m2, l2 = oracle.split_partials(grouped, kc, vc, None, 8, upper=12, acc_dtype=torch.float64)
    assert bool(torch.isinf(m2[:, :, 2:]).all()) and float(l2[:, :, 2:].abs().sum()) == 0.0
    out2 = oracle.combine_partials(acc2, m2, l2)
    ref2 = oracle.grouped_decode_attention(grouped, kc[:, :, :12], vc[:, :, :12], None,
                                           acc_dtype=torch.float64)
    assert (out2 - ref2).abs().max().item() < 1e-12


def test_special_cases_single_key_uniform_v_zero_k():
    gen = torch.Generator().manual_seed(6)
    grouped = _rand(gen, 1, 2, 7, 64)
    kc = _rand(gen, 1, 2, 50, 64)
    vc = _rand(gen, 1, 2, 50, 64)
    bias = torch.full((1, 50), oracle.FP16_MIN, dtype=torch.float16)
    bias[0, 31] = 0
    out = oracle.flash_decode(grouped, kc, vc, bias, 4, acc_dtype=torch.float64)
    assert (out - vc[:, :, 31:32].double()).abs().max().item() < 1e-12
    uni = vc[:, :, :1].expand(-1, -1, 50, -1).contiguous()
    out = oracle.flash_decode(grouped, kc, uni, None, 4, acc_dtype=torch.float64)
    assert (out - uni[:, :, :1].double()).abs().max().item() < 1e-12
    out = oracle.flash_decode(grouped, torch.zeros_like(kc), vc, None, 5, acc_dtype=torch.float64)
    assert (out - vc.double().mean(dim=2, keepdim=True)).abs().max().item() < 1e-12


def test_key_permutation_invariance():
    gen = torch.Generator().manual_seed(7)
    grouped = _rand(gen, 1, 2, 7, 64)
    kc = _rand(gen, 1, 2, 45, 64)
    vc = _rand(gen, 1, 2, 45, 64)
    bias = torch.zeros(1, 45, dtype=torch.float16)
    bias[0, ::3] = oracle.FP16_MIN
    perm = torch.randperm(45, generator=gen)
    a = oracle.flash_decode(grouped, kc, vc, bias, 3, acc_dtype=torch.float64)
    b = oracle.flash_decode(grouped, kc[:, :, perm], vc[:, :, perm], bias[:, perm], 6,
                            acc_dtype=torch.float64)
    assert (a - b).abs().max().item() < 1e-12


# ---------------------------------------------------------------- causal prefill

def test_causal_prefill_rows_equal_decode_over_prefix():
    gen = torch.Generator().manual_seed(8)
    q = _rand(gen, 1, 14, 23, 64)
    k = _rand(gen, 1, 2, 23, 64)
    v = _rand(gen, 1, 2, 23, 64)
    got = oracle.causal_prefill(q, k, v, acc_dtype=torch.float64)
    assert (got[:, :, 0] - v.double().repeat_interleave(7, 1)[:, :, 0]).abs().max().item() < 1e-12
    for i in (1, 9, 22):
        grouped = q[:, :, i].reshape(1, 2, 7, 64)
        row = oracle.grouped_decode_attention(grouped, k[:, :, :i + 1], v[:, :, :i + 1],
                                              acc_dtype=torch.float64)
        assert (got[:, :, i] - row.reshape(1, 14, 64)).abs().max().item() < 1e-12
    ref = F.scaled_dot_product_attention(q.double(), k.double().repeat_interleave(7, 1),
                                         v.double().repeat_interleave(7, 1), is_causal=True)
    assert (got - ref).abs().max().item() < 1e-12


# ---------------------------------------------------------------- RoPE

def test_inv_freq_closed_form():
    got = oracle.inv_freq(64, 1e6).double()
    ref = torch.tensor([1e6 ** (-(2 * i) / 64) for i in range(32)], dtype=torch.float64)
    assert ((got - ref).abs() / ref).max().item() < 4e-7


def test_rope_fp16_rounding_matches_torch_and_numpy_half_arithmetic():
    gen = torch.Generator().manual_seed(9)
    x = (torch.randn(4, 3, 5, 64, generator=gen) * 4).half()
    pos = torch.randint(0, 40000, (5,), generator=gen)
    cos, sin = oracle.rope_cos_sin(pos, oracle.inv_freq(64, 1e6))
    got = oracle.apply_rope_fp16(x, cos, sin)
    # torch CPU half arithmetic, op by op (SE:927-928).
    ref_t = x * cos + oracle.rotate_half(x) * sin
    assert torch.equal(got, ref_t)
    # numpy float16 arithmetic (an independent correctly rounded implementation).
    xn, cn, sn = x.numpy(), cos.numpy(), sin.numpy()
    rot = np.concatenate((-xn[..., 32:], xn[..., :32]), axis=-1)
    ref_n = (xn * cn) + (rot * sn)
    assert np.array_equal(got.numpy().view(np.uint16), ref_n.astype(np.float16).view(np.uint16))


def test_rope_rotate_half_sign_and_halves():
    x = torch.arange(64, dtype=torch.float32)
    r = oracle.rotate_half(x)
    assert torch.equal(r[:32], -x[32:]) and torch.equal(r[32:], x[:32])


def test_rope_position_zero_identity_and_norm_preservation():
    gen = torch.Generator().manual_seed(10)
    x = _rand(gen, 3, 64)
    cos, sin = oracle.rope_cos_sin(torch.zeros(3, dtype=torch.long), oracle.inv_freq(64, 1e6))
    assert torch.equal(oracle.apply_rope_fp16(x, cos, sin), x)
    # In fp64 the rotation preserves each (d, d+32) pair's norm.
    pos = torch.tensor([5, 777, 32767])
    f = pos.double()[:, None] * oracle.inv_freq(64, 1e6).double()
    emb = torch.cat((f, f), -1)
    y = oracle.rope.apply_rope_fp32(x.double(), emb.cos(), emb.sin())
    pair = lambda t: t[:, :32] ** 2 + t[:, 32:] ** 2  # noqa: E731
    assert (pair(y) - pair(x.double())).abs().max().item() < 1e-9


# ---------------------------------------------------------------- append / slots

def test_append_decode_brute_force():
    gen = torch.Generator().manual_seed(11)
    kc = _rand(gen, 3, 2, 9, 64)
    vc = _rand(gen, 3, 2, 9, 64)
    k = _rand(gen, 3, 2, 1, 64)
    v = _rand(gen, 3, 2, 1, 64)
    ekc, evc = kc.clone(), vc.clone()
    for b in range(3):
        for h in range(2):
            ekc[b, h, 4] = k[b, h, 0]
            evc[b, h, 4] = v[b, h, 0]
    gkc, gvc = oracle.append_decode(kc.clone(), vc.clone(), k, v, torch.tensor([4]))
    assert torch.equal(gkc, ekc) and torch.equal(gvc, evc)


def test_append_prefill_brute_force():
    gen = torch.Generator().manual_seed(12)
    kc = torch.zeros(2, 2, 20, 64, dtype=torch.float16)
    k = _rand(gen, 2, 2, 7, 64)
    v = _rand(gen, 2, 2, 7, 64)
    gkc, gvc = oracle.append_prefill(kc.clone(), kc.clone(), k, v, start=5)
    for s in range(20):
        if 5 <= s < 12:
            assert torch.equal(gkc[:, :, s], k[:, :, s - 5]) and torch.equal(gvc[:, :, s], v[:, :, s - 5])
        else:
            assert float(gkc[:, :, s].abs().sum()) == 0.0


def test_paged_identity_table_is_a_reshape():
    """Closed form: with table[b, j] = b * ppr + j the pool is the dense cache
    cut into pages, (B, KVH, ppr, P, D) -> (B * ppr, KVH, P, D)."""
    gen = torch.Generator().manual_seed(21)
    b, kvh, ppr, page, d = 3, 2, 4, 64, 64
    dense = _rand(gen, b, kvh, ppr * page, d)
    table = torch.arange(b * ppr, dtype=torch.int32).view(b, ppr)
    full = [ppr * page] * b
    pool = oracle.dense_to_pages(dense, table, full, b * ppr, page)
    closed = dense.view(b, kvh, ppr, page, d).permute(0, 2, 1, 3, 4).reshape(b * ppr, kvh, page, d)
    assert torch.equal(pool, closed)
    assert torch.equal(oracle.pages_to_dense(closed, table, full, ppr * page), dense)
    assert oracle.paged_location(table, 1, 130, page) == (1 * ppr + 2, 2)


def test_paged_gather_scatter_inverse_on_random_tables():
    gen = torch.Generator().manual_seed(22)
    b, kvh, ppr, page, d, n_pages = 3, 2, 3, 64, 64, 11
    lengths = [150, 64, 1]
    perm = torch.randperm(n_pages, generator=gen).to(torch.int32)
    table = perm[: b * ppr].view(b, ppr)
    dense = _rand(gen, b, kvh, ppr * page, d)
    for r, n in enumerate(lengths):
        dense[r, :, n:] = 0
    pool = oracle.dense_to_pages(dense, table, lengths, n_pages, page)
    assert torch.equal(oracle.pages_to_dense(pool, table, lengths, ppr * page), dense)
    # Pages no row maps stay zero.
    unused = perm[b * ppr:].tolist()
    assert float(pool[unused].abs().sum()) == 0.0


def test_append_rows_brute_force():
    gen = torch.Generator().manual_seed(23)
    kc = _rand(gen, 3, 2, 9, 64)
    vc = _rand(gen, 3, 2, 9, 64)
    k = _rand(gen, 3, 2, 1, 64)
    v = _rand(gen, 3, 2, 1, 64)
    slots = [4, 0, 9]  # row 2 is out of range: nothing written
    ekc, evc = kc.clone(), vc.clone()
    for r, s in enumerate(slots[:2]):
        ekc[r, :, s] = k[r, :, 0]
        evc[r, :, s] = v[r, :, 0]
    gkc, gvc = oracle.append_rows(kc.clone(), vc.clone(), k, v, torch.tensor(slots))
    assert torch.equal(gkc, ekc) and torch.equal(gvc, evc)
    # One shared slot reduces to the reference's index_copy_ append.
    skc, svc = oracle.append_rows(kc.clone(), vc.clone(), k, v, torch.tensor([5, 5, 5]))
    rkc, rvc = oracle.append_decode(kc.clone(), vc.clone(), k, v, torch.tensor([5]))
    assert torch.equal(skc, rkc) and torch.equal(svc, rvc)


def test_capacity_rule_brute_force():
    for p in range(1, 140, 7):
        for n in range(0, 70, 9):
            raw = max(p + max(n - 1, 0), p)
            assert oracle.capacity(p, n, graph=False) == raw
            rounded = oracle.capacity(p, n)
            assert rounded % 64 == 0 and rounded - 64 < raw <= rounded
    assert oracle.capacity(1024, 128) == 1152


def test_decode_slots_and_bias_holes():
    slots = oracle.decode_slots(10, 5)
    assert slots == [10, 11, 12, 13]
    bias = oracle.decode_bias([7, 10], 10, 64, steps_done=3)
    valid0 = (bias[0] == 0).nonzero().flatten().tolist()
    assert valid0 == list(range(7)) + [10, 11, 12]
    valid1 = (bias[1] == 0).nonzero().flatten().tolist()
    assert valid1 == list(range(13))
    assert float(bias[0, 8]) == oracle.FP16_MIN


def test_oracle_catches_a_planted_transpose():
    """A plausible mistake (V used transposed) must fail the library check."""
    gen = torch.Generator().manual_seed(13)
    q = _rand(gen, 1, 2, 64, 64)
    k = _rand(gen, 1, 2, 64, 64)
    v = _rand(gen, 1, 2, 64, 64)
    good = oracle.causal_prefill(q, k, v, acc_dtype=torch.float64)
    bad = oracle.causal_prefill(q, k, v.transpose(-2, -1).contiguous(), acc_dtype=torch.float64)
    ref = F.scaled_dot_product_attention(q.double(), k.double(), v.double(), is_causal=True)
    assert (good - ref).abs().max().item() < 1e-12
    assert (bad - ref).abs().max().item() > 1e-2
    assert math.isfinite(good.abs().max().item())


# ---------------------------------------------------------------- model step

def test_model_decode_step_continues_prefill():
    """Decoding token S over a prefilled cache reproduces prefill of S+1 tokens."""
    import oracle.model as om
    from qwenforge_amd.model import Qwen2Config, init_weights

    cfg = Qwen2Config(layers=2, vocab=512, hidden=256, heads=4, kv_heads=2, head_dim=64,
                      intermediate=256)
    w = init_weights(cfg, "cpu", seed=3, std=0.1)
    ids = torch.randint(0, cfg.vocab, (2, 12), generator=torch.Generator().manual_seed(4))
    full, _ = om.prefill(w, cfg, ids, 64)
    _, caches = om.prefill(w, cfg, ids[:, :11], 64)
    step = om.decode_step(w, cfg, ids[:, 11], torch.full((2,), 11), caches, 11)
    assert (full - step).abs().max().item() < 1e-4
