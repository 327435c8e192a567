"""Paged KV cache (include/qf_paged.h) against the dense path and the oracle.

The paged kernels are the dense kernels with cache rows found through a block
table, so on the same data they must agree with the dense entry points bit
for bit (same values, same summation order).  Each test also checks the
oracle directly: attention within 2e-3 of the fp32 oracle, appended rows
bit-exact (``oracle.dense_to_pages`` / ``pages_to_dense`` state the layout).
Page tables are random permutations, so a page-index mistake moves data.
"""

import pytest
import torch

import oracle
import oracle.step as ost
from oracle.rope import inv_freq, rope_cos_sin
from qwenforge_amd import ops, paged, step_ops

pytestmark = pytest.mark.gpu
TOL = 2e-3
QH, KVH, G, D = 14, 2, 7, 64


def _err(a, b):
    return (a.float().cpu() - b.float().cpu()).abs().max().item()


def _table(gen, b, ppr, n_pages):
    perm = torch.randperm(n_pages, generator=gen).to(torch.int32)
    return perm[: b * ppr].view(b, ppr).clone()


def _paged_copy(dense, table, lengths, n_pages, page, dev):
    k = oracle.dense_to_pages(dense, table, lengths, n_pages, page)
    return k.to(dev)


@pytest.mark.parametrize("page", [64, 256])
@pytest.mark.parametrize("lengths,splits", [([300, 1, 517], 4), ([700, 64, 129, 1000], 16),
                                            ([450], 1), ([2000, 33], 32)])
def test_decode_paged_matches_dense_and_oracle(dev, page, lengths, splits):
    gen = torch.Generator().manual_seed(sum(lengths) + page)
    b = len(lengths)
    ppr = (max(lengths) + page - 1) // page
    cap = ppr * page
    n_pages = b * ppr + 3
    kd = torch.randn(b, KVH, cap, D, generator=gen).half()
    vd = torch.randn(b, KVH, cap, D, generator=gen).half()
    for r, n in enumerate(lengths):
        kd[r, :, n:] = 0
        vd[r, :, n:] = 0
    table = _table(gen, b, ppr, n_pages)
    kp = _paged_copy(kd, table, lengths, n_pages, page, dev)
    vp = _paged_copy(vd, table, lengths, n_pages, page, dev)
    q = torch.randn(b, KVH, G, D, generator=gen).half()
    last = torch.tensor([n - 1 for n in lengths], device=dev)
    print(f"[paged decode] page={page} lengths={lengths} splits={splits}", flush=True)
    for fused in (False, True):
        if fused and splits == 1:
            continue
        flash_p = ops.make_flash_scratch(b, KVH, G, cap, dev, splits=splits, fused=fused)
        flash_d = ops.make_flash_scratch(b, KVH, G, cap, dev, splits=splits, fused=fused)
        got = paged.flash_decode_attention_paged(q.to(dev), kp, vp, table.to(dev), None, flash_p,
                                                 kv_last=last)
        ref = ops.flash_decode_attention(q.to(dev), kd.to(dev), vd.to(dev), None, flash_d,
                                         kv_last=last)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), ref.cpu()), f"fused={fused}"
    bias = torch.full((b, cap), oracle.FP16_MIN, dtype=torch.float16)
    for r, n in enumerate(lengths):
        bias[r, :n] = 0
    want = oracle.grouped_decode_attention(q, kd, vd, bias)
    assert _err(got, want) <= TOL


def test_decode_paged_window_reload_long_split(dev):
    """One split of 40,000 keys at 16 waves: each wave walks 79 tiles, so its
    page-id window (64 tiles) is reloaded once; a bias rides along."""
    gen = torch.Generator().manual_seed(5)
    page, n = 64, 40000
    ppr = (n + page - 1) // page
    n_pages = ppr + 5
    kd = torch.randn(1, KVH, ppr * page, D, generator=gen).half()
    vd = torch.randn(1, KVH, ppr * page, D, generator=gen).half()
    kd[:, :, n:] = 0
    vd[:, :, n:] = 0
    table = _table(gen, 1, ppr, n_pages)
    kp = _paged_copy(kd, table, [n], n_pages, page, dev)
    vp = _paged_copy(vd, table, [n], n_pages, page, dev)
    q = torch.randn(1, KVH, G, D, generator=gen).half()
    bias = torch.zeros(1, ppr * page, dtype=torch.float16)
    bias[:, n:] = oracle.FP16_MIN
    bias[:, ::97] = oracle.FP16_MIN
    last = torch.tensor([n - 1], device=dev)
    print("[paged decode] window reload, 40000 keys", flush=True)
    for splits in (1, 2):
        flash_p = ops.make_flash_scratch(1, KVH, G, ppr * page, dev, splits=splits)
        flash_d = ops.make_flash_scratch(1, KVH, G, ppr * page, dev, splits=splits)
        got = paged.flash_decode_attention_paged(q.to(dev), kp, vp, table.to(dev), bias.to(dev),
                                                 flash_p, kv_last=last)
        ref = ops.flash_decode_attention(q.to(dev), kd.to(dev), vd.to(dev), bias.to(dev), flash_d,
                                         kv_last=last)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), ref.cpu()), f"splits={splits}"
    assert _err(got, oracle.grouped_decode_attention(q, kd, vd, bias)) <= TOL


def test_rope_append_paged_per_row_slots(dev):
    gen = torch.Generator().manual_seed(7)
    b, page, ppr = 4, 64, 3
    n_pages = b * ppr + 2
    table = _table(gen, b, ppr, n_pages)
    slots = [0, 191, 70, -1]  # the last row writes nothing
    pos = torch.tensor([5, 191, 70, 3])
    cos, sin = rope_cos_sin(pos, inv_freq(D, 1e6))
    q = torch.randn(b, QH, 1, D, generator=gen).half()
    k = torch.randn(b, KVH, 1, D, generator=gen).half()
    v = torch.randn(b, KVH, 1, D, generator=gen).half()
    kp0 = torch.randn(n_pages, KVH, page, D, generator=gen).half()
    vp0 = torch.randn(n_pages, KVH, page, D, generator=gen).half()
    kp, vp = kp0.to(dev), vp0.to(dev)
    print("[paged rope_append]", flush=True)
    q_rot = paged.rope_append_paged(q.to(dev), k.to(dev), v.to(dev), cos.to(dev), sin.to(dev),
                                    kp, vp, table.to(dev), torch.tensor(slots, device=dev))
    torch.cuda.synchronize()
    assert torch.equal(q_rot.cpu(), oracle.apply_rope_fp16(q, cos.view(b, 1, 1, D), sin.view(b, 1, 1, D)))
    k_rot = oracle.apply_rope_fp16(k, cos.view(b, 1, 1, D), sin.view(b, 1, 1, D))
    kp_ref, vp_ref = kp0.clone(), vp0.clone()
    for r, s in enumerate(slots):
        if s < 0:
            continue
        p, row = oracle.paged_location(table, r, s, page)
        kp_ref[p, :, row] = k_rot[r, :, 0]
        vp_ref[p, :, row] = v[r, :, 0]
    assert torch.equal(kp.cpu(), kp_ref)
    assert torch.equal(vp.cpu(), vp_ref)


@pytest.mark.parametrize("page", [64, 128])
@pytest.mark.parametrize("lengths", [[1, 65, 200, 513], [130], [4200]])
def test_prefill_varlen_paged_matches_dense(dev, page, lengths):
    """Packed rows prefilled into pages: the output equals the dense varlen
    prefill bit for bit, the pages hold exactly the dense cache rows, and the
    rows match the per-row oracle.  4200 tokens walk 66 key tiles, past one
    64-page id window."""
    gen = torch.Generator().manual_seed(sum(lengths) + page)
    b, total = len(lengths), sum(lengths)
    q = torch.randn(total, QH, D, generator=gen).half()
    k = torch.randn(total, KVH, D, generator=gen).half()
    v = torch.randn(total, KVH, D, generator=gen).half()
    pos = torch.cat([torch.arange(n) for n in lengths])
    cos, sin = rope_cos_sin(pos, inv_freq(D, 1e6))
    starts = [0]
    for n in lengths:
        starts.append(starts[-1] + n)
    ppr = (max(lengths) + page - 1) // page
    cap = ppr * page
    n_pages = b * ppr + 1
    table = _table(gen, b, ppr, n_pages)
    cu = torch.tensor(starts, dtype=torch.int32, device=dev)
    kp = torch.zeros(n_pages, KVH, page, D, dtype=torch.float16, device=dev)
    vp = torch.zeros_like(kp)
    kc = torch.zeros(b, KVH, cap, D, dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    qd, kd, vd, cd, sd = q.to(dev), k.to(dev), v.to(dev), cos.to(dev), sin.to(dev)
    print(f"[paged prefill] page={page} lengths={lengths}", flush=True)
    got = paged.prefill_varlen_paged(qd, kd, vd, cu, max(lengths), cd, sd, kp, vp, table.to(dev), 0)
    ref = ops.prefill_varlen(qd, kd, vd, cu, max(lengths), cd, sd, kc, vc, 0)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), ref.cpu())
    assert torch.equal(kp.cpu(), oracle.dense_to_pages(kc.cpu(), table, lengths, n_pages, page))
    assert torch.equal(vp.cpu(), oracle.dense_to_pages(vc.cpu(), table, lengths, n_pages, page))
    got = got.cpu()
    for i, n in enumerate(lengths[:2]):
        sl = slice(starts[i], starts[i + 1])
        q_rot = oracle.apply_rope_fp16(q[sl].transpose(0, 1), cos[sl], sin[sl])
        k_rot = oracle.apply_rope_fp16(k[sl].transpose(0, 1), cos[sl], sin[sl])
        want = oracle.causal_prefill(q_rot[None], k_rot[None], v[sl].transpose(0, 1)[None])[0]
        assert _err(got[sl].transpose(0, 1), want) <= TOL, f"row {i}"


def test_prefill_varlen_paged_at_offset_without_rope(dev):
    """A chunk written at start_pos 128 of each row, K stored as given."""
    gen = torch.Generator().manual_seed(9)
    lengths, page, start = [40, 100], 64, 128
    b, total = len(lengths), sum(lengths)
    q = torch.randn(total, QH, D, generator=gen).half()
    k = torch.randn(total, KVH, D, generator=gen).half()
    v = torch.randn(total, KVH, D, generator=gen).half()
    ppr = 4
    n_pages = b * ppr
    table = _table(gen, b, ppr, n_pages)
    cu = torch.tensor([0, 40, 140], dtype=torch.int32, device=dev)
    kp = torch.zeros(n_pages, KVH, page, D, dtype=torch.float16, device=dev)
    vp = torch.zeros_like(kp)
    out = paged.prefill_varlen_paged(q.to(dev), k.to(dev), v.to(dev), cu, 100, None, None, kp, vp,
                                     table.to(dev), start)
    torch.cuda.synchronize()
    dense_k = torch.zeros(b, KVH, ppr * page, D, dtype=torch.float16)
    dense_v = torch.zeros_like(dense_k)
    for i, (s0, n) in enumerate(((0, 40), (40, 100))):
        dense_k[i, :, start:start + n] = k[s0:s0 + n].transpose(0, 1)
        dense_v[i, :, start:start + n] = v[s0:s0 + n].transpose(0, 1)
        want = oracle.causal_prefill(q[s0:s0 + n].transpose(0, 1)[None], k[s0:s0 + n].transpose(0, 1)[None],
                                     v[s0:s0 + n].transpose(0, 1)[None])[0]
        assert _err(out.cpu()[s0:s0 + n].transpose(0, 1), want) <= TOL
    full = [start + n for n in lengths]
    assert torch.equal(oracle.pages_to_dense(kp.cpu(), table, full, ppr * page), dense_k)
    assert torch.equal(oracle.pages_to_dense(vp.cpu(), table, full, ppr * page), dense_v)


@pytest.mark.parametrize("tiles", [False, True])
@pytest.mark.parametrize("batch", [1, 4])
def test_rms_qkv_rope_append_paged_matches_dense(dev, batch, tiles):
    gen = torch.Generator().manual_seed(40 + batch)
    hidden, width = 896, (QH + 2 * KVH) * D
    x = torch.randn(batch, hidden, generator=gen).half()
    nw = (torch.rand(hidden, generator=gen) + 0.5).half()
    w = (torch.randn(width, hidden, generator=gen) * 0.02).half()
    bias = (torch.randn(width, generator=gen) * 0.1).half()
    page, ppr = 64, 3
    n_pages = batch * ppr + 1
    table = _table(gen, batch, ppr, n_pages)
    slots = torch.tensor([5, 130, 64, 191][:batch])
    cos, sin = rope_cos_sin(slots, inv_freq(D, 1e6))
    kp0 = torch.randn(n_pages, KVH, page, D, generator=gen).half()
    vp0 = torch.randn(n_pages, KVH, page, D, generator=gen).half()
    kp, vp = kp0.to(dev), vp0.to(dev)
    q_out = torch.zeros(batch, QH, D, device=dev, dtype=torch.float16)
    print(f"[paged qkv] B={batch} tiles={tiles}", flush=True)
    wp = step_ops.pack_weight(w.to(dev), step_ops.PACK_ROPE) if tiles else w.to(dev)
    paged.rms_qkv_rope_append_paged(x.to(dev), nw.to(dev), 1e-6, wp, bias.to(dev),
                                    cos.to(dev), sin.to(dev), kp, vp, table.to(dev),
                                    slots.to(dev), q_out)
    # Dense twin: each row written at its own slot of a dense cache, one row at a time.
    kc = torch.zeros(batch, KVH, ppr * page, D, device=dev, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    q_ref = torch.zeros_like(q_out)
    for r in range(batch):
        step_ops.rms_qkv_rope_append(x[r:r + 1].to(dev), nw.to(dev), 1e-6, wp, bias.to(dev),
                                     cos[r:r + 1].to(dev), sin[r:r + 1].to(dev), kc[r:r + 1],
                                     vc[r:r + 1], torch.tensor([int(slots[r])], device=dev),
                                     q_ref[r:r + 1])
    torch.cuda.synchronize()
    assert torch.equal(q_out.cpu(), q_ref.cpu())
    kp_ref, vp_ref = kp0.clone(), vp0.clone()
    for r in range(batch):
        s = int(slots[r])
        p, row = oracle.paged_location(table, r, s, page)
        kp_ref[p, :, row] = kc[r, :, s].cpu()
        vp_ref[p, :, row] = vc[r, :, s].cpu()
    assert torch.equal(kp.cpu(), kp_ref)
    assert torch.equal(vp.cpu(), vp_ref)
    qo, ko, vo = ost.qkv_rope16(x, nw, 1e-6, w, bias, cos, sin, QH, KVH, D)
    assert ((q_out.float().cpu() - qo.float()).abs() / qo.float().abs().clamp_min(1)).max() <= 4e-3


def test_rms_qkv_rope_append_paged_positions_mode(dev):
    """Paged QKV append with in-kernel RoPE angles equals the table mode."""
    from qwenforge_amd.rope import cos_sin, inv_freq as make_inv

    gen = torch.Generator().manual_seed(44)
    batch, hidden, width = 2, 896, (QH + 2 * KVH) * D
    x = torch.randn(batch, hidden, generator=gen).half().to(dev)
    nw = (torch.rand(hidden, generator=gen) + 0.5).half().to(dev)
    w = (torch.randn(width, hidden, generator=gen) * 0.02).half().to(dev)
    page, ppr = 64, 2
    table = _table(gen, batch, ppr, batch * ppr).to(dev)
    slots = torch.tensor([7, 100], device=dev)
    inv = make_inv(D, 1e6, dev)
    cos, sin = cos_sin(slots, inv)
    outs = []
    for use_pos in (False, True):
        kp = torch.zeros(batch * ppr, KVH, page, D, device=dev, dtype=torch.float16)
        vp = torch.zeros_like(kp)
        q_out = torch.zeros(batch, QH, D, device=dev, dtype=torch.float16)
        if use_pos:
            paged.rms_qkv_rope_append_paged(x, nw, 1e-6, w, None, None, None, kp, vp, table, slots,
                                            q_out, positions=(slots, inv))
        else:
            paged.rms_qkv_rope_append_paged(x, nw, 1e-6, w, None, cos, sin, kp, vp, table, slots,
                                            q_out)
        outs.append((q_out, kp, vp))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a.cpu(), b.cpu())
