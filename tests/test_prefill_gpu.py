"""Parity of the HIP causal flash-prefill (+ fused RoPE and cache append).

Oracle: ``oracle.causal_prefill`` (SE:164-251 semantics, fp32) on inputs
rotated by ``oracle.apply_rope_fp16`` (the eager fp16 sequence, SE:927-928).
Attention tolerance 2e-3 max-abs-err; cache contents bit-exact.
"""

import pytest
import torch

import oracle
from qwenforge_amd import ops, workloads

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _err(a, b):
    return (a.float() - b.float()).abs().max().item()


def test_config4_rope_append_s2048(dev):
    case = workloads.prefill_case(2048, seed=0)
    print("[prefill cfg4 S=2048]", flush=True)
    c = case.to(dev)
    kc = torch.zeros(1, 2, 2048, 64, dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    out = torch.ops.student_qwen.gqa_flash_prefill_rope_append(c.query, c.key, c.value, c.cos, c.sin,
                                                              kc, vc, 0)
    torch.cuda.synchronize()
    q_rot = oracle.apply_rope_fp16(case.query, case.cos, case.sin)
    k_rot = oracle.apply_rope_fp16(case.key, case.cos, case.sin)
    ref = oracle.causal_prefill(q_rot, k_rot, case.value)
    assert _err(out.cpu(), ref) <= TOL
    assert torch.equal(kc.cpu(), k_rot)
    assert torch.equal(vc.cpu(), case.value)


@pytest.mark.parametrize("seq,batch", [(1100, 2), (4100, 1)])
def test_rope_append_long_prompts_repeat_and_replay(dev, seq, batch):
    """Fused RoPE + append on long prompts (18 and 65 query tiles: the two
    halves of each workgroup take 1-33 key tiles, one half idle in the last
    step of every odd count): three calls in a row and several replays of a
    captured graph must all match the oracle."""
    case = workloads.prefill_case(seq, batch=batch, seed=seq + batch)
    print(f"[prefill long prompt S={seq} B={batch}]", flush=True)
    c = case.to(dev)
    kc = torch.zeros(batch, 2, seq + 60, 64, dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    q_rot = oracle.apply_rope_fp16(case.query, case.cos, case.sin)
    k_rot = oracle.apply_rope_fp16(case.key, case.cos, case.sin)
    ref = oracle.causal_prefill(q_rot, k_rot, case.value)
    outs = [ops.gqa_flash_prefill_rope_append(c.query, c.key, c.value, c.cos, c.sin, kc, vc, 0)
            for _ in range(3)]
    torch.cuda.synchronize()
    for out in outs:
        assert _err(out.cpu(), ref) <= TOL
    assert torch.equal(kc[:, :, :seq].cpu(), k_rot)
    assert torch.equal(vc[:, :, :seq].cpu(), case.value)
    # Graph capture, several replays.
    static_out = torch.empty_like(c.query)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        static_out.copy_(ops.gqa_flash_prefill_rope_append(c.query, c.key, c.value, c.cos, c.sin,
                                                           kc, vc, 0))
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_out.copy_(ops.gqa_flash_prefill_rope_append(c.query, c.key, c.value, c.cos, c.sin,
                                                           kc, vc, 0))
    for _ in range(3):
        static_out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert _err(static_out.cpu(), ref) <= TOL


@pytest.mark.parametrize("seq", [1, 17, 64, 100, 513])
@pytest.mark.parametrize("batch", [1, 2])
def test_plain_prefill_ragged_lengths(dev, seq, batch):
    case = workloads.prefill_case(seq, batch=batch, seed=seq + batch)
    c = case.to(dev)
    out = torch.ops.student_qwen.gqa_flash_prefill(c.query, c.key, c.value)
    torch.cuda.synchronize()
    ref = oracle.causal_prefill(case.query, case.key, case.value)
    assert _err(out.cpu(), ref) <= TOL


def test_projection_views_with_distinct_v_strides(dev):
    """q/k/v as views of one fused projection (SE:754-766): V's strides differ from K's."""
    gen = torch.Generator("cpu").manual_seed(3)
    b, s = 2, 300
    projected = torch.randn(b, s, 1152, generator=gen).half()
    q, k, v = projected.split((896, 128, 128), dim=-1)
    q = q.view(b, s, 14, 64).transpose(1, 2)
    k = k.view(b, s, 2, 64).transpose(1, 2)
    v = v.view(b, s, 2, 64).transpose(1, 2)
    pg = projected.to(dev)
    qg, kg, vg = pg.split((896, 128, 128), dim=-1)
    qg = qg.view(b, s, 14, 64).transpose(1, 2)
    kg = kg.view(b, s, 2, 64).transpose(1, 2)
    vg = vg.view(b, s, 2, 64).transpose(1, 2)
    out = torch.ops.student_qwen.gqa_flash_prefill(qg, kg, vg)
    torch.cuda.synchronize()
    ref = oracle.causal_prefill(q, k, v)
    assert _err(out.cpu(), ref) <= TOL


def test_append_at_offset_leaves_other_slots(dev):
    case = workloads.prefill_case(130, batch=2, seed=9)
    c = case.to(dev)
    kc = torch.full((2, 2, 400, 64), 3.0, dtype=torch.float16, device=dev)
    vc = torch.full_like(kc, -2.0)
    start = 77
    out = ops.gqa_flash_prefill_rope_append(c.query, c.key, c.value, c.cos, c.sin, kc, vc, start)
    torch.cuda.synchronize()
    k_rot = oracle.apply_rope_fp16(case.key, case.cos, case.sin)
    kcc, vcc = kc.cpu(), vc.cpu()
    assert torch.equal(kcc[:, :, start:start + 130], k_rot)
    assert torch.equal(vcc[:, :, start:start + 130], case.value)
    assert bool((kcc[:, :, :start] == 3.0).all()) and bool((kcc[:, :, start + 130:] == 3.0).all())
    assert bool((vcc[:, :, :start] == -2.0).all()) and bool((vcc[:, :, start + 130:] == -2.0).all())
    q_rot = oracle.apply_rope_fp16(case.query, case.cos, case.sin)
    assert _err(out.cpu(), oracle.causal_prefill(q_rot, k_rot, case.value)) <= TOL


def test_first_row_is_first_value(dev):
    case = workloads.prefill_case(200, seed=4)
    c = case.to(dev)
    out = ops.gqa_flash_prefill(c.query, c.key, c.value).cpu()
    expect = case.value.repeat_interleave(7, dim=1)[:, :, 0]
    assert _err(out[:, :, 0], expect) == 0.0


@pytest.mark.parametrize("seq", [1100, 2048, 4100])
def test_long_plain_prefill_through_the_abi(dev, seq):
    """The plain op and a direct qf_prefill_attn call (no RoPE, no cache) on
    long prompts both match the oracle, and each other bit for bit."""
    from qwenforge_amd import _lib

    case = workloads.prefill_case(seq, batch=1, seed=seq)
    c = case.to(dev)
    lib = _lib.load()
    via_op = torch.ops.student_qwen.gqa_flash_prefill(c.query, c.key, c.value)
    direct = torch.empty_like(c.query)
    rc = lib.qf_prefill_attn(
        c.query.data_ptr(), *c.query.stride()[:3], c.key.data_ptr(), *c.key.stride()[:3],
        c.value.data_ptr(), *c.value.stride()[:3], None, None, 0, 0,
        None, 0, 0, 0, None, 0, 0, 0, 0, 0,
        direct.data_ptr(), *direct.stride()[:3], 1, 14, 2, seq, 64, 0.125,
        torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "qf_prefill_attn")
    torch.cuda.synchronize()
    ref = oracle.causal_prefill(case.query, case.key, case.value)
    print(f"[prefill plain S={seq}] op err {_err(via_op.cpu(), ref):.2e} "
          f"direct err {_err(direct.cpu(), ref):.2e}", flush=True)
    assert _err(via_op.cpu(), ref) <= TOL
    assert torch.equal(via_op, direct)


@pytest.mark.parametrize("lengths", [[1, 65, 200, 513], [130], [64, 64, 7]])
def test_varlen_prefill_rope_append_matches_per_row_oracle(dev, lengths):
    """Packed ragged rows (SE:1162-1204 semantics): each row is its own causal
    prefill at positions 0..len-1, K/V land in slots [0, len) of its cache row,
    every other slot is untouched."""
    from oracle.rope import inv_freq, rope_cos_sin

    gen = torch.Generator().manual_seed(sum(lengths))
    b, total, qh, kvh = len(lengths), sum(lengths), 14, 2
    q = torch.randn(total, qh, 64, generator=gen).half()
    k = torch.randn(total, kvh, 64, generator=gen).half()
    v = torch.randn(total, kvh, 64, generator=gen).half()
    pos = torch.cat([torch.arange(n) for n in lengths])
    cos, sin = rope_cos_sin(pos, inv_freq(64, 1e6))
    starts = [0]
    for n in lengths:
        starts.append(starts[-1] + n)
    cap = (max(lengths) + 63) // 64 * 64 + 64
    kc0 = torch.randn(b, kvh, cap, 64, generator=gen).half()
    vc0 = torch.randn(b, kvh, cap, 64, generator=gen).half()
    kc, vc = kc0.to(dev), vc0.to(dev)
    cu = torch.tensor(starts, dtype=torch.int32, device=dev)
    print(f"[prefill varlen] lengths={lengths}", flush=True)
    out = ops.prefill_varlen(q.to(dev), k.to(dev), v.to(dev), cu, max(lengths), cos.to(dev),
                             sin.to(dev), kc, vc, 0)
    torch.cuda.synchronize()
    out, kc, vc = out.cpu(), kc.cpu(), vc.cpu()
    for i, n in enumerate(lengths):
        sl = slice(starts[i], starts[i + 1])
        q_rot = oracle.apply_rope_fp16(q[sl].transpose(0, 1), cos[sl], sin[sl])   # (QH, n, 64)
        k_rot = oracle.apply_rope_fp16(k[sl].transpose(0, 1), cos[sl], sin[sl])   # (KVH, n, 64)
        ref = oracle.causal_prefill(q_rot[None], k_rot[None], v[sl].transpose(0, 1)[None])[0]
        assert _err(out[sl].transpose(0, 1), ref) <= TOL, f"row {i}"
        assert torch.equal(kc[i, :, :n], k_rot)
        assert torch.equal(vc[i, :, :n], v[sl].transpose(0, 1))
        assert torch.equal(kc[i, :, n:], kc0[i, :, n:])
        assert torch.equal(vc[i, :, n:], vc0[i, :, n:])


@pytest.mark.parametrize("seq,batch", [(1, 1), (100, 2), (1100, 1)])
def test_rope_without_cache(dev, seq, batch):
    """RoPE on q and k with no cache to append to (the register-staged kernel
    rotates each K tile on its way to LDS): matches the oracle on rotated
    inputs."""
    from qwenforge_amd import ops as ops_

    case = workloads.prefill_case(seq, batch=batch, seed=50 + seq)
    c = case.to(dev)
    print(f"[prefill rope, no cache] S={seq} B={batch}", flush=True)
    out = torch.empty_like(c.query)
    ops_._prefill_launch(c.query, c.key, c.value, out, c.cos, c.sin)
    torch.cuda.synchronize()
    q_rot = oracle.apply_rope_fp16(case.query, case.cos, case.sin)
    k_rot = oracle.apply_rope_fp16(case.key, case.cos, case.sin)
    assert _err(out.cpu(), oracle.causal_prefill(q_rot, k_rot, case.value)) <= TOL
