"""Bit-exactness of the HIP decode RoPE + KV append (SE:927-932)."""

import pytest
import torch

import oracle
from qwenforge_amd import ops

pytestmark = pytest.mark.gpu


def _inputs(batch, cap, seed):
    gen = torch.Generator("cpu").manual_seed(seed)
    projected = (torch.randn(batch, 1, 1152, generator=gen) * 3).half()
    q, k, v = projected.split((896, 128, 128), dim=-1)
    q = q.view(batch, 1, 14, 64).transpose(1, 2)
    k = k.view(batch, 1, 2, 64).transpose(1, 2)
    v = v.view(batch, 1, 2, 64).transpose(1, 2)
    pos = torch.randint(0, 32768, (batch,), generator=gen)
    cos, sin = oracle.rope_cos_sin(pos, oracle.inv_freq(64, 1e6))
    cos, sin = cos.view(batch, 1, 1, 64), sin.view(batch, 1, 1, 64)
    kc = torch.randn(batch, 2, cap, 64, generator=gen).half()
    vc = torch.randn(batch, 2, cap, 64, generator=gen).half()
    return projected, q, k, v, cos, sin, kc, vc


def _dev_views(projected, batch, dev):
    pg = projected.to(dev)
    q, k, v = pg.split((896, 128, 128), dim=-1)
    return (q.view(batch, 1, 14, 64).transpose(1, 2), k.view(batch, 1, 2, 64).transpose(1, 2),
            v.view(batch, 1, 2, 64).transpose(1, 2))


@pytest.mark.parametrize("batch", [1, 4])
@pytest.mark.parametrize("slot", [0, 517, 1151])
def test_bit_exact(dev, batch, slot):
    projected, q, k, v, cos, sin, kc, vc = _inputs(batch, 1152, seed=batch * 7 + slot)
    qg, kg, vg = _dev_views(projected, batch, dev)
    kcg, vcg = kc.to(dev), vc.to(dev)
    wi = torch.tensor([slot], dtype=torch.int64, device=dev)
    q_rot = ops.rope_append(qg, kg, vg, cos.to(dev), sin.to(dev), kcg, vcg, wi)
    torch.cuda.synchronize()
    rq = oracle.apply_rope_fp16(q, cos, sin)
    rk = oracle.apply_rope_fp16(k, cos, sin)
    ekc, evc = oracle.append_decode(kc.clone(), vc.clone(), rk, v, torch.tensor([slot]))
    assert torch.equal(q_rot.cpu(), rq)
    assert torch.equal(kcg.cpu(), ekc)
    assert torch.equal(vcg.cpu(), evc)


def test_out_of_range_slot_writes_nothing(dev):
    projected, q, k, v, cos, sin, kc, vc = _inputs(2, 64, seed=1)
    qg, kg, vg = _dev_views(projected, 2, dev)
    kcg, vcg = kc.to(dev), vc.to(dev)
    for slot in (-1, 64, 10**6):
        wi = torch.tensor([slot], dtype=torch.int64, device=dev)
        q_rot = ops.rope_append(qg, kg, vg, cos.to(dev), sin.to(dev), kcg, vcg, wi)
        torch.cuda.synchronize()
        assert torch.equal(kcg.cpu(), kc) and torch.equal(vcg.cpu(), vc)
        assert torch.equal(q_rot.cpu(), oracle.apply_rope_fp16(q, cos, sin))


def test_graph_replay_follows_write_index(dev):
    batch, cap = 4, 256
    projected, q, k, v, cos, sin, kc, vc = _inputs(batch, cap, seed=2)
    qg, kg, vg = _dev_views(projected, batch, dev)
    cg, sg = cos.to(dev), sin.to(dev)
    kcg, vcg = kc.to(dev), vc.to(dev)
    wi = torch.tensor([cap - 1], dtype=torch.int64, device=dev)
    out = torch.empty(batch, 14, 1, 64, dtype=torch.float16, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.rope_append(qg, kg, vg, cg, sg, kcg, vcg, wi, out=out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.rope_append(qg, kg, vg, cg, sg, kcg, vcg, wi, out=out)
    ekc, evc = kc.clone(), vc.clone()
    rk = oracle.apply_rope_fp16(k, cos, sin)
    ekc, evc = oracle.append_decode(ekc, evc, rk, v, torch.tensor([cap - 1]))
    for slot in (3, 100, 101, 7):
        wi.fill_(slot)
        g.replay()
        torch.cuda.synchronize()
        ekc, evc = oracle.append_decode(ekc, evc, rk, v, torch.tensor([slot]))
        assert torch.equal(kcg.cpu(), ekc) and torch.equal(vcg.cpu(), evc), f"slot {slot}"
