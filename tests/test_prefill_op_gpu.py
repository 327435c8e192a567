"""The prefill custom ops as drop-ins for compiled callers.

The reference calls ``student_qwen::gqa_flash_prefill`` from code compiled
with ``torch.compile(dynamic=True, fullgraph=True)`` (SE:464-469, SE:772-773),
which relies on the op's schema and its ``register_fake`` (SE:282-290).
``torch.library.opcheck`` checks the schema (including ``mutates_args`` of the
fused RoPE + append op), the fake against the real kernel (shapes, strides,
dtypes) and AOT dispatch with dynamic shapes.  A compiled caller shaped like
the reference's prefill block (projection views -> RoPE -> the op -> o_proj
layout) must return the eager result bit for bit at two prompt lengths
without recompiling, and the compiled mutating op must leave the same cache
contents as the eager call.
"""

import pytest
import torch
import torch.nn.functional as F

import oracle
from qwenforge_amd import ops, workloads  # noqa: F401  (registers the ops)
from qwenforge_amd.rope import cos_sin, inv_freq

pytestmark = pytest.mark.gpu
QH, KVH, D = 14, 2, 64


def _views(dev, s, seed):
    """Projection-output views as the reference forms them (SE:755-765): (B, S, H, D) -> (B, H, S, D)."""
    gen = torch.Generator().manual_seed(seed)
    proj = torch.randn(1, s, (QH + 2 * KVH) * D, generator=gen).half().to(dev)
    q, k, v = proj.split((QH * D, KVH * D, KVH * D), dim=-1)
    return (q.view(1, s, QH, D).transpose(1, 2), k.view(1, s, KVH, D).transpose(1, 2),
            v.view(1, s, KVH, D).transpose(1, 2))


def test_opcheck_gqa_flash_prefill(dev):
    q, k, v = _views(dev, 192, 0)
    torch.library.opcheck(torch.ops.student_qwen.gqa_flash_prefill.default, (q, k, v))
    case = workloads.prefill_case(130, seed=1).to(dev)
    torch.library.opcheck(torch.ops.student_qwen.gqa_flash_prefill.default,
                          (case.query, case.key, case.value))


def test_opcheck_gqa_flash_prefill_rope_append(dev):
    case = workloads.prefill_case(200, seed=2).to(dev)
    kc = torch.zeros(1, KVH, 256, D, dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    torch.library.opcheck(torch.ops.student_qwen.gqa_flash_prefill_rope_append.default,
                          (case.query, case.key, case.value, case.cos, case.sin, kc, vc, 0))
    torch.library.opcheck(torch.ops.student_qwen.gqa_flash_prefill_rope_append.default,
                          (case.query, case.key, case.value, case.cos, case.sin, kc, vc, 56))


def _prefill_block(q, k, v, cos, sin):
    # SE:767-775: eager RoPE on the projection views, the custom op, then the
    # (B, S, hidden) layout o_proj consumes.
    q = q * cos + oracle.rotate_half(q) * sin
    k = k * cos + oracle.rotate_half(k) * sin
    att = torch.ops.student_qwen.gqa_flash_prefill(q, k, v)
    b, h, s, d = att.shape
    return att.transpose(1, 2).reshape(b, s, h * d)


def test_compiled_caller_equals_eager(dev):
    torch._dynamo.reset()
    compiled = torch.compile(_prefill_block, backend="aot_eager", fullgraph=True, dynamic=True)
    inv = inv_freq(D, 1e6, dev)
    for i, s in enumerate((512, 700)):
        q, k, v = _views(dev, s, 10 + i)
        cos, sin = cos_sin(torch.arange(s, device=dev), inv)
        want = _prefill_block(q, k, v, cos, sin)
        got = compiled(q, k, v, cos, sin)
        torch.cuda.synchronize()
        print(f"[compiled prefill S={s}] max|d| {(got.float() - want.float()).abs().max():.3e}",
              flush=True)
        assert torch.equal(got, want)
        ref = oracle.causal_prefill(*(t.cpu() for t in (
            q * cos + oracle.rotate_half(q) * sin, k * cos + oracle.rotate_half(k) * sin, v)))
        assert (got.float().cpu().reshape(1, s, QH, D).transpose(1, 2) - ref).abs().max() <= 2e-3


def test_compiled_rope_append_op_mutates_caches_like_eager(dev):
    torch._dynamo.reset()

    def block(q, k, v, cos, sin, kc, vc):
        att = torch.ops.student_qwen.gqa_flash_prefill_rope_append(q, k, v, cos, sin, kc, vc, 64)
        return F.silu(att.float()).sum(dim=-1)

    compiled = torch.compile(block, backend="aot_eager", fullgraph=True, dynamic=True)
    case = workloads.prefill_case(300, seed=3).to(dev)
    args = (case.query, case.key, case.value, case.cos, case.sin)
    kc_e = torch.zeros(1, KVH, 384, D, dtype=torch.float16, device=dev)
    vc_e = torch.zeros_like(kc_e)
    kc_c, vc_c = kc_e.clone(), vc_e.clone()
    want = block(*args, kc_e, vc_e)
    got = compiled(*args, kc_c, vc_c)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(kc_c, kc_e) and torch.equal(vc_c, vc_e)
    assert torch.equal(kc_c[:, :, 64:364].cpu(),
                       oracle.apply_rope_fp16(case.key.cpu(), case.cos.cpu(), case.sin.cpu()))
    assert float(kc_c[:, :, :64].abs().sum()) == 0.0
