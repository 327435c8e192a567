"""CPU restatement of the graph decode step's projections with the fp16
rounding points of the reference's eager ops (test infrastructure only).

Each function evaluates the math in fp32 (products of fp16 values and their
sums; the projection sum order is free) and rounds to fp16 exactly where the
reference's torch ops store an fp16 tensor:

* ``rms_norm16``     -- ``F.rms_norm`` on fp16 (SE:904-906; the fused kernel
  rounds once: fp16((x * rsqrt(mean(x^2) + eps)) * w)).  With unit weights it
  equals the eager ``_rms_norm`` of SE:530-535.
* ``qkv_rope16``     -- ``F.linear(normalized, qkv_weight, qkv_bias)``
  (SE:919), split (SE:920-925), eager RoPE (SE:927-928 via
  ``apply_rope_fp16``).
* ``residual16``     -- ``residual + F.linear(inp, w)`` (SE:974, SE:978).
* ``swiglu16``       -- ``F.silu(gate) * up`` on the fp16 gate/up halves of
  ``F.linear(normalized, gate_up_weight)`` (SE:664-666).
* ``lm_head_argmax`` -- ``F.linear(rms_norm(hidden), lm_head)`` and
  ``torch.argmax`` (SE:980-982; first maximum on ties).

Pinned in ``tests/test_oracle_step.py``: ``residual16`` and ``swiglu16``
against torch-CPU half arithmetic (each torch half op computes in fp32 and
rounds once), ``rms_norm16`` against an fp64 evaluation and against the eager
two-rounding form with unit weights, ``qkv_rope16`` through
``apply_rope_fp16`` (pinned in ``tests/test_oracle.py``) plus a hand-checked
single-head case, ``lm_head_argmax`` against ``torch.argmax`` with planted
ties.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .rope import apply_rope_fp16


def _f(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.float32)


def rms_norm16(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """fp16 (B, H) -> fp16 (B, H): fp16((x * rsqrt(mean(x^2) + eps)) * w)."""
    xf = _f(x)
    rstd = torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return ((xf * rstd) * _f(w)).to(torch.float16)


def linear16(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """fp16 F.linear: fp32 accumulation (+ bias), one rounding."""
    acc = _f(x) @ _f(w).T
    if bias is not None:
        acc = acc + _f(bias)
    return acc.to(torch.float16)


def qkv_rope16(x16: torch.Tensor, norm_w, eps, w_qkv, bias, cos16, sin16, heads: int,
               kv_heads: int, head_dim: int = 64):
    """(B, H) fp16 residual rows -> q_rot (B, QH, D), k_rot (B, KVH, D), v (B, KVH, D), fp16.

    ``cos16``/``sin16``: (B, D) fp16 per-row tables (SE:912-915).
    """
    b = x16.shape[0]
    proj = linear16(rms_norm16(x16, norm_w, eps), w_qkv, bias)
    q, k, v = proj.split((heads * head_dim, kv_heads * head_dim, kv_heads * head_dim), dim=-1)
    q = q.reshape(b, heads, head_dim)
    k = k.reshape(b, kv_heads, head_dim)
    v = v.reshape(b, kv_heads, head_dim)
    c, s = cos16.unsqueeze(1), sin16.unsqueeze(1)
    return apply_rope_fp16(q, c, s), apply_rope_fp16(k, c, s), v


def residual16(residual: torch.Tensor, inp: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """fp16(residual + fp16(inp @ w^T))."""
    return (_f(residual) + _f(linear16(inp, w))).to(torch.float16)


def swiglu16(x16: torch.Tensor, norm_w, eps, w_gate_up: torch.Tensor) -> torch.Tensor:
    """h = fp16(fp16(silu(g)) * u) with [g | u] = fp16(rms_norm(x) @ w_gate_up^T)."""
    gu = linear16(rms_norm16(x16, norm_w, eps), w_gate_up)
    g, u = gu.chunk(2, dim=-1)
    gf = _f(g)
    s = (gf / (1.0 + torch.exp(-gf))).to(torch.float16)
    return (_f(s) * _f(u)).to(torch.float16)


def lm_head_argmax(x16: torch.Tensor, norm_w, eps, w_lm: torch.Tensor):
    """-> (fp16 logits (B, V), int64 argmax (B,)), first maximum on ties."""
    logits = linear16(rms_norm16(x16, norm_w, eps), w_lm)
    lf = _f(logits)
    best = lf.max(dim=-1, keepdim=True).values
    idx = torch.arange(lf.shape[-1]).expand_as(lf)
    first = torch.where(lf == best, idx, torch.full_like(idx, lf.shape[-1])).min(dim=-1).values
    return logits, first


def silu_mul_torch_half(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """The reference's literal ops on fp16 CPU tensors (SE:665-666), for pinning."""
    return F.silu(g) * u
