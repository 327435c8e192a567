"""CPU restatement of the reference's rotate-half RoPE (test infrastructure only)."""

from __future__ import annotations

import torch


def inv_freq(head_dim: int, theta: float) -> torch.Tensor:
    """``inv_freq = 1 / theta ** (arange(0, D, 2) / D)`` in fp32 (SE:362-363)."""
    idx = torch.arange(0, head_dim, 2, dtype=torch.float32)
    return 1.0 / (theta ** (idx / head_dim))


def rope_cos_sin(
    positions: torch.Tensor, inverse_frequency: torch.Tensor, dtype: torch.dtype = torch.float16
):
    """Per-position cos/sin table (SE:545-548, per-step form SE:912-915).

    ``f = positions.float()[..., None] * inv_freq``; ``emb = cat(f, f)``;
    cos/sin are evaluated in fp32 and cast to ``dtype``.  positions (...,)
    int64 -> cos, sin (..., D).
    """
    f = positions.to(torch.float32).unsqueeze(-1) * inverse_frequency
    emb = torch.cat((f, f), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """``[x1, x2] -> [-x2, x1]`` over the two halves of the last dim (SE:537-540)."""
    first, second = x.chunk(2, dim=-1)
    return torch.cat((-second, first), dim=-1)


def _round16(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.float16).to(torch.float32)


def apply_rope_fp16(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Eager fp16 RoPE ``x * cos + rotate_half(x) * sin`` (SE:927-928, SE:552-553).

    The eager graph step evaluates three fp16 ops, each rounded to fp16:
    ``t1 = fp16(x*cos)``, ``t2 = fp16(rot(x)*sin)``, ``out = fp16(t1 + t2)``.
    Each is computed here in fp32 and rounded once: the product of two fp16
    values is exact in fp32, and an fp32 sum rounded to fp16 equals the
    correctly rounded fp16 sum (fp32 carries more than 2*11+2 significand
    bits).  Returns fp16.  ``cos``/``sin`` broadcast against ``x``.
    """
    xf = x.to(torch.float32)
    t1 = _round16(xf * cos.to(torch.float32))
    t2 = _round16(rotate_half(xf) * sin.to(torch.float32))
    return (t1 + t2).to(torch.float16)


def apply_rope_fp32(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """The same formula in the input dtype (used by the whiteboard fp32 KAT)."""
    return x * cos + rotate_half(x) * sin
