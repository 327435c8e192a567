"""RoPE tables as the reference engine builds them (torch ops, run on the device).

``inv_freq`` follows SE:362-363 and ``cos_sin`` follows SE:910-915 /
SE:545-548: angles in fp32, ``cos``/``sin`` evaluated in fp32 and cast to the
model dtype.  The HIP kernels take these fp16 tables as inputs, so the rotated
values they produce are bit-identical to the eager ``x*cos + rotate_half(x)*sin``
sequence given the same table.
"""

from __future__ import annotations

import torch


def inv_freq(head_dim: int, theta: float, device=None) -> torch.Tensor:
    idx = torch.arange(0, head_dim, 2, device=device, dtype=torch.float32)
    return 1.0 / (theta ** (idx / head_dim))


def cos_sin(positions: torch.Tensor, inverse_frequency: torch.Tensor,
            dtype: torch.dtype = torch.float16):
    """positions (...,) int64 -> fp16 cos, sin of shape (..., D)."""
    f = positions.to(torch.float32).unsqueeze(-1) * inverse_frequency
    emb = torch.cat((f, f), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)
