"""Seeded synthetic inputs for the BASELINE configurations.

Draws follow one rule everywhere: ``torch.Generator('cpu').manual_seed(seed)``,
``randn`` in fp32, then ``.half()``, in the order Q, K, V; tensors are built on
the CPU and moved afterwards, so the CPU checker and the GPU kernels see the
same bits.  Layouts are the reference engine's (SE:939, SE:705-716,
SE:1017-1020).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

QH, KVH, G, D = 14, 2, 7, 64
THETA = 1e6
FP16_MIN = float(torch.finfo(torch.float16).min)


def _randn(gen: torch.Generator, *shape) -> torch.Tensor:
    return torch.randn(*shape, generator=gen, dtype=torch.float32).half()


@dataclass
class DecodeCase:
    grouped: torch.Tensor        # (B, KVH, G, D)
    key_cache: torch.Tensor      # (B, KVH, cap, D)
    value_cache: torch.Tensor    # (B, KVH, cap, D)
    bias: torch.Tensor | None    # (B, cap) fp16
    lengths: list                # valid slots per row (prefix [0, L_b))

    def to(self, device):
        mv = lambda t: None if t is None else t.to(device)  # noqa: E731
        return DecodeCase(mv(self.grouped), mv(self.key_cache), mv(self.value_cache),
                          mv(self.bias), list(self.lengths))

    @property
    def valid_bytes(self) -> int:
        """Algorithmic bytes of one decode-attention call: valid K+V plus q and out."""
        b, kvh, g, d = self.grouped.shape
        return 2 * kvh * d * 2 * sum(self.lengths) + 2 * (2 * b * kvh * g * d)


def decode_uniform(batch: int, length: int, seed: int = 0, cap: int | None = None,
                   heavy_frac: float = 0.0, with_bias: bool = False) -> DecodeCase:
    """Config 1 (B=1, L=512) and config 3 (B=1, L=32768, 1% keys x8) shapes.

    ``heavy_frac`` scales round(frac*L) randomly chosen key rows per kv head by
    8 (exact in fp16).  Slots past ``length`` (when ``cap > length``) are zero
    and masked by the bias.
    """
    cap = length if cap is None else cap
    gen = torch.Generator("cpu").manual_seed(seed)
    q = _randn(gen, batch, KVH, G, D)
    k = torch.zeros(batch, KVH, cap, D, dtype=torch.float16)
    v = torch.zeros_like(k)
    k[:, :, :length] = _randn(gen, batch, KVH, length, D)
    v[:, :, :length] = _randn(gen, batch, KVH, length, D)
    if heavy_frac > 0:
        n_heavy = round(heavy_frac * length)
        for b in range(batch):
            for h in range(KVH):
                rows = torch.randperm(length, generator=gen)[:n_heavy]
                k[b, h, rows] = k[b, h, rows] * 8
    bias = None
    if with_bias or cap > length:
        bias = torch.full((batch, cap), FP16_MIN, dtype=torch.float16)
        bias[:, :length] = 0.0
    return DecodeCase(q, k, v, bias, [length] * batch)


def decode_ragged(batch: int = 4, lo: int = 256, hi: int = 2048, seed: int = 0) -> DecodeCase:
    """Config 2 (one layer): per-row lengths ~ U[lo, hi], cap = roundup(max, 64).

    Slots ``>= L_b`` hold zeros (the reference zero-initialises caches,
    SE:705-714) and carry the fp16-min bias.
    """
    gen = torch.Generator("cpu").manual_seed(seed)
    lengths = torch.randint(lo, hi + 1, (batch,), generator=gen).tolist()
    cap = (max(lengths) + 63) // 64 * 64
    q = _randn(gen, batch, KVH, G, D)
    k = torch.zeros(batch, KVH, cap, D, dtype=torch.float16)
    v = torch.zeros_like(k)
    for b, n in enumerate(lengths):
        k[b, :, :n] = _randn(gen, KVH, n, D)
        v[b, :, :n] = _randn(gen, KVH, n, D)
    bias = torch.full((batch, cap), FP16_MIN, dtype=torch.float16)
    for b, n in enumerate(lengths):
        bias[b, :n] = 0.0
    return DecodeCase(q, k, v, bias, lengths)


def decode_ragged_layers(layers: int = 24, batch: int = 4, seed: int = 0):
    """Config 2: ``layers`` independent per-layer caches (seed + layer)."""
    return [decode_ragged(batch, seed=seed + i) for i in range(layers)]


@dataclass
class PrefillCase:
    query: torch.Tensor   # (B, QH, S, D) pre-RoPE
    key: torch.Tensor     # (B, KVH, S, D) pre-RoPE
    value: torch.Tensor   # (B, KVH, S, D)
    cos: torch.Tensor     # (S, D) fp16
    sin: torch.Tensor     # (S, D) fp16

    def to(self, device):
        return PrefillCase(*(t.to(device) for t in (self.query, self.key, self.value, self.cos, self.sin)))

    @property
    def flops(self) -> int:
        """Causal QK^T + PV flops: 2 * QH * D * S * (S + 1) per batch row."""
        b, qh, s, d = self.query.shape
        return 2 * b * qh * d * s * (s + 1)


def prefill_case(seq: int = 2048, batch: int = 1, seed: int = 0, theta: float = THETA) -> PrefillCase:
    """Config 4: pre-RoPE Q/K/V for positions 0..S-1 and the fp16 RoPE table."""
    from .rope import cos_sin, inv_freq

    gen = torch.Generator("cpu").manual_seed(seed)
    q = _randn(gen, batch, QH, seq, D)
    k = _randn(gen, batch, KVH, seq, D)
    v = _randn(gen, batch, KVH, seq, D)
    cos, sin = cos_sin(torch.arange(seq), inv_freq(D, theta))
    return PrefillCase(q, k, v, cos, sin)
