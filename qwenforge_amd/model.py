"""Qwen2-shaped model configuration and random-init weights.

The layout is the reference engine's (``_LayerWeights`` SE:295-304 built by
``_layer_weights`` SE:499-528): q/k/v projections concatenated into one
``[QH*D + 2*KVH*D, hidden]`` weight with its bias, gate/up concatenated into
one ``[2*inter, hidden]`` weight, tied ``lm_head``.  There is no checkpoint
loading: weights are drawn N(0, std) from a seed, biases are zero and RMSNorm
weights are one.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Qwen2Config:
    """Qwen2.5-0.5B shape (config.json fields read at SE:333-342)."""

    hidden: int = 896
    layers: int = 24
    heads: int = 14
    kv_heads: int = 2
    head_dim: int = 64
    intermediate: int = 4864
    vocab: int = 151936
    rms_eps: float = 1e-6
    rope_theta: float = 1e6

    @property
    def groups(self) -> int:
        return self.heads // self.kv_heads

    @property
    def qkv_width(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    def weight_bytes(self, dtype_bytes: int = 2) -> int:
        """Bytes one decode step streams: every layer weight plus the tied lm_head."""
        per_layer = (self.qkv_width * self.hidden + self.qkv_width + self.hidden * self.hidden
                     + 2 * self.intermediate * self.hidden + self.hidden * self.intermediate
                     + 2 * self.hidden)
        return dtype_bytes * (self.layers * per_layer + self.vocab * self.hidden + self.hidden)


def init_weights(cfg: Qwen2Config, device="cpu", seed: int = 0, std: float = 0.02,
                 dtype=torch.float16) -> dict:
    """Random-init weights in the reference's fused layout.

    Linear and embedding weights ~ N(0, std) from ``torch.Generator(device)``
    seeded with ``seed``; qkv bias 0; RMSNorm weights 1; ``lm_head`` tied to
    the embedding (SE:358-360).
    """
    gen = torch.Generator(device=device).manual_seed(seed)

    def rnd(*shape):
        return (torch.randn(*shape, generator=gen, device=device, dtype=torch.float32) * std).to(dtype)

    layers = []
    for _ in range(cfg.layers):
        layers.append({
            "input_norm": torch.ones(cfg.hidden, device=device, dtype=dtype),
            "qkv_weight": rnd(cfg.qkv_width, cfg.hidden),
            "qkv_bias": torch.zeros(cfg.qkv_width, device=device, dtype=dtype),
            "o_weight": rnd(cfg.hidden, cfg.heads * cfg.head_dim),
            "post_norm": torch.ones(cfg.hidden, device=device, dtype=dtype),
            "gate_up_weight": rnd(2 * cfg.intermediate, cfg.hidden),
            "down_weight": rnd(cfg.hidden, cfg.intermediate),
        })
    embed = rnd(cfg.vocab, cfg.hidden)
    return {
        "embed": embed,
        "final_norm": torch.ones(cfg.hidden, device=device, dtype=dtype),
        "lm_head": embed,
        "layers": layers,
    }


def weights_to(weights: dict, device) -> dict:
    """Copy a weight dict to ``device`` (keeping lm_head tied)."""
    embed = weights["embed"].to(device)
    return {
        "embed": embed,
        "final_norm": weights["final_norm"].to(device),
        "lm_head": embed,
        "layers": [{k: v.to(device) for k, v in layer.items()} for layer in weights["layers"]],
    }
