"""The reference's one-head toy decoder, restated on top of this oracle
(test infrastructure only).

The toy forward (whiteboard_minimal_transformer/whiteboard_llm_inference.py:
``ToyDecoderBlock.forward`` :418-440, ``CausalSelfAttention.forward`` :336-350,
``apply_rope`` :166-207, ``rms_norm`` :134-138, ``toy_ffn`` :237-257) is
rebuilt here from the oracle's own ``eager_attention(causal=True)`` and
rotate-half formula, so the reference's known-answer logits
(test_whiteboard_llm_inference.py:46-81) pin the oracle's causal convention
and RoPE layout.  The interleaved pairing exists only so the KAT can show it
gives different logits.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .attention import eager_attention
from .rope import apply_rope_fp32, inv_freq, rope_cos_sin


def _rotate_interleaved(x: torch.Tensor) -> torch.Tensor:
    pairs = x.reshape(*x.shape[:-1], -1, 2)
    return torch.stack((-pairs[..., 1], pairs[..., 0]), dim=-1).reshape_as(x)


def _rope(x: torch.Tensor, theta: float, mode: str) -> torch.Tensor:
    d = x.shape[-1]
    inv = inv_freq(d, theta)
    pos = torch.arange(x.shape[-2])
    if mode == "split_half":
        # The table and rotation the GPU tests use, so the KAT pins them.
        cos, sin = rope_cos_sin(pos, inv, dtype=torch.float32)
        return apply_rope_fp32(x, cos, sin)
    if mode == "interleaved":
        emb = torch.outer(pos.to(torch.float32), inv).repeat_interleave(2, dim=-1)
        return x * emb.cos() + _rotate_interleaved(x) * emb.sin()
    raise ValueError(f"rope mode {mode!r}")


def toy_forward(kat: dict, mode: str):
    """Next-token logits of the toy model for the KAT prompt. Returns (last_hidden, logits)."""
    t = lambda name: torch.tensor(kat[name], dtype=torch.float32)  # noqa: E731
    eps = kat["rms_norm_eps"]

    def rms(x):
        return x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps)

    x = t("embedding")[torch.tensor(kat["prompt_indices"])]            # (S, 4)
    h = rms(x)                                                         # q = k = v = h (identity projections)
    q = _rope(h, kat["rope_theta"], mode)
    k = _rope(h, kat["rope_theta"], mode)
    ctx = eager_attention(q[None, None], k[None, None], h[None, None], causal=True)[0, 0]
    x = x + ctx                                                        # identity o_proj
    f = rms(x)
    ffn = (F.silu(f @ t("w_gate")) * (f @ t("w_up"))) @ t("w_down")
    x = x + ffn
    last = x[-1]
    return last, last @ t("w_lm").T
