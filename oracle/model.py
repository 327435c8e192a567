"""CPU restatement of the reference's cached prefill and graph decode step for a
Qwen2-shaped model, fp32-accumulated (test infrastructure only).

``prefill`` follows ``StudentEngine._prefill`` (SE:679-737) and
``decode_step`` follows ``_decode_step_static`` (SE:876-982, math attention
branch SE:968-972), with every op evaluated in fp32 on fp16 weights.  RoPE
goes through ``rope.rope_cos_sin`` / ``rope.apply_rope_fp32`` (the functions
the GPU tests feed the kernels), so the pins below cover them too.

Pins (``tests/test_oracle_model.py``): the whole forward -- embedding, fused
QKV split, RoPE, GQA causal attention, o_proj, RMSNorm, SwiGLU MLP, tied
lm_head -- against ``transformers.Qwen2ForCausalLM`` (an independent
implementation of the official model) on a tiny random config, live and
through the committed logits in ``tests/golden/qwen2_tiny_logits.json``;
plus the prefill/decode consistency test in ``tests/test_oracle.py`` (the
decode step over a prefilled cache reproduces the prefill logits of the
longer prompt).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .attention import eager_attention, grouped_decode_attention
from .rope import apply_rope_fp32, inv_freq, rope_cos_sin


def _rms(x, w, eps):
    # SE:530-535 (fp32 upcast, rsqrt(mean(x^2) + eps), times weight).
    return x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps) * w


def _rope(x, pos, inverse_frequency):
    # SE:542-554 in fp32: the (B, T, D) table of rope_cos_sin, broadcast over heads.
    cos, sin = rope_cos_sin(pos, inverse_frequency, dtype=torch.float32)
    return apply_rope_fp32(x, cos.unsqueeze(1), sin.unsqueeze(1))


def _f(t):
    return t.to(torch.float32)


def _qkv(x, layer, cfg):
    b, t, _ = x.shape
    p = x @ _f(layer["qkv_weight"]).T + _f(layer["qkv_bias"])
    q, k, v = p.split((cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim,
                       cfg.kv_heads * cfg.head_dim), dim=-1)
    return (q.view(b, t, cfg.heads, cfg.head_dim).transpose(1, 2),
            k.view(b, t, cfg.kv_heads, cfg.head_dim).transpose(1, 2),
            v.view(b, t, cfg.kv_heads, cfg.head_dim).transpose(1, 2))


def _mlp(x, layer):
    gate, up = (x @ _f(layer["gate_up_weight"]).T).chunk(2, dim=-1)
    return (F.silu(gate) * up) @ _f(layer["down_weight"]).T


def inv_freq32(cfg):
    return inv_freq(cfg.head_dim, cfg.rope_theta)


def prefill(weights, cfg, input_ids, capacity):
    """Equal-length prompts -> (last-token logits (B, V), fp32 caches [(K, V)] of capacity)."""
    b, s = input_ids.shape
    inv = inv_freq32(cfg)
    pos = torch.arange(s).unsqueeze(0).expand(b, s)
    hidden = _f(weights["embed"])[input_ids]
    caches = []
    for layer in weights["layers"]:
        residual = hidden
        q, k, v = _qkv(_rms(hidden, _f(layer["input_norm"]), cfg.rms_eps), layer, cfg)
        q, k = _rope(q, pos, inv), _rope(k, pos, inv)
        kc = torch.zeros(b, cfg.kv_heads, capacity, cfg.head_dim)
        vc = torch.zeros_like(kc)
        kc[:, :, :s] = k
        vc[:, :, :s] = v
        caches.append((kc, vc))
        att = eager_attention(q, k, v, causal=True)
        hidden = residual + att.transpose(1, 2).reshape(b, s, cfg.hidden) @ _f(layer["o_weight"]).T
        residual = hidden
        hidden = residual + _mlp(_rms(hidden, _f(layer["post_norm"]), cfg.rms_eps), layer)
    last = _rms(hidden[:, -1], _f(weights["final_norm"]), cfg.rms_eps)
    return last @ _f(weights["lm_head"]).T, caches


def decode_step(weights, cfg, tokens, positions, caches, write_index, bias=None):
    """One graph-step decode (SE:876-982) -> logits (B, V); appends at ``write_index``.

    ``bias`` (B, cap) additive; None treats slots ``<= write_index`` as valid and
    the rest as empty (the no-padding case).
    """
    b = tokens.shape[0]
    inv = inv_freq32(cfg)
    hidden = _f(weights["embed"])[tokens].view(b, 1, cfg.hidden)
    cap = caches[0][0].shape[2]
    if bias is None:
        bias = torch.full((b, cap), float(torch.finfo(torch.float16).min))
        bias[:, :write_index + 1] = 0.0
    for layer, (kc, vc) in zip(weights["layers"], caches):
        residual = hidden
        q, k, v = _qkv(_rms(hidden, _f(layer["input_norm"]), cfg.rms_eps), layer, cfg)
        q, k = _rope(q, positions.view(b, 1), inv), _rope(k, positions.view(b, 1), inv)
        kc[:, :, write_index] = k[:, :, 0]
        vc[:, :, write_index] = v[:, :, 0]
        grouped = q.reshape(b, cfg.kv_heads, cfg.groups, cfg.head_dim)
        att = grouped_decode_attention(grouped, kc, vc, bias)
        hidden = residual + att.reshape(b, 1, cfg.hidden) @ _f(layer["o_weight"]).T
        residual = hidden
        hidden = residual + _mlp(_rms(hidden, _f(layer["post_norm"]), cfg.rms_eps), layer)
    hidden = _rms(hidden, _f(weights["final_norm"]), cfg.rms_eps).squeeze(1)
    return hidden @ _f(weights["lm_head"]).T
