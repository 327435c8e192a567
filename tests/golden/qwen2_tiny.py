"""Tiny Qwen2 model shared by the oracle-model pin and its fixture writer.

``python tests/golden/qwen2_tiny.py`` evaluates the model with
``transformers.Qwen2ForCausalLM`` (eager attention, fp32) and writes
``qwen2_tiny_logits.json`` beside this file: the last-token logits of a
prefill and of one decode step.  ``tests/test_oracle_model.py`` checks
``oracle.model`` against that file, and against transformers live when it is
importable.

The weights are this build's fused layout (``qwenforge_amd.model``) drawn
from a seeded CPU generator, with random qkv biases and RMSNorm weights so
that a dropped bias or norm weight changes the logits.
"""

from __future__ import annotations

import json
import os
import sys
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

FIXTURE = HERE / "qwen2_tiny_logits.json"
SEED = 11
STD = 0.08
BATCH, PROMPT = 2, 13


def config():
    from qwenforge_amd.model import Qwen2Config

    return Qwen2Config(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64,
                       intermediate=384, vocab=512, rms_eps=1e-6, rope_theta=1e6)


def weights(cfg):
    """fp16 weights in the fused layout: N(0, STD) linears and embedding,
    N(0, 0.1) qkv bias, RMSNorm weights 1 + N(0, 0.2); tied lm_head."""
    from qwenforge_amd.model import init_weights

    w = init_weights(cfg, "cpu", seed=SEED, std=STD)
    gen = torch.Generator().manual_seed(SEED + 1)

    def rnd(n, scale, base=0.0):
        return (base + torch.randn(n, generator=gen) * scale).to(torch.float16)

    for layer in w["layers"]:
        layer["qkv_bias"] = rnd(cfg.qkv_width, 0.1)
        layer["input_norm"] = rnd(cfg.hidden, 0.2, 1.0)
        layer["post_norm"] = rnd(cfg.hidden, 0.2, 1.0)
    w["final_norm"] = rnd(cfg.hidden, 0.2, 1.0)
    return w


def prompt_ids(cfg):
    """(BATCH, PROMPT + 1) token ids: the prompt plus the decoded token."""
    gen = torch.Generator().manual_seed(SEED + 2)
    return torch.randint(0, cfg.vocab, (BATCH, PROMPT + 1), generator=gen)


def hf_model(cfg, w):
    """transformers.Qwen2ForCausalLM holding the same weights (fp32, eager attention)."""
    from transformers import Qwen2Config as HfConfig
    from transformers import Qwen2ForCausalLM

    hc = HfConfig(vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.intermediate,
                  num_hidden_layers=cfg.layers, num_attention_heads=cfg.heads,
                  num_key_value_heads=cfg.kv_heads, max_position_embeddings=4096,
                  rope_theta=cfg.rope_theta, rms_norm_eps=cfg.rms_eps,
                  tie_word_embeddings=True, attn_implementation="eager")
    model = Qwen2ForCausalLM(hc).float().eval()
    f = lambda t: t.to(torch.float32)  # noqa: E731
    qd, kd = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    with torch.no_grad():
        model.model.embed_tokens.weight.copy_(f(w["embed"]))
        model.model.norm.weight.copy_(f(w["final_norm"]))
        for hl, layer in zip(model.model.layers, w["layers"]):
            qkv, bias = f(layer["qkv_weight"]), f(layer["qkv_bias"])
            att = hl.self_attn
            att.q_proj.weight.copy_(qkv[:qd]); att.q_proj.bias.copy_(bias[:qd])
            att.k_proj.weight.copy_(qkv[qd:qd + kd]); att.k_proj.bias.copy_(bias[qd:qd + kd])
            att.v_proj.weight.copy_(qkv[qd + kd:]); att.v_proj.bias.copy_(bias[qd + kd:])
            att.o_proj.weight.copy_(f(layer["o_weight"]))
            gate, up = f(layer["gate_up_weight"]).chunk(2, dim=0)
            hl.mlp.gate_proj.weight.copy_(gate)
            hl.mlp.up_proj.weight.copy_(up)
            hl.mlp.down_proj.weight.copy_(f(layer["down_weight"]))
            hl.input_layernorm.weight.copy_(f(layer["input_norm"]))
            hl.post_attention_layernorm.weight.copy_(f(layer["post_norm"]))
    model.tie_weights()
    return model


def hf_logits(cfg, w, ids):
    """(prefill logits of ids[:, :-1], logits after ids[:, -1]) from transformers."""
    model = hf_model(cfg, w)
    with torch.no_grad():
        out = model(input_ids=ids).logits
    return out[:, -2], out[:, -1]


def main():
    cfg = config()
    w = weights(cfg)
    ids = prompt_ids(cfg)
    pre, dec = hf_logits(cfg, w, ids)
    import transformers

    data = {
        "what": "last-token logits of transformers.Qwen2ForCausalLM (fp32, eager attention) "
                "on the tiny config of tests/golden/qwen2_tiny.py",
        "transformers": transformers.__version__,
        "torch": torch.__version__,
        "seed": SEED, "std": STD,
        "ids": ids.tolist(),
        "prefill_logits": [[float(f"{x:.7g}") for x in row] for row in pre.tolist()],
        "decode_logits": [[float(f"{x:.7g}") for x in row] for row in dec.tolist()],
    }
    FIXTURE.write_text(json.dumps(data) + "\n")
    print(f"wrote {FIXTURE} ({os.path.getsize(FIXTURE)} bytes)")


if __name__ == "__main__":
    main()
