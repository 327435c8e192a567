"""Pins of ``oracle.model`` (the config-5 restatement of SE:679-737 and
SE:876-982) against an independent implementation of the official model,
``transformers.Qwen2ForCausalLM``, on a tiny random Qwen2 config: random
qkv biases and RMSNorm weights, GQA 4/2 heads at head_dim 64, theta 1e6,
tied lm_head.  The reference validated its own forward against the official
model the same way (docs/optimization_journey.md:354-359).

The committed fixture (tests/golden/qwen2_tiny_logits.json, written by
tests/golden/qwen2_tiny.py) pins the oracle where transformers is absent; the
live comparison runs where it is importable.  A planted mistake -- interleaved
RoPE pairs instead of rotate-half -- must fail the same check.
"""

import importlib.util
import json
from pathlib import Path

import pytest
import torch

import oracle.model as om
from oracle import rope as orope

GOLDEN = Path(__file__).resolve().parent / "golden"
TOL = 2e-4  # fp32 vs fp32, different summation orders; logits have std ~1


def _tiny():
    spec = importlib.util.spec_from_file_location("qwen2_tiny", GOLDEN / "qwen2_tiny.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _oracle_logits(tiny, cfg, w, ids):
    """Prefill logits of ids[:, :-1] and the decode-step logits of ids[:, -1]."""
    b, n = ids.shape
    s = n - 1
    cap = 64
    pre, caches = om.prefill(w, cfg, ids[:, :s], cap)
    dec = om.decode_step(w, cfg, ids[:, s], torch.full((b,), s), caches, s)
    return pre, dec


def test_oracle_model_matches_committed_transformers_logits():
    tiny = _tiny()
    cfg, w = tiny.config(), tiny.weights(tiny.config())
    data = json.loads(tiny.FIXTURE.read_text())
    ids = torch.tensor(data["ids"])
    assert torch.equal(ids, tiny.prompt_ids(cfg))
    pre, dec = _oracle_logits(tiny, cfg, w, ids)
    want_pre = torch.tensor(data["prefill_logits"])
    want_dec = torch.tensor(data["decode_logits"])
    assert want_pre.std().item() > 0.3  # the logits carry signal, not noise around 0
    assert (pre - want_pre).abs().max().item() < TOL
    assert (dec - want_dec).abs().max().item() < TOL


def test_oracle_model_matches_transformers_live():
    pytest.importorskip("transformers")
    tiny = _tiny()
    cfg = tiny.config()
    w = tiny.weights(cfg)
    ids = tiny.prompt_ids(cfg)
    want_pre, want_dec = tiny.hf_logits(cfg, w, ids)
    pre, dec = _oracle_logits(tiny, cfg, w, ids)
    assert (pre - want_pre).abs().max().item() < TOL
    assert (dec - want_dec).abs().max().item() < TOL


def test_planted_interleaved_rope_fails_the_model_pin(monkeypatch):
    """The same check rejects a plausible RoPE layout mistake in the oracle."""
    tiny = _tiny()
    cfg = tiny.config()
    w = tiny.weights(cfg)
    data = json.loads(tiny.FIXTURE.read_text())
    ids = torch.tensor(data["ids"])

    def interleaved_table(positions, inverse_frequency, dtype=torch.float16):
        f = positions.to(torch.float32).unsqueeze(-1) * inverse_frequency
        emb = f.repeat_interleave(2, dim=-1)
        return emb.cos().to(dtype), emb.sin().to(dtype)

    monkeypatch.setattr(om, "rope_cos_sin", interleaved_table)
    pre, _ = _oracle_logits(tiny, cfg, w, ids)
    assert (pre - torch.tensor(data["prefill_logits"])).abs().max().item() > 100 * TOL


def test_planted_dropped_qkv_bias_fails_the_model_pin():
    tiny = _tiny()
    cfg = tiny.config()
    w = tiny.weights(cfg)
    for layer in w["layers"]:
        layer["qkv_bias"] = torch.zeros_like(layer["qkv_bias"])
    data = json.loads(tiny.FIXTURE.read_text())
    pre, _ = _oracle_logits(tiny, cfg, w, torch.tensor(data["ids"]))
    assert (pre - torch.tensor(data["prefill_logits"])).abs().max().item() > 100 * TOL


def test_rope_table_closed_form_at_long_positions():
    """``rope_cos_sin`` at theta=1e6, D=64 for positions far from 0.

    Closed form: dim i uses angle p * theta**(-2 (i mod 32) / 64) (rotate-half
    layout: dims i and i + 32 share a frequency).  The reference forms the
    angle in fp32 (SE:912: ``pos.float() * inv_freq``), so two checks:
      * bit level: fp64 numpy cos/sin of that fp32 angle, rounded to fp16,
        equals the table within one fp16 ulp (torch's fp32 cos/sin may sit
        one fp32 ulp off, which can move an fp16 rounding by one step);
      * the exact fp64 angle: within one fp16 ulp plus the fp32 angle error
        (|angle| * 2**-22: two fp32 roundings in inv_freq, one in the product).
    An interleaved table, a dropped factor 2, a wrong theta or swapped cos/sin
    fails both.
    """
    import numpy as np

    theta, d = 1e6, 64
    pos = np.array([1, 2047, 32767, 131071], dtype=np.int64)
    cos, sin = orope.rope_cos_sin(torch.from_numpy(pos), orope.inv_freq(d, theta))
    assert cos.dtype == torch.float16 and cos.shape == (4, 64)
    c, s = cos.numpy().astype(np.float64), sin.numpy().astype(np.float64)
    assert np.array_equal(c[:, :32], c[:, 32:]) and np.array_equal(s[:, :32], s[:, 32:])

    inv32 = orope.inv_freq(d, theta).numpy()                       # (32,) fp32
    ang32 = (pos.astype(np.float32)[:, None] * inv32[None, :]).astype(np.float64)
    ang32 = np.concatenate((ang32, ang32), axis=1)
    ulp = lambda x: np.maximum(np.abs(x), 2.0 ** -14) * 2.0 ** -10  # noqa: E731 (fp16 spacing bound)
    for got, fn in ((c, np.cos), (s, np.sin)):
        want = fn(ang32).astype(np.float16).astype(np.float64)
        assert np.all(np.abs(got - want) <= ulp(want)), fn.__name__

    i = np.arange(64) % 32
    exact = pos.astype(np.float64)[:, None] * theta ** (-2.0 * i / d)[None, :]
    for got, fn in ((c, np.cos), (s, np.sin)):
        want = fn(exact)
        tol = ulp(want) + np.abs(exact) * 2.0 ** -22
        assert np.all(np.abs(got - want) <= tol), fn.__name__
    # Position 1 sits where the fp32 angle error is far below an fp16 ulp.
    assert np.all(np.abs(c[0] - np.cos(exact[0])) <= ulp(np.cos(exact[0])))
    # The layout mistakes the closed form must reject.
    inter = np.repeat(pos.astype(np.float64)[:, None] * theta ** (-2.0 * np.arange(32) / d), 2, axis=1)
    assert np.abs(c - np.cos(inter)).max() > 0.1
    half = pos.astype(np.float64)[:, None] * theta ** (-1.0 * i / d)[None, :]
    assert np.abs(c - np.cos(half)).max() > 0.1
