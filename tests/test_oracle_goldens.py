"""The CPU oracle and the seeded input generators against the committed goldens.

``tests/golden/oracle_goldens.npz`` holds the oracle's outputs on reduced
BASELINE configs (config 1 at full size, config 2 with rows of 256-512 slots,
config 3 at L=4096 with its 1% of keys x8, config 4 at S=96 with a tail tile)
and the fp16 RoPE table at positions 0, 1, 2047 and 32767, written by
``tests/golden/make_oracle_goldens.py``.  Inputs are regenerated from their
seeds; each case's SHA-256 of the fp16 input bytes must match first, so a
changed generator and a changed oracle fail different assertions.

Tolerances: decode outputs are fp32 and agree to 1e-5 (the CPU's own summation
order may differ between machines); the prefill output is stored rounded to
fp16, so a value may land one fp16 step away (<= 1e-3 at |x| < 2); the rotated
keys and the RoPE table are bit-exact.
"""

import importlib.util
from pathlib import Path

import numpy as np
import torch

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def _maker():
    spec = importlib.util.spec_from_file_location("make_oracle_goldens",
                                                  GOLDEN / "make_oracle_goldens.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


MK = _maker()
G = np.load(GOLDEN / "oracle_goldens.npz")


def test_decode_goldens():
    for name, case in MK.decode_cases():
        assert np.array_equal(MK.decode_inputs_fingerprint(case), G[f"{name}_inputs_sha256"]), name
        ref = oracle.grouped_decode_attention(case.grouped, case.key_cache, case.value_cache,
                                              case.bias).float().numpy()
        err = np.abs(ref - G[f"{name}_out"]).max()
        assert err <= 1e-5, (name, err)


def test_prefill_golden():
    pc = MK.prefill_case()
    assert np.array_equal(MK.fingerprint(pc.query, pc.key, pc.value, pc.cos, pc.sin),
                          G["cfg4_inputs_sha256"])
    k_rot, out = MK.prefill_reference(pc)
    assert np.array_equal(k_rot.numpy(), G["cfg4_k_rot"])
    diff = np.abs(out.float().numpy() - G["cfg4_out"].astype(np.float32))
    assert diff.max() <= 1e-3
    assert (diff == 0).mean() >= 0.999


def test_rope_table_golden():
    cos, sin = MK.rope_table()
    assert np.array_equal(G["rope_positions"], np.array(MK.ROPE_POSITIONS))
    assert np.array_equal(cos.numpy(), G["rope_cos"])
    assert np.array_equal(sin.numpy(), G["rope_sin"])
    # Position 0 is the identity rotation, whatever produced the file.
    assert np.all(G["rope_cos"][0] == 1.0) and np.all(G["rope_sin"][0] == 0.0)


def test_golden_decode_outputs_are_attention_of_the_inputs():
    """Independent of the oracle: config 1's golden row equals fp64 SDPA."""
    name, case = MK.decode_cases()[0]
    q = case.grouped.double()
    k = case.key_cache.double().unsqueeze(2).expand(-1, -1, q.shape[2], -1, -1)
    v = case.value_cache.double().unsqueeze(2).expand(-1, -1, q.shape[2], -1, -1)
    ref = torch.nn.functional.scaled_dot_product_attention(q.unsqueeze(3), k, v).squeeze(3)
    assert np.abs(ref.numpy() - G[f"{name}_out"]).max() <= 1e-5
