"""Writes ``oracle_goldens.npz``: outputs of the CPU oracle on reduced BASELINE configs.

Run from the repository root: ``python tests/golden/make_oracle_goldens.py``.

The inputs are not stored: they are regenerated from their seeds by
``qwenforge_amd.workloads`` (a seeded CPU generator, so every machine draws the
same bits), and each case stores a SHA-256 of its fp16 input bytes so a test can
tell a changed generator from a changed oracle.  Cases:

* ``cfg1``: config 1 at full size (B=1, L=cap=512), ``oracle.grouped_decode_attention``.
* ``cfg2``: config 2 reduced (B=4 ragged rows, lengths ~ U[256, 512], bias holes).
* ``cfg3``: config 3 reduced (B=1, L=4096, 1% of keys x8).
* ``cfg4``: config 4 reduced (S=96, a tail tile): the rotated K (fp16, the cache
  contents ``oracle.apply_rope_fp16`` gives) and ``oracle.causal_prefill`` on the
  rotated q/k, stored as fp16.
* ``rope``: the fp16 cos/sin table of ``oracle.rope_cos_sin`` at positions
  0, 1, 2047 and 32767 (theta 1e6, head dim 64).
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from qwenforge_amd import workloads  # noqa: E402

OUT = Path(__file__).resolve().parent / "oracle_goldens.npz"
ROPE_POSITIONS = (0, 1, 2047, 32767)
PREFILL_SEQ = 96


def fingerprint(*tensors: torch.Tensor) -> np.ndarray:
    """SHA-256 of the tensors' bytes in order, as 32 uint8."""
    h = hashlib.sha256()
    for t in tensors:
        h.update(t.contiguous().view(torch.uint8).numpy().tobytes())
    return np.frombuffer(h.digest(), dtype=np.uint8).copy()


def decode_cases():
    """(name, DecodeCase) of the decode goldens."""
    return [
        ("cfg1", workloads.decode_uniform(1, 512, seed=0)),
        ("cfg2", workloads.decode_ragged(4, lo=256, hi=512, seed=0)),
        ("cfg3", workloads.decode_uniform(1, 4096, seed=0, heavy_frac=0.01)),
    ]


def decode_inputs_fingerprint(case) -> np.ndarray:
    parts = [case.grouped, case.key_cache, case.value_cache]
    if case.bias is not None:
        parts.append(case.bias)
    return fingerprint(*parts)


def prefill_case():
    return workloads.prefill_case(PREFILL_SEQ, seed=0)


def prefill_reference(case):
    """(rotated k fp16, attention output fp16) of the reduced config 4."""
    q_rot = oracle.apply_rope_fp16(case.query, case.cos, case.sin)
    k_rot = oracle.apply_rope_fp16(case.key, case.cos, case.sin)
    out = oracle.causal_prefill(q_rot, k_rot, case.value)
    return k_rot, out.to(torch.float16)


def rope_table():
    cos, sin = oracle.rope_cos_sin(torch.tensor(ROPE_POSITIONS), oracle.inv_freq(64, 1e6))
    return cos, sin


def build() -> dict:
    arrays = {}
    for name, case in decode_cases():
        ref = oracle.grouped_decode_attention(case.grouped, case.key_cache, case.value_cache,
                                              case.bias)
        arrays[f"{name}_out"] = ref.float().numpy()
        arrays[f"{name}_inputs_sha256"] = decode_inputs_fingerprint(case)
    pc = prefill_case()
    k_rot, out = prefill_reference(pc)
    arrays["cfg4_k_rot"] = k_rot.numpy()
    arrays["cfg4_out"] = out.numpy()
    arrays["cfg4_inputs_sha256"] = fingerprint(pc.query, pc.key, pc.value, pc.cos, pc.sin)
    cos, sin = rope_table()
    arrays["rope_positions"] = np.array(ROPE_POSITIONS, dtype=np.int64)
    arrays["rope_cos"] = cos.numpy()
    arrays["rope_sin"] = sin.numpy()
    return arrays


if __name__ == "__main__":
    np.savez_compressed(OUT, **build())
    print(OUT, OUT.stat().st_size, "bytes")
