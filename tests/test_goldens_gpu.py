"""The HIP path against the committed oracle goldens.

Same cases as ``tests/test_oracle_goldens.py`` (inputs regenerated from their
seeds, checked against the stored SHA-256 first): decode attention at config 1
(full size) and reduced configs 2 and 3, with the planner's merge mode and
both explicit ones; the cached prefill at S=96 (attention within 2e-3 of the
golden, cache rows bit-exact to the stored rotated keys and the raw values);
the decode RoPE + append driven by the golden cos/sin table at positions 0, 1,
2047 and 32767, bit-exact against ``oracle.apply_rope_fp16`` on that table.
"""

import importlib.util
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from qwenforge_amd import ops

pytestmark = pytest.mark.gpu
TOL = 2e-3
GOLDEN = Path(__file__).resolve().parent / "golden"


def _maker():
    spec = importlib.util.spec_from_file_location("make_oracle_goldens",
                                                  GOLDEN / "make_oracle_goldens.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


MK = _maker()
G = np.load(GOLDEN / "oracle_goldens.npz")


@pytest.mark.parametrize("fused", [None, True, False])
@pytest.mark.parametrize("name", ["cfg1", "cfg2", "cfg3"])
def test_decode_against_golden(dev, name, fused):
    case = dict(MK.decode_cases())[name]
    assert np.array_equal(MK.decode_inputs_fingerprint(case), G[f"{name}_inputs_sha256"])
    print(f"[golden decode {name} fused={fused}]", flush=True)
    c = case.to(dev)
    b, kvh, g, _ = c.grouped.shape
    cap = c.key_cache.shape[2]
    flash = ops.make_flash_scratch(b, kvh, g, cap, dev, fused=fused)
    out = ops.flash_decode_attention(c.grouped, c.key_cache, c.value_cache, c.bias, flash)
    torch.cuda.synchronize()
    err = np.abs(out.float().cpu().numpy() - G[f"{name}_out"]).max()
    assert err <= TOL, err


def test_prefill_rope_append_against_golden(dev):
    pc = MK.prefill_case()
    assert np.array_equal(MK.fingerprint(pc.query, pc.key, pc.value, pc.cos, pc.sin),
                          G["cfg4_inputs_sha256"])
    c = pc.to(dev)
    s = pc.query.shape[2]
    kc = torch.zeros(1, 2, s, 64, dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    out = ops.gqa_flash_prefill_rope_append(c.query, c.key, c.value, c.cos, c.sin, kc, vc, 0)
    torch.cuda.synchronize()
    err = np.abs(out.float().cpu().numpy() - G["cfg4_out"].astype(np.float32)).max()
    assert err <= TOL, err
    assert np.array_equal(kc.cpu().numpy(), G["cfg4_k_rot"])
    assert torch.equal(vc.cpu(), pc.value)


def test_rope_append_with_golden_table(dev):
    cos = torch.from_numpy(G["rope_cos"]).view(4, 1, 1, 64)
    sin = torch.from_numpy(G["rope_sin"]).view(4, 1, 1, 64)
    gen = torch.Generator("cpu").manual_seed(5)
    q = (torch.randn(4, 14, 1, 64, generator=gen) * 3).half()
    k = (torch.randn(4, 2, 1, 64, generator=gen) * 3).half()
    v = torch.randn(4, 2, 1, 64, generator=gen).half()
    kc = torch.zeros(4, 2, 16, 64, dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    wi = torch.tensor([3], dtype=torch.int64, device=dev)
    q_rot = ops.rope_append(q.to(dev), k.to(dev), v.to(dev), cos.to(dev), sin.to(dev), kc, vc, wi)
    torch.cuda.synchronize()
    assert torch.equal(q_rot.cpu(), oracle.apply_rope_fp16(q, cos, sin))
    assert torch.equal(kc[:, :, 3:4].cpu(), oracle.apply_rope_fp16(k, cos, sin))
    assert torch.equal(vc[:, :, 3:4].cpu(), v)
