"""The engine's registry of captured decode steps (CPU only): least recently
used first, evicted past a KV byte budget, never the entry just stored
(the reference's rule, SE:1090-1118 with the 2.4 GB budget of SE:394)."""

import torch

from qwenforge_amd.engine import GraphRegistry


def _ctx(batch, cap, layers=2):
    shape = (batch, 2, cap, 64)
    return {"caches": [(torch.zeros(shape, dtype=torch.float16),
                        torch.zeros(shape, dtype=torch.float16)) for _ in range(layers)]}


def test_kv_bytes_counts_every_layer_and_both_caches():
    assert GraphRegistry.kv_bytes(_ctx(3, 128, layers=4)) == 4 * 2 * 3 * 2 * 128 * 64 * 2


def test_hits_refresh_and_the_budget_evicts_oldest_first():
    unit = GraphRegistry.kv_bytes(_ctx(1, 64))
    reg = GraphRegistry(byte_budget=3 * unit)
    for key in ("a", "b", "c"):
        reg.put(key, _ctx(1, 64))
    assert reg.keys() == ["a", "b", "c"]
    assert reg.get("a") is not None and reg.keys() == ["b", "c", "a"]
    assert reg.get("zz") is None
    reg.put("d", _ctx(1, 64))             # 4 units: "b" is the least recently used
    assert reg.keys() == ["c", "a", "d"]
    reg.put("e", _ctx(2, 64))             # 2 units: two entries go
    assert reg.keys() == ["d", "e"]
    assert len(reg) == 2


def test_the_newest_entry_stays_even_over_budget():
    reg = GraphRegistry(byte_budget=1)
    reg.put("a", _ctx(1, 64))
    assert reg.keys() == ["a"]
    reg.put("b", _ctx(1, 64))
    assert reg.keys() == ["b"]
    reg.put("b", _ctx(1, 128))            # storing a key again replaces it
    assert reg.keys() == ["b"] and reg.get("b")["caches"][0][0].shape[2] == 128
    reg.clear()
    assert len(reg) == 0


def test_default_budget_is_the_reference_one():
    assert GraphRegistry().byte_budget == 2_400_000_000
