"""Host-side launch planning: the decode split count (CPU only).

The rule was measured on MI355X; these cases pin what it returns at the
benchmark shapes and that it never leaves a few CUs with a second workgroup
(a count just above one per CU), the case that costs up to 30%.
"""

import pytest

from qwenforge_amd import ops


@pytest.mark.parametrize("batch,length,splits", [
    (1, 512, 8),       # config 1: splits of >= 64 keys
    (4, 2048, 16),     # config 2 (cap 2048): >= 128 keys with 8 pairs
    (1, 32768, 128),   # config 3: two launches
    (1, 4096, 32),     # the single-launch merge's limit
    (16, 32768, 8),    # bandwidth regime: one workgroup per CU
    (64, 4096, 2),
    (12, 5760, 21),    # the reference's benchmark shape: two per CU, fused
    (20, 4096, 12),
    (100, 4096, 1),    # 200 pairs: one split, no merge
    (8, 4096, 16),     # one per CU fits exactly; twice would give 128-key splits
    (16, 4096, 16),    # exact fit, but 256-key splits: twice
    (32, 1024, 4),
    (128, 1024, 1),    # 256 pairs: one split per row fills the chip, no merge
])
def test_choose_splits_at_benchmark_shapes(batch, length, splits):
    assert ops.choose_splits(batch, 2, length) == splits


@pytest.mark.parametrize("batch", list(range(1, 129)))
def test_workgroups_fill_cus_once_or_twice(batch):
    for length in (512, 1024, 2048, 4096, 5760, 8192, 16384, 32768):
        s = ops.choose_splits(batch, 2, length)
        wg = 2 * batch * s
        if s == 1:
            continue  # at least as many pairs as CUs: nothing to split
        # Either at most one workgroup per CU, or two per CU with the
        # single-launch merge, or a long-context case with <= 8 pairs.
        assert wg <= ops.NUM_CUS or (s <= 32 and wg <= 2 * ops.NUM_CUS) or 2 * batch <= 8, \
            (batch, length, s)
        # Splits keep at least one 32-key tile.
        assert -(-length // s) >= 32


def test_engine_capacity_rule_equals_oracle():
    """The engine's KV capacity (engine.cache_capacity, used by generate and
    generate_ragged) against the oracle's restatement of SE:1263-1273."""
    import oracle
    from qwenforge_amd.engine import cache_capacity

    for p in list(range(1, 200, 3)) + [511, 512, 1023, 1024, 1025, 2048]:
        for n in (0, 1, 2, 3, 63, 64, 65, 127, 128, 129, 300):
            assert cache_capacity(p, n) == oracle.capacity(p, n), (p, n)
    assert cache_capacity(1024, 128) == 1152
