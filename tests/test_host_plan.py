"""Host-side launch planning: the decode split count (CPU only).

The rule was measured on MI355X; these cases pin what it returns at the
benchmark shapes and that it never leaves a few CUs with a second workgroup
(a count just above one per CU), the case that costs up to 30%.
"""

import pytest

from qwenforge_amd import ops


@pytest.mark.parametrize("batch,length,splits,fused", [
    (1, 128, 1, False),      # one split, no merge: 3.73 us vs 5.27 for 4 fused splits
    (1, 256, 1, False),      # 4.82 us vs 5.35 for 8 fused splits
    (8, 256, 1, False),      # 4.99 us vs 6.02 for 4 fused splits
    (12, 256, 1, False),     # 24 pairs: 5.00 us vs 6.29 for 2 fused splits
    (32, 256, 1, False),     # 64 pairs: 5.14 us vs 6.57 for 2 fused splits
    (32, 128, 1, False),     # 4.19 us vs 6.02 for 2 fused splits
    (12, 512, 4, True),      # 24 pairs: 6.59 us vs 7.08 for one split
    (1, 320, 10, True),      # from 320 slots the single-launch merge wins (5.54 at 8 vs 5.80 at 1)
    (1, 512, 16, True),      # config 1: 32-key splits, single launch (5.46 us vs 5.58 at 8)
    (1, 2048, 16, True),     # 128-key splits: 6.23 us vs 6.47 for 64 split + combine
    (2, 512, 8, True),       # 6.23 us vs 6.58 at 4
    (4, 512, 8, True),       # 6.55 us vs 6.70 at 4
    (4, 2048, 16, True),     # config 2 (cap 2048): 7.00 us vs 7.31 for 32 split + combine
    (8, 512, 4, True),       # 16 pairs, short rows: 6.55 us vs 6.72 for 16 split + combine
    (1, 32768, 128, False),  # config 3: split + combine
    (1, 4096, 64, False),    # one workgroup per CU, 64-key splits: 6.71 us vs 6.96 at 32 fused
    (1, 8192, 128, False),   # 7.10 us
    (2, 4096, 64, False),    # 7.05 us vs 7.45 for 16 fused splits
    (4, 4096, 32, False),    # 7.84 us vs 8.25 for 16 fused splits
    (4, 8192, 32, False),    # 9.14 us vs 9.41 at 64
    (4, 16384, 32, False),   # 11.79 us vs 12.44 at 128
    (8, 2048, 16, False),    # 7.87 us vs 8.19 for 12 fused splits
    (8, 4096, 16, False),    # 9.15 us vs 9.39 at 32
    (8, 16384, 16, False),   # 16.79 us vs 17.71 at 64
    (5, 5000, 25, False),    # 8.82 us vs 9.51 at 39
    (1, 2500, 40, False),    # 64-key floor: 40 splits, 80 workgroups
    (16, 32768, 8, True),    # bandwidth regime: one workgroup per CU
    (64, 4096, 2, True),
    (12, 5760, 10, True),    # the reference's benchmark shape: once per CU (12.55 vs 13.35 us at 21)
    (20, 4096, 6, True),     # once per CU (12.86 vs 13.18 us at 12)
    (100, 4096, 1, False),   # 200 pairs: one split, no merge
    (16, 4096, 8, True),     # exact fit, once per CU (11.58 vs 13.13 us at 16)
    (32, 1024, 4, True),
    (128, 1024, 1, False),   # 256 pairs: one split per row fills the chip, no merge
])
def test_decode_plan_at_benchmark_shapes(batch, length, splits, fused):
    assert ops.decode_plan(batch, 2, length, cus=256) == (splits, fused)
    assert ops.choose_splits(batch, 2, length, cus=256) == splits


@pytest.mark.parametrize("batch", list(range(1, 129)))
def test_workgroup_counts_stay_in_the_measured_ranges(batch):
    for length in (64, 256, 320, 512, 1024, 2048, 4096, 5760, 8192, 16384, 32768):
        s, fused = ops.decode_plan(batch, 2, length, cus=256)
        pairs, wg = 2 * batch, 2 * batch * s
        assert 1 <= s <= 128
        if length <= 256:
            assert (s, fused) == (1, False)  # one split per (b, kv head), no merge
        assert fused == (s > 1 and (pairs > 16 and s <= 32 or pairs <= 16 and fused))
        if fused:
            assert s <= 32  # the single-launch merge folds <= 8 partials per lane
        if s == 1:
            continue  # at least as many pairs as CUs, or a row too short to split
        if pairs <= 16:
            # Single launch: at most 192 workgroups; two launches: one
            # workgroup per CU (floor(CUs / pairs) splits, never a count just
            # above it), fewer only where 64-key splits or 128 splits cap it.
            full = ops.NUM_CUS // pairs
            want = min(full, 128, -(-length // 64))
            assert (wg <= 192) if fused else (s == want and wg <= ops.NUM_CUS), \
                (batch, length, s)
        else:
            # Once per CU.
            assert wg <= ops.NUM_CUS, (batch, length, s)
        # Splits keep at least one 32-key tile.
        assert -(-length // s) >= 32


@pytest.mark.parametrize("cus", [32, 64, 80, 128, 304])
def test_plan_follows_the_device_cu_count(cus):
    """A partitioned MI355X (e.g. 32 CUs per partition) or another part: no
    plan puts more workgroups on the device than it has CUs (one per CU for
    split + combine and the fill rule, three per four CUs for the capped
    single launch), and the count comes from the device when none is given."""
    for batch in (1, 2, 4, 8, 16, 64):
        for length in (320, 512, 2048, 4096, 32768):
            s, fused = ops.decode_plan(batch, 2, length, cus=cus)
            wg = 2 * batch * s
            assert s >= 1
            if s > 1:
                assert wg <= cus, (cus, batch, length, s)
            if fused and 2 * batch <= max(1, cus // 16):
                assert wg <= 3 * cus // 4 or s == 1, (cus, batch, length, s)


def test_plan_reads_the_cu_count_from_the_device(monkeypatch):
    """ops.num_cus() is the default: a stubbed device with 64 CUs gives the
    64-CU plan (config 3: 32 splits per kv head instead of 128)."""
    monkeypatch.setattr(ops, "num_cus", lambda device=None: 64)
    assert ops.decode_plan(1, 2, 32768) == ops.decode_plan(1, 2, 32768, cus=64)
    assert ops.decode_plan(1, 2, 32768)[0] * 2 <= 64
    assert ops.decode_plan(1, 2, 32768, cus=256) != ops.decode_plan(1, 2, 32768)


def test_engine_capacity_rule_equals_oracle():
    """The engine's KV capacity (engine.cache_capacity, used by generate and
    generate_ragged) against the oracle's restatement of SE:1263-1273."""
    import oracle
    from qwenforge_amd.engine import cache_capacity

    for p in list(range(1, 200, 3)) + [511, 512, 1023, 1024, 1025, 2048]:
        for n in (0, 1, 2, 3, 63, 64, 65, 127, 128, 129, 300):
            assert cache_capacity(p, n) == oracle.capacity(p, n), (p, n)
    assert cache_capacity(1024, 128) == 1152
