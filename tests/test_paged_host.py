"""Host-side page bookkeeping of ``qwenforge_amd.paged.PagedKvCache`` (CPU tensors)."""

import pytest
import torch

from qwenforge_amd import paged


def test_allocator_maps_grows_and_releases_rows():
    cache = paged.PagedKvCache(layers=2, kv_heads=2, n_pages=10, page_size=64, max_rows=3,
                               pages_per_row=4, device="cpu")
    assert cache.capacity == 256
    assert cache.map_row(0, 130) == [0, 1, 2]
    assert cache.map_row(1, 64) == [3]
    assert cache.map_row(0, 200) == [0, 1, 2, 4]      # grows by one page
    assert cache.map_row(0, 10) == [0, 1, 2, 4]       # never shrinks
    assert cache.free_pages() == 5
    cache.release_row(0)
    assert cache.free_pages() == 9
    assert cache.map_row(2, 256) == [0, 1, 2, 4]      # lowest free ids first
    t = cache.table
    assert t[0].tolist() == [-1, -1, -1, -1]
    assert t[1].tolist() == [3, -1, -1, -1]
    assert t[2].tolist() == [0, 1, 2, 4]
    assert cache.map_row(0, 256) == [5, 6, 7, 8]
    with pytest.raises(RuntimeError):
        cache.map_row(1, 256)                          # 3 more pages, 1 free
    with pytest.raises(ValueError):
        cache.map_row(1, 257)                          # beyond the row's 4 pages
    assert len(cache.pools) == 2 and cache.pools[0][0].shape == (10, 2, 64, 64)


def test_allocator_gather_reads_logical_slots():
    cache = paged.PagedKvCache(layers=1, kv_heads=2, n_pages=4, page_size=64, max_rows=2,
                               pages_per_row=2, device="cpu")
    cache.map_row(1, 64)       # row 1 takes page 0
    cache.map_row(0, 100)      # row 0 takes pages 1, 2
    k_pool, v_pool = cache.pools[0]
    k_pool.copy_(torch.arange(k_pool.numel(), dtype=torch.float32).view(k_pool.shape).half())
    k, _ = cache.gather(0, 0, 100)
    assert k.shape == (2, 100, 64)
    assert torch.equal(k[:, 0], k_pool[1, :, 0]) and torch.equal(k[:, 70], k_pool[2, :, 6])


@pytest.mark.parametrize("page", [32, 96, 8192])
def test_page_size_rules(page):
    with pytest.raises(ValueError):
        paged.PagedKvCache(layers=1, kv_heads=2, n_pages=4, page_size=page, max_rows=1,
                           pages_per_row=1, device="cpu")


def test_check_cu_seqlens_rejects_bad_offsets():
    """Host validation of ragged-prefill offsets (CPU tensors suffice: the
    check reads them on the host)."""
    import torch

    from qwenforge_amd.ops import check_cu_seqlens

    cu = torch.tensor([0, 3, 7, 12], dtype=torch.int32)
    check_cu_seqlens(cu, 12, 5)
    check_cu_seqlens(cu, 12, 5, lengths=[3, 4, 5])
    bad = [
        (torch.tensor([0, 3, 7, 11], dtype=torch.int32), 12, 5, None),   # does not end at T
        (torch.tensor([1, 3, 7, 12], dtype=torch.int32), 12, 5, None),   # does not start at 0
        (torch.tensor([0, 8, 7, 12], dtype=torch.int32), 12, 8, None),   # decreasing
        (cu, 12, 4, None),                                              # a row longer than max_seqlen
        (cu, 12, 5, [3, 4]),                                            # lengths of the wrong row count
    ]
    for c, total, mx, lengths in bad:
        with pytest.raises(ValueError):
            check_cu_seqlens(c, total, mx, lengths)
