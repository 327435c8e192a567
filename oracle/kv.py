"""CPU restatement of the KV-cache append and slot bookkeeping (test infrastructure only)."""

from __future__ import annotations

import torch

from .attention import FP16_MIN


def append_decode(key_cache, value_cache, key, value, write_index):
    """``cache.index_copy_(2, write_index, new)`` for K and V (SE:930-932).

    key_cache/value_cache (B, KVH, cap, D) are updated in place (clones are
    the caller's business); key/value (B, KVH, 1, D); write_index is a
    one-element int64 tensor: every batch row writes the same slot.
    """
    slot = int(write_index.reshape(-1)[0])
    key_cache.index_copy_(2, torch.tensor([slot]), key)
    value_cache.index_copy_(2, torch.tensor([slot]), value)
    return key_cache, value_cache


def append_prefill(key_cache, value_cache, key, value, start: int = 0):
    """``cache[:, :, start:start+S].copy_(new)`` (SE:715-716 with start 0)."""
    s = key.shape[2]
    key_cache[:, :, start:start + s].copy_(key)
    value_cache[:, :, start:start + s].copy_(value)
    return key_cache, value_cache


def capacity(prompt_len: int, new_tokens: int, graph: bool = True, multiple: int = 64) -> int:
    """KV capacity rule of ``_generate_batch`` (SE:1263-1273).

    ``cap = P + max(N - 1, 0)``, at least P; rounded up to ``multiple`` on the
    graph-decode path.
    """
    cap = max(prompt_len + max(new_tokens - 1, 0), prompt_len)
    if graph:
        cap = (cap + multiple - 1) // multiple * multiple
    return cap


def decode_slots(max_prompt_len: int, max_new_tokens: int):
    """Shared cache slot written at each graph replay (SE:1126-1129).

    Step ``t`` in ``1..N-1`` writes slot ``P_max + t - 1``.
    """
    return [max_prompt_len + step - 1 for step in range(1, max_new_tokens)]


def decode_bias(lengths, max_prompt_len: int, cap: int, steps_done: int) -> torch.Tensor:
    """Additive decode bias after ``steps_done`` replays (SE:1017-1020, SE:1127).

    Row ``b`` is 0 on its prompt slots ``[0, len_b)`` and on the decode slots
    ``[P_max, P_max + steps_done)``, and fp16-min elsewhere (holes between
    ``len_b`` and ``P_max`` for right-padded rows).  Returns (B, cap) fp16.
    """
    bias = torch.full((len(lengths), cap), FP16_MIN, dtype=torch.float16)
    for b, n in enumerate(lengths):
        bias[b, :n] = 0.0
        bias[b, max_prompt_len:max_prompt_len + steps_done] = 0.0
    return bias


# --------------------------------------------------------------------------
# Paged layout (block table).  The reference keeps dense (B, KVH, cap, D)
# caches and lists block-level KV management only as a roadmap item
# (README.md:144), so this is the data contract of the paged kernels stated
# as plain indexing: logical slot s of row b lives in
# pool[table[b, s // P], :, s % P].
# --------------------------------------------------------------------------

def paged_location(table, b: int, slot: int, page_size: int):
    """(physical page, row in page) of logical slot ``slot`` of row ``b``."""
    return int(table[b, slot // page_size]), slot % page_size


def pages_to_dense(pool, table, lengths, cap: int):
    """Gather a paged pool (n_pages, KVH, P, D) into a dense (B, KVH, cap, D)
    cache: slots below ``lengths[b]`` come from the pages, the rest are zero
    (the dense caches are zero-initialised, SE:705-714)."""
    n_pages, kvh, page, d = pool.shape
    dense = torch.zeros(len(lengths), kvh, cap, d, dtype=pool.dtype)
    for b, n in enumerate(lengths):
        for s in range(n):
            p, r = paged_location(table, b, s, page)
            dense[b, :, s] = pool[p, :, r]
    return dense


def dense_to_pages(dense, table, lengths, n_pages: int, page_size: int):
    """Scatter slots ``[0, lengths[b])`` of a dense cache into a fresh zero pool."""
    b_, kvh, cap, d = dense.shape
    pool = torch.zeros(n_pages, kvh, page_size, d, dtype=dense.dtype)
    for b, n in enumerate(lengths):
        for s in range(n):
            p, r = paged_location(table, b, s, page_size)
            pool[p, :, r] = dense[b, :, s]
    return pool


def append_rows(key_cache, value_cache, key, value, slots):
    """Per-row decode append (each row at its own slot; a slot outside
    [0, cap) writes nothing): the no-holes form of SE:930-932 that a paged
    batch uses.  key/value (B, KVH, 1, D); caches updated in place."""
    cap = key_cache.shape[2]
    for b, s in enumerate(int(x) for x in slots):
        if 0 <= s < cap:
            key_cache[b, :, s] = key[b, :, 0]
            value_cache[b, :, s] = value[b, :, 0]
    return key_cache, value_cache
