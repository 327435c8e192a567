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
