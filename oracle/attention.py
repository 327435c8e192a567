"""CPU restatement of the reference attention maths (test infrastructure only).

All inputs are fp16 tensors as the engine stores them; every function upcasts
to ``acc_dtype`` (fp32 by default, fp64 for the tightest pins) and returns a
tensor in that dtype, i.e. the "fp32-accumulated" oracle the parity tolerance
(max-abs-err 2e-3 on fp16 outputs) is defined against.
"""

from __future__ import annotations

import math

import torch

# ``torch.finfo(torch.float16).min``: the additive bias the reference puts on
# empty cache slots (SE:1017-1020) and the fill of masked scores (SE:590-597).
FP16_MIN = float(torch.finfo(torch.float16).min)


def eager_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attention_mask: torch.Tensor | None = None,
    causal: bool = False,
    acc_dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """``StudentEngine._eager_attention`` (SE:579-599), fp32-accumulated.

    query (B, QH, Lq, D); key/value (B, KVH, Lk, D).  K/V heads are repeated
    ``QH // KVH`` times (``repeat_interleave`` on dim 1, so query head ``h``
    reads kv head ``h // G``).  Scores are ``Q @ K^T * D**-0.5``; the causal
    mask is bottom-right aligned (``tril(diagonal=Lk - Lq)``) and, like the
    optional boolean key mask, fills with the dtype minimum; softmax runs in
    fp32 (here: ``acc_dtype``) and the probabilities multiply V.
    """
    groups = query.shape[1] // key.shape[1]
    q = query.to(acc_dtype)
    k = key.to(acc_dtype).repeat_interleave(groups, dim=1)
    v = value.to(acc_dtype).repeat_interleave(groups, dim=1)
    scores = torch.matmul(q, k.transpose(-2, -1)) * (query.shape[-1] ** -0.5)
    fill = torch.finfo(acc_dtype).min
    if causal:
        lq, lk = scores.shape[-2:]
        keep = torch.ones((lq, lk), dtype=torch.bool).tril(diagonal=lk - lq)
        scores = scores.masked_fill(~keep, fill)
    if attention_mask is not None:
        scores = scores.masked_fill(~attention_mask, fill)
    probs = torch.softmax(scores, dim=-1)
    return torch.matmul(probs, v)


def eager_attention_fp16(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    causal: bool = True,
) -> torch.Tensor:
    """The reference's own fp16 form of ``_eager_attention`` (SE:579-599), for
    the CPU baseline of the prefill: K/V heads repeated G times, fp16 scores
    ``Q @ K^T * D**-0.5``, the bottom-right causal mask filled with the fp16
    minimum, ``softmax(scores.float())`` rounded to fp16, then fp16
    ``probabilities @ V``.  Returns fp16 (B, QH, Lq, D).
    """
    groups = query.shape[1] // key.shape[1]
    k = key.repeat_interleave(groups, dim=1)
    v = value.repeat_interleave(groups, dim=1)
    scores = torch.matmul(query, k.transpose(-2, -1)) * (query.shape[-1] ** -0.5)
    if causal:
        lq, lk = scores.shape[-2:]
        keep = torch.ones((lq, lk), dtype=torch.bool).tril(diagonal=lk - lq)
        scores = scores.masked_fill(~keep, torch.finfo(scores.dtype).min)
    probabilities = torch.softmax(scores.float(), dim=-1).to(query.dtype)
    return torch.matmul(probabilities, v)


def grouped_decode_attention(
    grouped: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    attn_bias: torch.Tensor | None = None,
    scale: float | None = None,
    acc_dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """Graph-step math attention (SE:939-972), fp32-accumulated.

    grouped (B, KVH, G, D) is the one-token query with the G query heads of a
    kv group on the row axis (SE:939); key/value caches are (B, KVH, cap, D);
    attn_bias (B, cap) is added to every score of its batch row
    (``bias.view(B, 1, 1, -1)``, SE:898 and SE:970).  Returns (B, KVH, G, D).
    """
    d = grouped.shape[-1]
    scale = d ** -0.5 if scale is None else scale
    q = grouped.to(acc_dtype)
    k = key_cache.to(acc_dtype)
    v = value_cache.to(acc_dtype)
    scores = torch.matmul(q, k.transpose(-2, -1)) * scale
    if attn_bias is not None:
        scores = scores + attn_bias.to(acc_dtype)[:, None, None, :]
    probs = torch.softmax(scores, dim=-1)
    return torch.matmul(probs, v)


def grouped_decode_attention_fp16(
    grouped: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    attn_bias: torch.Tensor | None = None,
    scale: float | None = None,
) -> torch.Tensor:
    """The reference's own fp16 form of the graph-step math attention
    (SE:968-971), for the CPU baseline: ``scores = (grouped @ K^T) * scale``
    and ``+ bias`` in fp16, ``softmax(scores.float())`` rounded to fp16, then
    ``probabilities @ V`` in fp16.  Returns fp16 (B, KVH, G, D).
    """
    d = grouped.shape[-1]
    scale = d ** -0.5 if scale is None else scale
    scores = torch.matmul(grouped, key_cache.transpose(-2, -1)) * scale
    if attn_bias is not None:
        scores = scores + attn_bias[:, None, None, :]
    probabilities = torch.softmax(scores.float(), dim=-1).to(grouped.dtype)
    return torch.matmul(probabilities, value_cache)


def split_partials(
    grouped: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    attn_bias: torch.Tensor | None,
    splits: int,
    scale: float | None = None,
    split_len: int | None = None,
    upper: int | None = None,
    acc_dtype: torch.dtype = torch.float32,
):
    """Per-split online-softmax partials of ``_flash_decode_split_kernel``
    (SE:32-115).

    Split ``s`` covers slots ``[s*split_len, min((s+1)*split_len, upper))``
    with ``split_len = ceil(cap / splits)`` (SE:851) unless given and
    ``upper = cap`` unless given.  Scores are ``q.k * scale + bias``; slots
    outside the split are -inf (SE:86-89).  Returns ``acc`` (B, KVH, S, G, D)
    = sum_n p_n v_n, ``m`` (B, KVH, S, G) = max score (-inf for an empty
    split) and ``l`` = sum_n p_n, with ``p_n = exp(score_n - m)`` and p = 0
    where the score is -inf (SE:92-97).  The streaming rescale the kernel does
    tile by tile is algebraically the same as this one-shot form.
    """
    b, kvh, g, d = grouped.shape
    cap = key_cache.shape[2]
    scale = d ** -0.5 if scale is None else scale
    upper = cap if upper is None else upper
    split_len = (cap + splits - 1) // splits if split_len is None else split_len
    q = grouped.to(acc_dtype)
    k = key_cache.to(acc_dtype)
    v = value_cache.to(acc_dtype)
    scores = torch.matmul(q, k.transpose(-2, -1)) * scale  # (B, KVH, G, cap)
    if attn_bias is not None:
        scores = scores + attn_bias.to(acc_dtype)[:, None, None, :]
    acc = torch.zeros((b, kvh, splits, g, d), dtype=acc_dtype)
    m = torch.full((b, kvh, splits, g), float("-inf"), dtype=acc_dtype)
    l = torch.zeros((b, kvh, splits, g), dtype=acc_dtype)
    for s in range(splits):
        lo = s * split_len
        hi = min(lo + split_len, upper)
        if hi <= lo:
            continue
        sc = scores[..., lo:hi]
        ms = sc.max(dim=-1).values
        safe = torch.where(torch.isinf(ms) & (ms < 0), torch.zeros_like(ms), ms)
        p = torch.exp(sc - safe[..., None])
        p = torch.where(torch.isinf(sc) & (sc < 0), torch.zeros_like(p), p)
        acc[:, :, s] = torch.matmul(p, v[:, :, lo:hi])
        m[:, :, s] = ms
        l[:, :, s] = p.sum(dim=-1)
    return acc, m, l


def combine_partials(acc: torch.Tensor, m: torch.Tensor, l: torch.Tensor) -> torch.Tensor:
    """``_flash_decode_combine_kernel`` (SE:117-162): log-sum-exp merge.

    ``m* = max_s m_s`` (0 if every split is empty); ``w_s = exp(m_s - m*)``
    (0 for an empty split); ``out = sum_s w_s acc_s / sum_s w_s l_s``.
    Input layout (B, KVH, S, G, D) / (B, KVH, S, G); returns (B, KVH, G, D).
    """
    m_glob = m.max(dim=2).values
    safe = torch.where(torch.isinf(m_glob) & (m_glob < 0), torch.zeros_like(m_glob), m_glob)
    w = torch.exp(m - safe[:, :, None, :])
    w = torch.where(torch.isinf(m) & (m < 0), torch.zeros_like(w), w)
    l_tot = (l * w).sum(dim=2)
    acc_tot = (acc * w[..., None]).sum(dim=2)
    return acc_tot / l_tot[..., None]


def flash_decode(
    grouped: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    attn_bias: torch.Tensor | None,
    splits: int,
    scale: float | None = None,
    acc_dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """Split + combine (SE:834-874) evaluated in ``acc_dtype``."""
    acc, m, l = split_partials(
        grouped, key_cache, value_cache, attn_bias, splits, scale, acc_dtype=acc_dtype
    )
    return combine_partials(acc, m, l)


def causal_prefill(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    scale: float | None = None,
    acc_dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """``_gqa_flash_prefill_kernel`` semantics (SE:164-251), fp32-accumulated.

    query (B, QH, S, D), key/value (B, KVH, S, D).  Query head ``h`` reads kv
    head ``h // G`` (SE:188); key position ``j`` is visible to query position
    ``i`` iff ``j <= i`` (SE:220, top-left aligned; with Lq == Lk this is the
    eager path's bottom-right mask).  V is addressed with its own layout (the
    true ``softmax(QK^T)V``), not with K's strides.
    """
    b, qh, s, d = query.shape
    groups = qh // key.shape[1]
    scale = d ** -0.5 if scale is None else scale
    q = query.to(acc_dtype)
    k = key.to(acc_dtype).repeat_interleave(groups, dim=1)
    v = value.to(acc_dtype).repeat_interleave(groups, dim=1)
    scores = torch.matmul(q, k.transpose(-2, -1)) * scale
    keep = torch.ones((s, s), dtype=torch.bool).tril()
    scores = scores.masked_fill(~keep, float("-inf"))
    probs = torch.softmax(scores, dim=-1)
    return torch.matmul(probs, v)


def brute_force_attention_fp64(q_rows, keys, values, scale, bias=None):
    """Pure-Python fp64 softmax attention for tiny shapes (pin for the above).

    q_rows: list of query vectors; keys/values: lists of vectors; bias: list
    (per key) or None.  Returns a list of output vectors.
    """
    out = []
    for q in q_rows:
        scores = []
        for j, k in enumerate(keys):
            s = sum(float(a) * float(b) for a, b in zip(q, k)) * scale
            if bias is not None:
                s += float(bias[j])
            scores.append(s)
        mx = max(scores)
        w = [math.exp(s - mx) for s in scores]
        tot = sum(w)
        row = [sum(w[j] * float(values[j][c]) for j in range(len(keys))) / tot
               for c in range(len(values[0]))]
        out.append(row)
    return out
