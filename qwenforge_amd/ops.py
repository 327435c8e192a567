"""Torch-facing drop-ins for the reference engine's attention hot path.

Each function keeps the call signature ``student_engine.py`` uses today and
forwards raw device pointers, strides and the current HIP stream to the C ABI
(``include/qf_attn.h``).  Nothing here computes on the host: a missing
library or a CPU tensor raises.

* ``flash_decode_attention(grouped, key_cache, value_cache, attn_bias, flash)``
  -- ``StudentEngine._flash_decode_attention`` (SE:834-874).
* ``torch.ops.student_qwen.gqa_flash_prefill(query, key, value)``
  -- the custom op of SE:254-292 (same name, schema and fake).
* ``torch.ops.student_qwen.gqa_flash_prefill_rope_append(q, k, v, cos, sin,
  key_cache, value_cache, start_pos)`` -- prefill with RoPE and the slice
  append of SE:715-716 fused in.
* ``rope_append(q, k, v, cos, sin, key_cache, value_cache, write_index)``
  -- the graph step's RoPE + ``index_copy_`` append (SE:927-932).
* ``prefill_varlen(q, k, v, cu_seqlens, max_seqlen, cos, sin, key_cache,
  value_cache)`` -- the ragged prefill of ``_prefill_ragged`` (SE:1162-1204)
  over packed rows in one launch.
"""

from __future__ import annotations

import math

import torch

from . import _lib

HEAD_DIM = 64
MAX_GROUPS = 16
# MI355X: 256 compute units in 8 XCDs.  The planner reads the count from the
# device (a partitioned MI355X exposes fewer); this is the value it assumes
# where no device is visible (host-side planning, CPU tests).
NUM_CUS = 256
_CU_COUNT: dict = {}


def num_cus(device=None) -> int:
    """Compute units of ``device`` (default: the current HIP device), read once
    per device from its properties; ``NUM_CUS`` when no GPU is visible."""
    if not torch.cuda.is_available():
        return NUM_CUS
    idx = torch.cuda.current_device() if device is None else torch.device(device).index
    if idx is None:
        idx = torch.cuda.current_device()
    if idx not in _CU_COUNT:
        _CU_COUNT[idx] = int(torch.cuda.get_device_properties(idx).multi_processor_count)
    return _CU_COUNT[idx]


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _require_cuda_fp16(name: str, t: torch.Tensor, ndim: int | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be a HIP device tensor (got {t.device}); there is no CPU path")
    if t.dtype != torch.float16:
        raise TypeError(f"{name} must be float16 (got {t.dtype})")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name} must be {ndim}-D (got shape {tuple(t.shape)})")
    if t.shape[-1] != HEAD_DIM or t.stride(-1) != 1:
        raise ValueError(f"{name}: last dim must be {HEAD_DIM} with stride 1 (shape {tuple(t.shape)}, "
                         f"stride {t.stride()})")


# --------------------------------------------------------------------------
# decode
# --------------------------------------------------------------------------

def decode_plan(batch: int, kv_heads: int, length: int,
                cus: int | None = None) -> tuple[int, bool]:
    """(split count, single-launch merge) for a decode call over rows of
    ``length`` slots on a device with ``cus`` compute units (default: the
    current device's, ``num_cus()``; 256 on a whole MI355X, where every figure
    below was measured).  The workgroup bounds scale with the CU count: one
    workgroup per CU for split + combine, three per four CUs for the capped
    single launch, and the one-workgroup-per-CU fill past ``cus / 16`` pairs.

    Rows of at most 256 slots, any number of (b, kv head) pairs: one split,
    no merge (one workgroup per pair whose waves take a 32-key tile each and
    merge in LDS) -- measured on MI355X: B=1, L=128: 3.73 us against 5.27 for
    4 fused splits; B=1, L=256: 4.82 against 5.35 for 8; B=8, L=256: 4.99
    against 6.02 for 4; 24 pairs, L=256: 5.00 against 6.29 for 2; 64 pairs,
    L=256: 5.14 against 6.57 for 2 (from 320 slots the single-launch merge
    wins: B=1, L=320: 5.54 for 8 fused splits against 5.80; 24 pairs,
    L=512: 6.59 for 4 against 7.08).

    Longer rows, up to 16 pairs (measured on MI355X, graph-replayed calls
    over caches rotated past the MALL, every split count from 4 to 256 in both
    merge modes at 1-8 rows and 512-32768 slots):

    * short rows (``length <= 2048`` with at most 8 pairs, or ``<= 512``):
      the single-launch merge.  With at most 8 pairs, splits of 32 keys (64
      with more than 2 pairs), at most 16 -- e.g. config 1 (B=1, L=512): 16
      splits (5.46 us against 5.58 at 8 and 6.23 for 16 split + combine);
      B=1, L=2048: 16 (6.23 against 6.47 for 64 split + combine); config 2
      (B=4, cap 2048, ragged with a bias): 16 (7.00 against 7.31 for 32 split
      + combine; re-measured single launches: 16 6.83-6.85, 8 7.34-7.35, 12
      6.91, 20 7.33, 24 7.49, 32 8.06).  With more pairs, splits of 128 keys, at most 192
      workgroups -- e.g. B=8, L=512: 4 (6.55 against 6.72 for 16 split +
      combine);
    * longer rows: split + combine launches with one workgroup per CU
      (``NUM_CUS // pairs`` splits), at most 128 splits and none shorter than
      64 keys -- e.g. config 3 (B=1, L=32768): 128 (9.24 us); B=4, L=4096: 32
      (7.84 against 8.25 for 16 fused splits); B=4, L=16384: 32 (11.79
      against 12.44 for 128); B=8, L=1536: 16 (7.53 against 8.08 for 12
      fused); B=5, L=5000: 25 (8.82 against 9.51 for 39).  Write-through
      partials and non-temporal tile loads made the two launches the faster
      form here: the combine launch now costs less than the single-launch
      merge's serial tail.

    Longer rows, more pairs: one workgroup per CU (``_fill_splits``), single launch.  (The reference's
    rule, ``max(1, min(32, 272 // (B*KVH), cap // 256))`` at SE:1027, targets
    68 SMs and always uses two launches.)
    """
    cus = num_cus() if cus is None else max(1, int(cus))
    pairs = max(1, batch * kv_heads)
    if length <= 256:
        return 1, False
    if pairs > max(1, cus // 16):
        s = _fill_splits(pairs, length, target_workgroups=cus)
        return s, prefer_fused(s)
    if pairs <= 8 and length <= 2048:
        keys = 32 if pairs <= 2 else 64
        s = max(1, min(math.ceil(length / keys), 16, max(1, 3 * cus // 4 // pairs)))
        return s, s > 1
    if length <= 512:
        s = max(1, min(math.ceil(length / 128), 3 * cus // 4 // pairs, 32))
        return s, s > 1
    s = max(1, min(cus // pairs, 128, math.ceil(length / 64)))
    return s, False


def choose_splits(batch: int, kv_heads: int, length: int, cus: int | None = None) -> int:
    """Split count of ``decode_plan``."""
    return decode_plan(batch, kv_heads, length, cus)[0]


def _fill_splits(pairs: int, length: int, min_keys: int = 128,
                 target_workgroups: int = NUM_CUS) -> int:
    """Split count for more than 16 (b, kv head) pairs.

    The (split, b, kv-head) workgroups fill the CUs once -- floor(CUs / pairs)
    splits -- never a count just above it (which leaves a few CUs with a
    second workgroup: B=12 L=5760 at 11 splits, 264 workgroups, took 16.7 us
    against 13.1 at 10).  Splits are never shorter than ``min_keys`` slots.
    Measured on MI355X with the single-launch merge, one workgroup per CU
    against two (twice the splits): B=12 L=5760 12.55 vs 13.35 us; B=16
    L=4096 11.58 vs 13.13; B=10 L=4096 10.51 vs 11.94; B=12 L=2048 8.94 vs
    9.99; B=24 L=2048 10.23 vs 10.97; B=12 L=8192 14.83 vs 15.81.
    """
    by_len = max(1, math.ceil(length / min_keys))
    s = max(1, target_workgroups // pairs)
    return max(1, min(by_len, s, 1024))


def prefer_fused(splits: int) -> bool:
    """Merge mode for an explicit split count without a shape: the
    single-launch merge (the last workgroup of each (b, kv head) merges) up to
    32 splits, where each of its lanes folds at most eight partials in one
    round trip; above that the second (combine) launch is cheaper (measured on
    MI355X).  ``decode_plan`` picks the mode per shape."""
    return 1 < splits <= 32


def make_flash_scratch(batch: int, kv_heads: int, groups: int, capacity: int,
                       device, splits: int | None = None, fused: bool | None = None,
                       head_dim: int = HEAD_DIM):
    """Static scratch for ``flash_decode_attention`` (cf. SE:1028-1045).

    Returns ``(acc, m, l, out)`` -- the reference's tuple -- plus a zeroed
    int32 ``ticket`` (``ticket_size`` counters) when ``fused`` (single-launch
    merge).  Defaults: ``decode_plan`` for the shape when ``splits`` is None,
    else ``prefer_fused(splits)``.  All addresses stay fixed, so the tuple can
    be captured into a hipGraph.
    """
    if splits is None:
        splits, planned = decode_plan(batch, kv_heads, capacity, num_cus(device))
        fused = planned if fused is None else fused
    fused = prefer_fused(splits) if fused is None else fused
    f32 = dict(device=device, dtype=torch.float32)
    acc = torch.zeros(batch, kv_heads, splits, groups, head_dim, **f32)
    m = torch.zeros(batch, kv_heads, splits, groups, **f32)
    l = torch.zeros(batch, kv_heads, splits, groups, **f32)
    out = torch.zeros(batch, kv_heads, groups, head_dim, device=device, dtype=torch.float16)
    if not fused:
        return acc, m, l, out
    ticket = torch.zeros(ticket_size(batch, kv_heads, splits), device=device, dtype=torch.int32)
    return acc, m, l, out, ticket


def ticket_size(batch: int, kv_heads: int, splits: int) -> int:
    """int32 counters the single-launch merge needs: one per (b, kv head).

    ``splits`` does not change the count (the workgroup that completes a
    (b, h) counter merges all of its partials); it stays in the signature so
    callers size the ticket from the same arguments as the partials."""
    del splits
    return batch * kv_heads


def decode_kernel_name(batch: int, kv_heads: int, groups: int, capacity: int, splits: int,
                       fused: bool, bias: str = "vec", paged: bool = False) -> str:
    """Name of the split-kernel instance a decode call launches, from the
    library's own launch plan (``qf_decode_waves``): decode_split_kernel<waves,
    bias (0 none, 1 16-byte vector, 2 scalar), mode (0 direct, 1 partial, 2
    single-launch merge), paged>."""
    waves = _lib.load().qf_decode_waves(batch, kv_heads, groups, capacity, splits, int(fused))
    _lib.check(min(waves, 0), "qf_decode_waves")
    mode = 0 if splits == 1 else (2 if fused else 1)
    kind = {"none": 0, "vec": 1, "scalar": 2}[bias]
    return f"qf::decode_split_kernel<{waves}, {kind}, {mode}, {str(paged).lower()}>"


def _decode_args(grouped, key_cache, value_cache, attn_bias, flash, kv_last):
    """Validate the decode operands; returns the parsed pieces."""
    _require_cuda_fp16("grouped", grouped, 4)
    _require_cuda_fp16("key_cache", key_cache, 4)
    _require_cuda_fp16("value_cache", value_cache, 4)
    b, kvh = grouped.shape[:2]
    if key_cache.shape[:2] != (b, kvh) or value_cache.shape != key_cache.shape:
        raise ValueError(f"cache shape {tuple(key_cache.shape)} / {tuple(value_cache.shape)} "
                         f"does not match grouped {tuple(grouped.shape)}")
    return _scratch_args(grouped, key_cache.shape[2], attn_bias, flash, kv_last)


def _scratch_args(grouped, cap, attn_bias, flash, kv_last):
    """Validate the query, bias, bound and scratch operands of a decode call
    over ``cap`` slots per row; returns the parsed pieces."""
    acc, m, l, out = flash[:4]
    ticket = flash[4] if len(flash) > 4 else None
    _require_cuda_fp16("grouped", grouped, 4)
    _require_cuda_fp16("out", out, 4)
    b, kvh, g, d = grouped.shape
    splits = acc.shape[2]
    if acc.shape != (b, kvh, splits, g, d) or m.shape != (b, kvh, splits, g) or l.shape != m.shape:
        raise ValueError("flash scratch shapes do not match (B, KVH, S, G, D) / (B, KVH, S, G)")
    for name, t in (("acc", acc), ("m", m), ("l", l)):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.device != grouped.device:
            raise ValueError(f"flash scratch {name} must be contiguous fp32 on {grouped.device}")
    if out.shape != (b, kvh, g, d):
        raise ValueError(f"out must be {(b, kvh, g, d)}")
    if attn_bias is not None:
        if attn_bias.dtype != torch.float16 or attn_bias.device != grouped.device:
            raise TypeError("attn_bias must be fp16 on the same device")
        if attn_bias.dim() != 2 or attn_bias.shape != (b, cap) or attn_bias.stride(1) != 1:
            raise ValueError(f"attn_bias must be (B, cap) = {(b, cap)} with unit last stride")
    if ticket is not None:
        need = ticket_size(b, kvh, splits)
        if ticket.dtype != torch.int32 or ticket.numel() < need or not ticket.is_contiguous():
            raise ValueError(f"ticket must be a contiguous int32 tensor with {need} elements")
        if ticket.device != grouped.device:
            raise ValueError(f"ticket must be on {grouped.device} (got {ticket.device}): the "
                             "kernel increments it with device-scope atomics")
    kv_last_sb = 0
    if kv_last is not None:
        if kv_last.dtype != torch.int64 or kv_last.device != grouped.device:
            raise TypeError("kv_last must be an int64 device tensor")
        if kv_last.numel() == 1:
            kv_last_sb = 0
        elif kv_last.numel() == b and kv_last.dim() == 1:
            kv_last_sb = kv_last.stride(0)
        else:
            raise ValueError("kv_last must hold 1 or B elements")
    return acc, m, l, out, ticket, splits, cap, kv_last_sb


def _qkv_bias_args(grouped, key_cache, value_cache, attn_bias, kv_last, kv_last_sb):
    return (grouped.data_ptr(), grouped.stride(0), grouped.stride(1), grouped.stride(2),
            key_cache.data_ptr(), key_cache.stride(0), key_cache.stride(1), key_cache.stride(2),
            value_cache.data_ptr(), value_cache.stride(0), value_cache.stride(1), value_cache.stride(2),
            _ptr(attn_bias), 0 if attn_bias is None else attn_bias.stride(0),
            _ptr(kv_last), kv_last_sb)


def flash_decode_attention(grouped: torch.Tensor, key_cache: torch.Tensor,
                           value_cache: torch.Tensor, attn_bias: torch.Tensor | None,
                           flash, kv_last: torch.Tensor | None = None,
                           scale: float | None = None) -> torch.Tensor:
    """Drop-in for ``StudentEngine._flash_decode_attention`` (SE:834-874).

    grouped (B, KVH, G, D) fp16; key_cache/value_cache (B, KVH, cap, D) fp16;
    attn_bias (B, cap) fp16 additive bias or None; ``flash`` is the
    reference's ``(acc, m, l, out)`` static scratch -- the split count is
    ``acc.shape[2]`` as in the reference -- optionally followed by an int32
    ``ticket`` (see ``make_flash_scratch``) that selects the single-launch
    merge.  ``kv_last`` (optional, device int64, shape (1,) or (B,)) is the
    last slot that can be valid; slots after it are skipped (the engine passes
    its ``write_index``).  Writes and returns ``out``.
    """
    acc, m, l, out, ticket, splits, cap, kv_last_sb = _decode_args(
        grouped, key_cache, value_cache, attn_bias, flash, kv_last)
    b, kvh, g, d = grouped.shape
    scale = d ** -0.5 if scale is None else scale
    lib = _lib.load()
    with torch.cuda.device(grouped.device):
        rc = lib.qf_decode_attn(
            *_qkv_bias_args(grouped, key_cache, value_cache, attn_bias, kv_last, kv_last_sb),
            acc.data_ptr(), m.data_ptr(), l.data_ptr(), splits,
            _ptr(ticket),
            out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
            b, kvh, g, d, cap, float(scale), _stream(grouped.device))
    _lib.check(rc, "qf_decode_attn")
    return out


def flash_decode_split(grouped, key_cache, value_cache, attn_bias, flash, kv_last=None,
                       scale=None, split_capacity=False):
    """The split launch alone (``_flash_decode_split_kernel``, SE:32-115 / SE:854-865):
    fills the partials ``flash[0:3]`` = (acc, m, l).

    ``split_capacity``: split the capacity as the reference does (SE:851)
    with ``kv_last`` as a mask only (``qf_decode_split_capacity``), so the
    first loads do not wait for it -- for rows that fill most of the cache."""
    acc, m, l, out, _, splits, cap, kv_last_sb = _decode_args(
        grouped, key_cache, value_cache, attn_bias, flash, kv_last)
    b, kvh, g, d = grouped.shape
    scale = d ** -0.5 if scale is None else scale
    lib = _lib.load()
    name = "qf_decode_split_capacity" if split_capacity else "qf_decode_split"
    with torch.cuda.device(grouped.device):
        rc = getattr(lib, name)(
            *_qkv_bias_args(grouped, key_cache, value_cache, attn_bias, kv_last, kv_last_sb),
            acc.data_ptr(), m.data_ptr(), l.data_ptr(), splits,
            b, kvh, g, d, cap, float(scale), _stream(grouped.device))
    _lib.check(rc, name)
    return acc, m, l


def flash_decode_combine(flash):
    """The combine launch alone (``_flash_decode_combine_kernel``, SE:117-162 /
    SE:866-873): merges the partials of ``flash`` into ``flash[3]``."""
    acc, m, l, out = flash[:4]
    _require_cuda_fp16("out", out, 4)
    b, kvh, splits, g, d = acc.shape
    for name, t in (("acc", acc), ("m", m), ("l", l)):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.device != out.device:
            raise ValueError(f"flash scratch {name} must be contiguous fp32 on {out.device}")
    if m.shape != (b, kvh, splits, g) or l.shape != m.shape or out.shape != (b, kvh, g, d):
        raise ValueError("flash scratch shapes do not match")
    lib = _lib.load()
    with torch.cuda.device(out.device):
        rc = lib.qf_decode_combine(acc.data_ptr(), m.data_ptr(), l.data_ptr(), splits,
                                   out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
                                   b, kvh, g, d, _stream(out.device))
    _lib.check(rc, "qf_decode_combine")
    return out


def decode_attention(grouped, key_cache, value_cache, attn_bias=None, splits=None,
                     kv_last=None, fused=None):
    """Convenience wrapper: allocates scratch and runs ``flash_decode_attention``."""
    b, kvh, g, _ = grouped.shape
    flash = make_flash_scratch(b, kvh, g, key_cache.shape[2], grouped.device, splits, fused)
    return flash_decode_attention(grouped, key_cache, value_cache, attn_bias, flash, kv_last)


# --------------------------------------------------------------------------
# decode RoPE + append
# --------------------------------------------------------------------------

def _as_rows(name: str, t: torch.Tensor, batch: int) -> torch.Tensor:
    """View a per-row table ((B, D), (B, 1, D) or (B, 1, 1, D)) as (B, D)."""
    if t.numel() != batch * HEAD_DIM:
        raise ValueError(f"{name} must hold B*D = {batch * HEAD_DIM} values (shape {tuple(t.shape)})")
    return t.reshape(batch, HEAD_DIM)


def rope_append(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                cos: torch.Tensor, sin: torch.Tensor, key_cache: torch.Tensor,
                value_cache: torch.Tensor, write_index: torch.Tensor,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """RoPE + KV-cache append of the graph decode step (SE:927-932).

    query (B, QH, 1, D), key/value (B, KVH, 1, D) -- the transposed views of
    the fused QKV projection; cos/sin the per-step fp16 tables (B, 1, 1, D)
    (SE:912-915, any shape holding B*D values); caches (B, KVH, cap, D);
    write_index a one-element int64 device tensor.  Writes
    ``key_cache[:, :, slot] = rope(key)`` and ``value_cache[:, :, slot] =
    value`` with ``slot = write_index[0]`` read on the device, and returns
    ``rope(query)`` (a new (B, QH, 1, D) tensor, or ``out``).
    """
    for n, t in (("query", query), ("key", key), ("value", value),
                 ("key_cache", key_cache), ("value_cache", value_cache)):
        _require_cuda_fp16(n, t, 4)
    b, qh, tq, d = query.shape
    kvh = key.shape[1]
    if tq != 1 or key.shape != (b, kvh, 1, d) or value.shape != key.shape:
        raise ValueError("rope_append expects one token: query (B, QH, 1, D), key/value (B, KVH, 1, D)")
    if key_cache.shape[:2] != (b, kvh) or value_cache.shape != key_cache.shape:
        raise ValueError("cache shape does not match key")
    if write_index.dtype != torch.int64 or write_index.device != query.device:
        raise TypeError("write_index must be an int64 device tensor")
    cos2 = _as_rows("cos", cos, b)
    sin2 = _as_rows("sin", sin, b)
    for n, t in (("cos", cos2), ("sin", sin2)):
        if t.dtype != torch.float16 or t.device != query.device or t.stride(1) != 1:
            raise ValueError(f"{n} must be fp16 on the query's device with unit last stride")
    if cos2.stride(0) != sin2.stride(0):
        cos2, sin2 = cos2.contiguous(), sin2.contiguous()
    if out is None:
        out = torch.empty((b, qh, 1, d), device=query.device, dtype=query.dtype)
    lib = _lib.load()
    with torch.cuda.device(query.device):
        rc = lib.qf_rope_append(
            query.data_ptr(), query.stride(0), query.stride(1),
            key.data_ptr(), key.stride(0), key.stride(1),
            value.data_ptr(), value.stride(0), value.stride(1),
            cos2.data_ptr(), sin2.data_ptr(), cos2.stride(0),
            key_cache.data_ptr(), key_cache.stride(0), key_cache.stride(1), key_cache.stride(2),
            value_cache.data_ptr(), value_cache.stride(0), value_cache.stride(1), value_cache.stride(2),
            write_index.data_ptr(),
            out.data_ptr(), out.stride(0), out.stride(1),
            b, qh, kvh, d, key_cache.shape[2], _stream(query.device))
    _lib.check(rc, "qf_rope_append")
    return out


# --------------------------------------------------------------------------
# prefill
# --------------------------------------------------------------------------

def _prefill_launch(query, key, value, out, cos=None, sin=None, key_cache=None,
                    value_cache=None, start_pos=0):
    for n, t in (("query", query), ("key", key), ("value", value), ("out", out)):
        _require_cuda_fp16(n, t, 4)
    b, qh, s, d = query.shape
    kvh = key.shape[1]
    if key.shape != (b, kvh, s, d) or value.shape != key.shape or qh % kvh != 0:
        raise ValueError(f"prefill shapes: query {tuple(query.shape)}, key {tuple(key.shape)}, "
                         f"value {tuple(value.shape)}")
    cs_sb = cs_sn = 0
    if cos is not None or sin is not None:
        if cos is None or sin is None:
            raise ValueError("cos and sin go together")
        # Accept (S, D), (B, S, D) or the engine's (B, 1, S, D).
        def table(n, t):
            _require_cuda_fp16(n, t)
            if t.dim() == 4:
                t = t.squeeze(1)
            if t.dim() == 2:
                t = t.unsqueeze(0)
            if t.dim() != 3 or t.shape[1] != s or t.shape[0] not in (1, b):
                raise ValueError(f"{n} must be (S, D), (B, S, D) or (B, 1, S, D) for S={s}")
            return t
        cos, sin = table("cos", cos), table("sin", sin)
        if cos.stride() != sin.stride() or cos.shape != sin.shape:
            cos, sin = cos.contiguous(), sin.contiguous()
        cs_sb = 0 if cos.shape[0] == 1 else cos.stride(0)
        cs_sn = cos.stride(1)
    cap = 0
    if key_cache is not None or value_cache is not None:
        if key_cache is None or value_cache is None:
            raise ValueError("key_cache and value_cache go together")
        _require_cuda_fp16("key_cache", key_cache, 4)
        _require_cuda_fp16("value_cache", value_cache, 4)
        cap = key_cache.shape[2]
        if key_cache.shape[:2] != (b, kvh) or value_cache.shape != key_cache.shape:
            raise ValueError("cache shape does not match key")
        if start_pos < 0 or start_pos + s > cap:
            raise ValueError(f"start_pos {start_pos} + S {s} exceeds cache capacity {cap}")
    kc_s = key_cache.stride()[:3] if key_cache is not None else (0, 0, 0)
    vc_s = value_cache.stride()[:3] if value_cache is not None else (0, 0, 0)
    lib = _lib.load()
    with torch.cuda.device(query.device):
        rc = lib.qf_prefill_attn(
            query.data_ptr(), *query.stride()[:3],
            key.data_ptr(), *key.stride()[:3],
            value.data_ptr(), *value.stride()[:3],
            _ptr(cos), _ptr(sin), cs_sb, cs_sn,
            _ptr(key_cache), *kc_s,
            _ptr(value_cache), *vc_s,
            int(start_pos), cap,
            out.data_ptr(), *out.stride()[:3],
            b, qh, kvh, s, d, float(d ** -0.5),
            _stream(query.device))
    _lib.check(rc, "qf_prefill_attn")
    return out


def check_cu_seqlens(cu_seqlens: torch.Tensor, total: int, max_seqlen: int,
                     lengths=None) -> None:
    """Host check of packed-row offsets before a ragged prefill launch.

    The kernels clamp each row to ``max_seqlen`` and to ``[0, total)`` so that
    nothing reads or writes out of bounds, but tokens past a row's clamp
    would be neither attended nor appended.  So: ``cu[0] == 0``, non-
    decreasing, ``cu[B] == total`` and no row longer than ``max_seqlen``.
    ``lengths`` (host ints, the rows' token counts) lets a caller that built
    ``cu_seqlens`` from them skip the device read; otherwise the offsets are
    copied to the host (a synchronisation), except under graph capture, where
    they cannot be read and the caller owns the precondition.
    """
    if lengths is not None:
        cu = [0]
        for n in lengths:
            cu.append(cu[-1] + int(n))
    elif cu_seqlens.is_cuda and torch.cuda.is_current_stream_capturing():
        return
    else:
        cu = [int(x) for x in cu_seqlens.tolist()]
    if len(cu) != cu_seqlens.numel():
        raise ValueError(f"cu_seqlens has {cu_seqlens.numel()} entries, lengths describe {len(cu)}")
    if cu[0] != 0 or cu[-1] != total:
        raise ValueError(f"cu_seqlens must start at 0 and end at T={total} (got {cu[0]}, {cu[-1]})")
    rows = [b - a for a, b in zip(cu, cu[1:])]
    if min(rows) < 0:
        raise ValueError("cu_seqlens must be non-decreasing")
    if max(rows) > max_seqlen:
        raise ValueError(f"a row holds {max(rows)} tokens > max_seqlen={max_seqlen}")


def prefill_varlen(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                   cu_seqlens: torch.Tensor, max_seqlen: int, cos: torch.Tensor | None = None,
                   sin: torch.Tensor | None = None, key_cache: torch.Tensor | None = None,
                   value_cache: torch.Tensor | None = None, start_pos: int = 0,
                   lengths=None) -> torch.Tensor:
    """Ragged causal prefill of packed rows (``_prefill_ragged``, SE:1162-1204, in one launch).

    query (T, QH, 64), key/value (T, KVH, 64): rows packed along the token axis;
    ``cu_seqlens`` (B+1,) int32 on the device: row b is tokens
    [cu[b], cu[b+1]).  Optional ``cos``/``sin`` (T, 64) per-token tables (each
    row's own positions) rotate q and k; with ``key_cache``/``value_cache``
    (B, KVH, cap, 64) token i of row b is written to slot start_pos + i of row
    b (RoPE needs the caches).  ``lengths`` (optional host ints) are the rows'
    token counts ``cu_seqlens`` was built from (see ``check_cu_seqlens``).
    Returns (T, QH, 64).
    """
    for n, t in (("query", query), ("key", key), ("value", value)):
        _require_cuda_fp16(n, t, 3)
    t_, qh, d = query.shape
    kvh = key.shape[1]
    if key.shape != (t_, kvh, d) or value.shape != key.shape or qh % kvh != 0:
        raise ValueError("packed prefill shapes: query (T, QH, D), key/value (T, KVH, D)")
    if cu_seqlens.dtype != torch.int32 or cu_seqlens.dim() != 1 or cu_seqlens.device != query.device:
        raise TypeError("cu_seqlens must be a 1-D int32 device tensor")
    b = cu_seqlens.numel() - 1
    if b < 1 or not 1 <= max_seqlen <= t_:
        raise ValueError(f"need B >= 1 rows and 1 <= max_seqlen <= T (got {b}, {max_seqlen})")
    check_cu_seqlens(cu_seqlens, t_, max_seqlen, lengths)
    cs_sn = 0
    if (cos is None) != (sin is None):
        raise ValueError("cos and sin go together")
    if cos is not None:
        for n, t in (("cos", cos), ("sin", sin)):
            _require_cuda_fp16(n, t, 2)
            if t.shape[0] != t_:
                raise ValueError(f"{n} must be (T, 64) per-token tables")
        if cos.stride() != sin.stride():
            cos, sin = cos.contiguous(), sin.contiguous()
        cs_sn = cos.stride(0)
    if (key_cache is None) != (value_cache is None):
        raise ValueError("key_cache and value_cache go together")
    cap = 0
    if key_cache is not None:
        _require_cuda_fp16("key_cache", key_cache, 4)
        _require_cuda_fp16("value_cache", value_cache, 4)
        cap = key_cache.shape[2]
        if key_cache.shape[:2] != (b, kvh) or value_cache.shape != key_cache.shape:
            raise ValueError("caches must be (B, KVH, cap, 64)")
        if start_pos < 0 or start_pos + max_seqlen > cap:
            raise ValueError("start_pos + max_seqlen exceeds the cache capacity")
    elif cos is not None:
        raise ValueError("rotated keys need the caches")
    out = torch.empty_like(query)
    kc_s = key_cache.stride()[:3] if key_cache is not None else (0, 0, 0)
    vc_s = value_cache.stride()[:3] if value_cache is not None else (0, 0, 0)
    lib = _lib.load()
    with torch.cuda.device(query.device):
        rc = lib.qf_prefill_varlen(
            query.data_ptr(), query.stride(1), query.stride(0),
            key.data_ptr(), key.stride(1), key.stride(0),
            value.data_ptr(), value.stride(1), value.stride(0),
            cu_seqlens.data_ptr(), t_, int(max_seqlen),
            _ptr(cos), _ptr(sin), cs_sn,
            _ptr(key_cache), *kc_s, _ptr(value_cache), *vc_s,
            int(start_pos), cap,
            out.data_ptr(), out.stride(1), out.stride(0),
            b, qh, kvh, d, float(d ** -0.5), _stream(query.device))
    _lib.check(rc, "qf_prefill_varlen")
    return out


@torch.library.custom_op("student_qwen::gqa_flash_prefill", mutates_args=())
def gqa_flash_prefill(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> torch.Tensor:
    """Causal GQA flash-prefill (SE:254-280): (B, QH, S, D) x (B, KVH, S, D)^2 -> (B, QH, S, D)."""
    out = torch.empty(query.shape, device=query.device, dtype=query.dtype)
    return _prefill_launch(query, key, value, out)


@gqa_flash_prefill.register_fake
def _gqa_flash_prefill_fake(query, key, value):
    return torch.empty(query.shape, device=query.device, dtype=query.dtype)


@torch.library.custom_op("student_qwen::gqa_flash_prefill_rope_append",
                         mutates_args=("key_cache", "value_cache"))
def gqa_flash_prefill_rope_append(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                                  cos: torch.Tensor, sin: torch.Tensor,
                                  key_cache: torch.Tensor, value_cache: torch.Tensor,
                                  start_pos: int) -> torch.Tensor:
    """Causal prefill on pre-RoPE q/k with RoPE and the cache append fused.

    Rotates q and k with the fp16 tables ``cos``/``sin`` ((S, D), (B, S, D) or
    (B, 1, S, D); SE:545-548), attends causally, writes the rotated k and the
    raw v to ``cache[:, :, start_pos:start_pos+S]`` (SE:715-716) and returns
    the attention output (B, QH, S, D), stored token-major ((B, S, QH, D)
    memory order, the layout o_proj consumes: ``out.transpose(1, 2)`` is
    contiguous, so the reshape to (B, S, hidden) copies nothing).
    """
    return _prefill_launch(query, key, value, _token_major_out(query), cos, sin, key_cache,
                           value_cache, start_pos)


def _token_major_out(query: torch.Tensor) -> torch.Tensor:
    """Uninitialised (B, QH, S, D) tensor laid out as (B, S, QH, D)."""
    b, qh, s, d = query.shape
    return torch.empty((b, s, qh, d), device=query.device, dtype=query.dtype).transpose(1, 2)


@gqa_flash_prefill_rope_append.register_fake
def _gqa_flash_prefill_rope_append_fake(query, key, value, cos, sin, key_cache, value_cache,
                                        start_pos):
    return _token_major_out(query)
