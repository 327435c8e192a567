"""Paged KV cache: page pools, block tables and the paged attention-path ops.

The reference engine keeps one dense ``(B, KVH, cap, 64)`` cache per layer
and right-pads ragged batches (SE:1162-1204, SE:1263-1319); block-level KV
management is on its roadmap ("PagedAttention & Continuous Batching",
README.md:144).  Here the caches of all layers are page pools
``(n_pages, KVH, page_size, 64)`` fp16 and one int32 block table per batch
maps a row's logical pages to physical pages, so rows have no padding holes
and can be admitted and retired independently.  The ops call the C ABI in
``include/qf_paged.h``; like ``ops``, nothing computes on the host.

* ``PagedKvCache`` -- pools for every layer, the device block table and a
  host free list of pages.
* ``flash_decode_attention_paged`` / ``flash_decode_split_paged`` -- split-K
  decode (SE:834-874 semantics) through the block table.
* ``rope_append_paged`` -- one-token RoPE + append at a per-row slot.
* ``prefill_varlen_paged`` -- packed ragged prefill appending into pages.
* ``rms_qkv_rope_append_paged`` -- the fused decode-step QKV kernel appending
  into pages.
"""

from __future__ import annotations

import torch

from . import _lib
from .ops import HEAD_DIM, _ptr, _require_cuda_fp16, _scratch_args, _stream, check_cu_seqlens
from .step_ops import PACK_ROPE, _batch, _check, _rows, _weight, rope_args

MIN_PAGE, MAX_PAGE = 64, 4096


def _check_page_size(page_size: int) -> None:
    if not (MIN_PAGE <= page_size <= MAX_PAGE) or page_size & (page_size - 1):
        raise ValueError(f"page_size must be a power of two in [{MIN_PAGE}, {MAX_PAGE}] (got {page_size})")


class PagedKvCache:
    """Page pools of ``layers`` layers plus the block table of up to ``max_rows`` rows.

    ``pools[i] = (k_pool, v_pool)``, each ``(n_pages, kv_heads, page_size, 64)``
    fp16, zero-initialised.  ``table`` is ``(max_rows, pages_per_row)`` int32 on
    the device; unmapped entries hold -1.  Pages are handed out from a host
    free list (lowest id first); ``map_row`` / ``release_row`` update the
    device table with one small copy each, so they belong between graph
    replays, not inside them.
    """

    def __init__(self, layers: int, kv_heads: int, n_pages: int, page_size: int, max_rows: int,
                 pages_per_row: int, device, dtype=torch.float16):
        _check_page_size(page_size)
        if n_pages < 1 or max_rows < 1 or pages_per_row < 1:
            raise ValueError("need n_pages, max_rows and pages_per_row >= 1")
        self.page_size = page_size
        self.n_pages = n_pages
        self.kv_heads = kv_heads
        self.pages_per_row = pages_per_row
        self.device = torch.device(device)
        shape = (n_pages, kv_heads, page_size, HEAD_DIM)
        self.pools = [(torch.zeros(shape, device=self.device, dtype=dtype),
                       torch.zeros(shape, device=self.device, dtype=dtype)) for _ in range(layers)]
        self.table = torch.full((max_rows, pages_per_row), -1, device=self.device, dtype=torch.int32)
        self._free = list(range(n_pages))
        self._rows: dict[int, list[int]] = {}

    @property
    def capacity(self) -> int:
        """Logical slots per row."""
        return self.pages_per_row * self.page_size

    def free_pages(self) -> int:
        return len(self._free)

    def row_pages(self, row: int) -> list[int]:
        return list(self._rows.get(row, []))

    def map_row(self, row: int, n_slots: int) -> list[int]:
        """Make slots ``[0, n_slots)`` of ``row`` backed by pages (growing its
        mapping as needed); returns the row's page list."""
        need = -(-n_slots // self.page_size)
        if need > self.pages_per_row:
            raise ValueError(f"{n_slots} slots exceed the row capacity {self.capacity}")
        pages = self._rows.setdefault(row, [])
        if need - len(pages) > len(self._free):
            raise RuntimeError(f"page pool exhausted: need {need - len(pages)}, {len(self._free)} free")
        first = len(pages)
        while len(pages) < need:
            pages.append(self._free.pop(0))
        if len(pages) > first:
            ids = torch.tensor(pages[first:], dtype=torch.int32)
            self.table[row, first:len(pages)].copy_(ids)
        return list(pages)

    def release_row(self, row: int) -> None:
        """Return the row's pages to the free list and unmap it."""
        pages = self._rows.pop(row, [])
        self._free.extend(pages)
        self._free.sort()
        self.table[row].fill_(-1)

    def gather(self, layer: int, row: int, length: int):
        """Slots ``[0, length)`` of ``row`` as dense ``(KVH, length, 64)`` K and V
        (device indexing; for inspection and tests)."""
        k_pool, v_pool = self.pools[layer]
        pages = torch.tensor(self._rows[row], device=self.device, dtype=torch.long)
        slot = torch.arange(length, device=self.device)
        page = pages[slot // self.page_size]
        off = slot % self.page_size
        return k_pool[page, :, off].transpose(0, 1), v_pool[page, :, off].transpose(0, 1)


# --------------------------------------------------------------------------
# argument helpers
# --------------------------------------------------------------------------

def _pool_args(k_pool: torch.Tensor, v_pool: torch.Tensor, block_table: torch.Tensor, batch: int):
    """Validate the pools and the (B, pages_per_row) table; returns the ABI pieces."""
    _require_cuda_fp16("k_pool", k_pool, 4)
    _require_cuda_fp16("v_pool", v_pool, 4)
    if v_pool.shape != k_pool.shape:
        raise ValueError("k_pool and v_pool must have the same shape")
    n_pages, _, page_size, _ = k_pool.shape
    _check_page_size(page_size)
    if not isinstance(block_table, torch.Tensor) or block_table.dtype != torch.int32:
        raise TypeError("block_table must be an int32 tensor")
    if block_table.device != k_pool.device:
        raise RuntimeError("block_table must be on the pools' device")
    if block_table.dim() != 2 or block_table.shape[0] != batch or block_table.stride(1) != 1:
        raise ValueError(f"block_table must be (B={batch}, pages_per_row) with unit inner stride")
    ppr = block_table.shape[1]
    return ((k_pool.data_ptr(), k_pool.stride(0), k_pool.stride(1), k_pool.stride(2),
             v_pool.data_ptr(), v_pool.stride(0), v_pool.stride(1), v_pool.stride(2),
             block_table.data_ptr(), block_table.stride(0), ppr, n_pages, page_size),
            ppr * page_size)


def _slot_args(slots: torch.Tensor, batch: int, device):
    if not isinstance(slots, torch.Tensor) or slots.dtype != torch.int64 or slots.device != device:
        raise TypeError("slots must be an int64 device tensor")
    if slots.dim() != 1 or slots.numel() != batch:
        raise ValueError(f"slots must hold one slot per row ({batch})")
    return slots.data_ptr(), slots.stride(0)


# --------------------------------------------------------------------------
# decode
# --------------------------------------------------------------------------

def _paged_decode_args(grouped, k_pool, v_pool, block_table, attn_bias, flash, kv_last):
    b = grouped.shape[0]
    pool, cap = _pool_args(k_pool, v_pool, block_table, b)
    kvh = grouped.shape[1]
    if k_pool.shape[1] != kvh:
        raise ValueError(f"pools hold {k_pool.shape[1]} kv heads, grouped {kvh}")
    acc, m, l, out, ticket, splits, _, kv_last_sb = _scratch_args(
        grouped, cap, attn_bias, flash, kv_last)
    head = (grouped.data_ptr(), grouped.stride(0), grouped.stride(1), grouped.stride(2))
    bias = (_ptr(attn_bias), 0 if attn_bias is None else attn_bias.stride(0),
            _ptr(kv_last), kv_last_sb)
    return head, pool, bias, acc, m, l, out, ticket, splits


def flash_decode_attention_paged(grouped: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                                 block_table: torch.Tensor, attn_bias: torch.Tensor | None, flash,
                                 kv_last: torch.Tensor | None = None,
                                 scale: float | None = None) -> torch.Tensor:
    """``flash_decode_attention`` over paged caches (SE:834-874 semantics).

    grouped (B, KVH, G, 64); pools (n_pages, KVH, P, 64); block_table
    (B, pages_per_row) int32; attn_bias (B, pages_per_row * P) or None;
    ``flash`` as in ``ops.make_flash_scratch``; kv_last (1,) or (B,) int64
    bounds each row's slots.  Writes and returns ``flash[3]``.
    """
    head, pool, bias, acc, m, l, out, ticket, splits = _paged_decode_args(
        grouped, k_pool, v_pool, block_table, attn_bias, flash, kv_last)
    b, kvh, g, d = grouped.shape
    scale = d ** -0.5 if scale is None else scale
    with torch.cuda.device(grouped.device):
        rc = _lib.load().qf_decode_attn_paged(
            *head, *pool, *bias, acc.data_ptr(), m.data_ptr(), l.data_ptr(), splits, _ptr(ticket),
            out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
            b, kvh, g, d, float(scale), _stream(grouped.device))
    _lib.check(rc, "qf_decode_attn_paged")
    return out


def flash_decode_split_paged(grouped, k_pool, v_pool, block_table, attn_bias, flash, kv_last=None,
                             scale=None):
    """The split launch alone over paged caches: fills ``flash[0:3]`` = (acc, m, l)."""
    head, pool, bias, acc, m, l, _, _, splits = _paged_decode_args(
        grouped, k_pool, v_pool, block_table, attn_bias, flash, kv_last)
    b, kvh, g, d = grouped.shape
    scale = d ** -0.5 if scale is None else scale
    with torch.cuda.device(grouped.device):
        rc = _lib.load().qf_decode_split_paged(
            *head, *pool, *bias, acc.data_ptr(), m.data_ptr(), l.data_ptr(), splits,
            b, kvh, g, d, float(scale), _stream(grouped.device))
    _lib.check(rc, "qf_decode_split_paged")
    return acc, m, l


# --------------------------------------------------------------------------
# appends and prefill
# --------------------------------------------------------------------------

def rope_append_paged(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                      cos: torch.Tensor, sin: torch.Tensor, k_pool: torch.Tensor,
                      v_pool: torch.Tensor, block_table: torch.Tensor, slots: torch.Tensor,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """``ops.rope_append`` (SE:927-932) into paged caches at per-row slots.

    query (B, QH, 1, 64), key/value (B, KVH, 1, 64); cos/sin hold B*64 values
    (each row's own position); slots (B,) int64 on the device.  Returns
    rope(query) as (B, QH, 1, 64).
    """
    for n, t in (("query", query), ("key", key), ("value", value)):
        _require_cuda_fp16(n, t, 4)
    b, qh, tq, d = query.shape
    kvh = key.shape[1]
    if tq != 1 or key.shape != (b, kvh, 1, d) or value.shape != key.shape:
        raise ValueError("one token: query (B, QH, 1, D), key/value (B, KVH, 1, D)")
    pool, _ = _pool_args(k_pool, v_pool, block_table, b)
    if k_pool.shape[1] != kvh:
        raise ValueError("pools' kv heads do not match key")
    slot = _slot_args(slots, b, query.device)
    cos2, sin2 = cos.reshape(b, d), sin.reshape(b, d)
    for n, t in (("cos", cos2), ("sin", sin2)):
        if t.dtype != torch.float16 or t.device != query.device or t.stride(1) != 1:
            raise ValueError(f"{n} must be fp16 on the query's device with unit last stride")
    if cos2.stride(0) != sin2.stride(0):
        cos2, sin2 = cos2.contiguous(), sin2.contiguous()
    if out is None:
        out = torch.empty((b, qh, 1, d), device=query.device, dtype=query.dtype)
    with torch.cuda.device(query.device):
        rc = _lib.load().qf_rope_append_paged(
            query.data_ptr(), query.stride(0), query.stride(1),
            key.data_ptr(), key.stride(0), key.stride(1),
            value.data_ptr(), value.stride(0), value.stride(1),
            cos2.data_ptr(), sin2.data_ptr(), cos2.stride(0),
            *pool, *slot, out.data_ptr(), out.stride(0), out.stride(1),
            b, qh, kvh, d, _stream(query.device))
    _lib.check(rc, "qf_rope_append_paged")
    return out


def prefill_varlen_paged(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                         cu_seqlens: torch.Tensor, max_seqlen: int, cos: torch.Tensor | None,
                         sin: torch.Tensor | None, k_pool: torch.Tensor, v_pool: torch.Tensor,
                         block_table: torch.Tensor, start_pos: int = 0,
                         lengths=None) -> torch.Tensor:
    """``ops.prefill_varlen`` appending into paged caches.

    Packed query (T, QH, 64), key/value (T, KVH, 64); cu_seqlens (B+1,) int32
    on the device; optional per-token cos/sin (T, 64).  Token i of row b goes
    to logical slot start_pos + i of row b (start_pos a multiple of 64), then
    each row attends causally over its own tokens.  Returns (T, QH, 64).
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
    if start_pos % 64:
        raise ValueError("start_pos must be a multiple of 64")
    pool, cap = _pool_args(k_pool, v_pool, block_table, b)
    if k_pool.shape[1] != kvh:
        raise ValueError("pools' kv heads do not match key")
    if start_pos + max_seqlen > cap:
        raise ValueError(f"start_pos + max_seqlen exceeds the row capacity {cap}")
    cs_sn = 0
    if (cos is None) != (sin is None):
        raise ValueError("cos and sin go together")
    if cos is not None:
        for n, t in (("cos", cos), ("sin", sin)):
            _require_cuda_fp16(n, t, 2)
            if t.shape[0] != t_:
                raise ValueError(f"{n} must be (T, 64)")
        if cos.stride(0) != sin.stride(0):
            cos, sin = cos.contiguous(), sin.contiguous()
        cs_sn = cos.stride(0)
    out = torch.empty((t_, qh, d), device=query.device, dtype=torch.float16)
    with torch.cuda.device(query.device):
        rc = _lib.load().qf_prefill_varlen_paged(
            query.data_ptr(), query.stride(1), query.stride(0),
            key.data_ptr(), key.stride(1), key.stride(0),
            value.data_ptr(), value.stride(1), value.stride(0),
            cu_seqlens.data_ptr(), t_, int(max_seqlen),
            _ptr(cos), _ptr(sin), cs_sn,
            *pool, int(start_pos),
            out.data_ptr(), out.stride(1), out.stride(0),
            b, qh, kvh, d, float(d ** -0.5), _stream(query.device))
    _lib.check(rc, "qf_prefill_varlen_paged")
    return out


def rms_qkv_rope_append_paged(x: torch.Tensor, norm_w: torch.Tensor, eps: float,
                              w_qkv, bias: torch.Tensor | None,
                              cos: torch.Tensor | None, sin: torch.Tensor | None,
                              k_pool: torch.Tensor, v_pool: torch.Tensor,
                              block_table: torch.Tensor, slots: torch.Tensor,
                              q_out: torch.Tensor, token: torch.Tensor | None = None,
                              hidden_out: torch.Tensor | None = None, positions=None) -> None:
    """``step_ops.rms_qkv_rope_append`` appending into paged caches at per-row
    ``slots`` (B,) int64; RoPE from cos/sin tables or ``positions =
    (pos, inv_freq)`` as there."""
    _check("q_out", q_out)
    if q_out.dim() != 3 or q_out.shape[2] != HEAD_DIM or q_out.stride(2) != 1:
        raise ValueError(f"q_out must be (B, QH, 64) (got {tuple(q_out.shape)})")
    b, qh = q_out.shape[0], q_out.shape[1]
    _batch(b)
    pool, _ = _pool_args(k_pool, v_pool, block_table, b)
    kvh = k_pool.shape[1]
    hidden = norm_w.shape[0]
    _check("norm_w", norm_w)
    w_ptr, w_layout = _weight("w_qkv", w_qkv, (qh + 2 * kvh) * HEAD_DIM, hidden, PACK_ROPE)
    if bias is not None:
        _check("bias", bias)
        if tuple(bias.shape) != ((qh + 2 * kvh) * HEAD_DIM,) or not bias.is_contiguous():
            raise ValueError("bias must be contiguous ((QH + 2 KVH) * 64,)")
    rope = rope_args(cos, sin, positions, b)
    slot = _slot_args(slots, b, q_out.device)
    if token is not None:
        _check("token", token, torch.int64)
        if token.shape != (b,) or not token.is_contiguous():
            raise ValueError("token must be contiguous (B,)")
        _check("x", x)
        if x.dim() != 2 or x.shape[1] != hidden or x.stride(1) != 1:
            raise ValueError("embedding table must be (vocab, hidden)")
        x_sb = x.stride(0)
        ho_sb = _rows("hidden_out", hidden_out, b, hidden) if hidden_out is not None else 0
    else:
        x_sb = _rows("x", x, b, hidden)
        ho_sb = 0
        hidden_out = None
    rc = _lib.load().qf_rms_qkv_rope_append_paged(
        x.data_ptr(), x_sb, _ptr(token), _ptr(hidden_out), ho_sb,
        norm_w.data_ptr(), float(eps), w_ptr, w_layout, _ptr(bias), *rope, *pool, *slot,
        q_out.data_ptr(), q_out.stride(0), q_out.stride(1),
        b, hidden, qh, kvh, HEAD_DIM, _stream(x.device))
    _lib.check(rc, "qf_rms_qkv_rope_append_paged")
