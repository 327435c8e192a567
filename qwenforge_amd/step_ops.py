"""Torch-facing wrappers of the fused decode-step kernels (``include/qf_step.h``).

They replace the torch op sequence inside the reference's graph step
``_decode_step_static`` (SE:896-982) for batches of 1..4 rows:

* ``rms_qkv_rope_append`` -- rms_norm + QKV linear (+bias) + eager RoPE +
  ``index_copy_`` append (SE:917-932); optionally gathers the embedding rows
  of ``token`` first (SE:896).
* ``gemv_residual`` -- ``hidden = residual + F.linear(inp, w)`` in place
  (o_proj SE:973-974, down_proj SE:978 / SE:666).
* ``attn_merge_o_proj`` -- the split-K decode merge (SE:117-162) folded into
  the o_proj + residual GEMV.
* ``rms_gate_up_swiglu`` -- rms_norm + gate/up linear + ``silu(gate) * up``
  (SE:976-977, SE:664-666).
* ``rms_lm_head`` + ``argmax_step`` -- final rms_norm, lm_head, argmax
  (SE:980-982) and the per-step slot/position/token bookkeeping that the
  reference does on the host between replays (SE:1126-1132).

Every function launches on the current HIP stream and returns nothing but
what it writes; there is no host computation and no fallback.
"""

from __future__ import annotations

import torch

from . import _lib
from .ops import _ptr, _stream

MAX_BATCH = 4
HEAD_DIM = 64
# lm_head workgroups (the width of the argmax keys): four per CU on the 256-CU
# part for the row kernel, two for the matrix-core kernel (measured on MI355X
# at vocab 151936, B=4: 44.3 us at 512 workgroups, 45.9 at 1024, 48.0 at 256).
LM_BLOCKS = 1024
LM_TILE_BLOCKS = 512


def lm_blocks(w_lm) -> int:
    """Workgroups (argmax key columns) for an lm_head call with ``w_lm``."""
    return LM_TILE_BLOCKS if isinstance(w_lm, Tiles) else LM_BLOCKS

# Weight layouts and packing row maps (include/qf_step.h).
W_ROWS, W_TILES = 0, 1
PACK_PLAIN, PACK_SWIGLU, PACK_ROPE = 0, 1, 2


class Tiles:
    """A projection weight packed into matrix-core tiles by ``pack_weight``.

    ``data`` holds the same N*K fp16 values as the (N, K) weight in tile order;
    ``layout`` is the row map it was packed with.  The step entry points take
    it in place of the row-major weight and run their MFMA kernels."""

    def __init__(self, data: torch.Tensor, n: int, k: int, layout: int):
        self.data, self.n, self.k, self.layout = data, n, k, layout

    @property
    def shape(self):
        return (self.n, self.k)


def pack_weight(w: torch.Tensor, layout: int = PACK_PLAIN) -> Tiles:
    """Repack a (N, K) fp16 weight (torch Linear layout) into MFMA tiles on its
    device (one launch; a load-time step with no counterpart in the reference)."""
    _check("w", w)
    if w.dim() != 2 or w.stride(1) != 1:
        raise ValueError("w must be 2-D with unit inner stride")
    n, k = w.shape
    out = torch.empty(n * k, device=w.device, dtype=torch.float16)
    rc = _lib.load().qf_pack_weight(w.data_ptr(), w.stride(0), out.data_ptr(), n, k, layout,
                                    _stream(w.device))
    _lib.check(rc, "qf_pack_weight")
    return Tiles(out, n, k, layout)


def _check(name: str, t: torch.Tensor, dtype=torch.float16) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be a HIP device tensor (got {t.device}); there is no CPU path")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype} (got {t.dtype})")


def _rows(name: str, t: torch.Tensor, batch: int, width: int) -> int:
    """Row stride of a (batch, width) view with unit inner stride."""
    _check(name, t)
    if t.dim() != 2 or tuple(t.shape) != (batch, width) or t.stride(1) != 1:
        raise ValueError(f"{name} must be ({batch}, {width}) with unit inner stride "
                         f"(got {tuple(t.shape)}, stride {t.stride()})")
    return t.stride(0)


def _weight(name: str, w, out_f: int, in_f: int, pack: int | None = None):
    """(pointer, w_layout) of a row-major weight or of its ``Tiles``; ``pack``
    is the row map an entry point's MFMA kernel expects (None: rows only)."""
    if isinstance(w, Tiles):
        if pack is None:
            raise TypeError(f"{name}: this entry point takes row-major weights only")
        if w.layout != pack or (w.n, w.k) != (out_f, in_f):
            raise ValueError(f"{name}: tiles must be ({out_f}, {in_f}) packed with row map {pack} "
                             f"(got ({w.n}, {w.k}) map {w.layout})")
        _check(name, w.data)
        return w.data.data_ptr(), W_TILES
    _check(name, w)
    if tuple(w.shape) != (out_f, in_f) or not w.is_contiguous():
        raise ValueError(f"{name} must be contiguous ({out_f}, {in_f}) (got {tuple(w.shape)})")
    return w.data_ptr(), W_ROWS


def _batch(b: int) -> None:
    if not 1 <= b <= MAX_BATCH:
        raise ValueError(f"fused decode-step kernels take 1..{MAX_BATCH} rows (got {b})")


def rope_args(cos, sin, positions, batch: int):
    """ABI pieces (cos, sin, cs_sb, pos, inv_freq) of the two RoPE sources:
    (B, 64) fp16 tables, or ``positions = (pos (B,) int64, inv_freq (32,)
    fp32)`` from which the kernel forms the same tables itself."""
    if positions is not None:
        if cos is not None or sin is not None:
            raise ValueError("pass cos/sin tables or positions, not both")
        pos, inv = positions
        _check("pos", pos, torch.int64)
        _check("inv_freq", inv, torch.float32)
        if pos.shape != (batch,) or not pos.is_contiguous():
            raise ValueError("pos must be contiguous (B,)")
        if inv.shape != (HEAD_DIM // 2,) or not inv.is_contiguous():
            raise ValueError(f"inv_freq must be contiguous ({HEAD_DIM // 2},)")
        return None, None, 0, pos.data_ptr(), inv.data_ptr()
    if cos is None or sin is None:
        raise ValueError("need cos and sin tables or positions")
    cs_sb = _rows("cos", cos, batch, HEAD_DIM)
    if _rows("sin", sin, batch, HEAD_DIM) != cs_sb:
        raise ValueError("cos and sin must share a row stride")
    return cos.data_ptr(), sin.data_ptr(), cs_sb, None, None


def rms_qkv_rope_append(x: torch.Tensor, norm_w: torch.Tensor, eps: float, w_qkv,
                        bias: torch.Tensor | None, cos: torch.Tensor | None,
                        sin: torch.Tensor | None, key_cache: torch.Tensor,
                        value_cache: torch.Tensor, write_index: torch.Tensor,
                        q_out: torch.Tensor, token: torch.Tensor | None = None,
                        hidden_out: torch.Tensor | None = None, positions=None) -> None:
    """q_out <- RoPE(q); caches[:, :, write_index] <- RoPE(k), v.

    ``x`` is the (B, hidden) residual stream, or -- with ``token`` (B,) int64
    -- the (vocab, hidden) embedding table whose rows ``token`` are gathered
    (and copied to ``hidden_out`` when given).  RoPE from ``cos``/``sin``
    (B, 64) fp16 tables, or from ``positions = (pos, inv_freq)`` (the kernel
    forms the identical tables; cos/sin then None).  ``q_out``: (B, QH, 64).
    ``w_qkv``: the ((QH + 2 KVH) * 64, hidden) weight, or its ``Tiles`` packed
    with PACK_ROPE (matrix-core kernel).
    """
    b, kvh, cap, d = key_cache.shape
    _batch(b)
    _check("key_cache", key_cache)
    _check("value_cache", value_cache)
    if d != HEAD_DIM or value_cache.shape != key_cache.shape:
        raise ValueError("caches must be (B, KVH, cap, 64) and alike")
    if key_cache.stride(-1) != 1 or value_cache.stride(-1) != 1:
        raise ValueError("caches need unit stride on the head dimension")
    _check("q_out", q_out)
    if q_out.dim() != 3 or q_out.shape[0] != b or q_out.shape[2] != d or q_out.stride(2) != 1:
        raise ValueError(f"q_out must be (B, QH, 64) (got {tuple(q_out.shape)})")
    qh = q_out.shape[1]
    hidden = norm_w.shape[0]
    _check("norm_w", norm_w)
    w_ptr, w_layout = _weight("w_qkv", w_qkv, (qh + 2 * kvh) * d, hidden, PACK_ROPE)
    if bias is not None:
        _check("bias", bias)
        if tuple(bias.shape) != ((qh + 2 * kvh) * d,) or not bias.is_contiguous():
            raise ValueError("bias must be contiguous ((QH + 2 KVH) * 64,)")
    rope = rope_args(cos, sin, positions, b)
    _check("write_index", write_index, torch.int64)
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
    lib = _lib.load()
    rc = lib.qf_rms_qkv_rope_append(
        x.data_ptr(), x_sb, _ptr(token), _ptr(hidden_out), ho_sb,
        norm_w.data_ptr(), float(eps), w_ptr, w_layout, _ptr(bias), *rope,
        key_cache.data_ptr(), *key_cache.stride()[:3],
        value_cache.data_ptr(), *value_cache.stride()[:3],
        write_index.data_ptr(), q_out.data_ptr(), q_out.stride(0), q_out.stride(1),
        b, hidden, qh, kvh, d, cap, _stream(x.device))
    _lib.check(rc, "qf_rms_qkv_rope_append")


def gemv_residual(inp: torch.Tensor, w: torch.Tensor, hidden: torch.Tensor) -> None:
    """hidden <- fp16(hidden + fp16(inp @ w^T)), in place."""
    b, k = inp.shape
    _batch(b)
    n = w.shape[0]
    in_sb = _rows("inp", inp, b, k)
    _weight("w", w, n, k)
    h_sb = _rows("hidden", hidden, b, n)
    rc = _lib.load().qf_gemv_residual(inp.data_ptr(), in_sb, w.data_ptr(), hidden.data_ptr(),
                                      h_sb, b, k, n, _stream(inp.device))
    _lib.check(rc, "qf_gemv_residual")


def attn_merge_o_proj(flash, w_o, hidden: torch.Tensor) -> None:
    """hidden <- fp16(hidden + fp16(merge(flash partials) @ w_o^T)), in place.

    ``flash`` is the decode scratch filled by ``ops.flash_decode_split``:
    acc (B, KVH, S, G, 64), m and l (B, KVH, S, G), fp32 contiguous.  The
    merge replaces the combine launch (SE:117-162); see include/qf_step.h.
    ``w_o``: the (hidden, KVH*G*64) weight, or its ``Tiles`` packed with
    PACK_PLAIN (matrix-core kernel).
    """
    acc, m, l = flash[:3]
    b, kvh, splits, g, d = acc.shape
    _batch(b)
    for name, t in (("acc", acc), ("m", m), ("l", l)):
        _check(name, t, torch.float32)
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    if d != HEAD_DIM or m.shape != (b, kvh, splits, g) or l.shape != m.shape:
        raise ValueError("flash partials must be (B, KVH, S, G, 64) / (B, KVH, S, G)")
    n = w_o.shape[0]
    w_ptr, w_layout = _weight("w_o", w_o, n, kvh * g * d, PACK_PLAIN)
    h_sb = _rows("hidden", hidden, b, n)
    rc = _lib.load().qf_attn_merge_o_proj(acc.data_ptr(), m.data_ptr(), l.data_ptr(), splits,
                                          kvh, g, w_ptr, w_layout, hidden.data_ptr(), h_sb, b, n,
                                          _stream(hidden.device))
    _lib.check(rc, "qf_attn_merge_o_proj")


def rms_gate_up_swiglu(x: torch.Tensor, norm_w: torch.Tensor, eps: float, w_gate_up,
                       h_out: torch.Tensor) -> None:
    """h_out <- fp16(fp16(silu(g)) * u), [g | u] = rms_norm(x) @ w_gate_up^T.

    ``w_gate_up``: the (2I, hidden) weight, or its ``Tiles`` packed with
    PACK_SWIGLU (matrix-core kernel)."""
    b, hidden = x.shape
    _batch(b)
    inter = w_gate_up.shape[0] // 2
    x_sb = _rows("x", x, b, hidden)
    _check("norm_w", norm_w)
    w_ptr, w_layout = _weight("w_gate_up", w_gate_up, 2 * inter, hidden, PACK_SWIGLU)
    ho_sb = _rows("h_out", h_out, b, inter)
    rc = _lib.load().qf_rms_gate_up_swiglu(x.data_ptr(), x_sb, norm_w.data_ptr(), float(eps),
                                           w_ptr, w_layout, h_out.data_ptr(), ho_sb,
                                           b, hidden, inter, _stream(x.device))
    _lib.check(rc, "qf_rms_gate_up_swiglu")


def rms_lm_head(x: torch.Tensor, norm_w: torch.Tensor, eps: float, w_lm,
                logits: torch.Tensor, keys: torch.Tensor) -> None:
    """logits <- fp16(rms_norm(x) @ w_lm^T); keys (B, n_blocks) uint64-as-int64
    <- per-block argmax keys.  ``w_lm``: the (V, hidden) weight, or its
    ``Tiles`` packed with PACK_PLAIN (matrix-core kernel)."""
    b, hidden = x.shape
    _batch(b)
    vocab = w_lm.shape[0]
    x_sb = _rows("x", x, b, hidden)
    _check("norm_w", norm_w)
    w_ptr, w_layout = _weight("w_lm", w_lm, vocab, hidden, PACK_PLAIN)
    lg_sb = _rows("logits", logits, b, vocab)
    _check("keys", keys, torch.int64)
    if keys.dim() != 2 or keys.shape[0] != b or not keys.is_contiguous():
        raise ValueError("keys must be contiguous (B, n_blocks) int64")
    rc = _lib.load().qf_rms_lm_head(x.data_ptr(), x_sb, norm_w.data_ptr(), float(eps),
                                    w_ptr, w_layout, logits.data_ptr(), lg_sb, keys.data_ptr(),
                                    keys.shape[1], b, hidden, vocab, _stream(x.device))
    _lib.check(rc, "qf_rms_lm_head")


def argmax_step(keys: torch.Tensor, token: torch.Tensor, rows: torch.Tensor | None = None,
                step: torch.Tensor | None = None, write_index: torch.Tensor | None = None,
                pos: torch.Tensor | None = None) -> None:
    """token <- argmax from the lm_head keys; rows[:, step] <- token; step,
    write_index and pos advance by one (each optional)."""
    _check("keys", keys, torch.int64)
    b, n_blocks = keys.shape
    _batch(b)
    _check("token", token, torch.int64)
    if token.shape != (b,) or not token.is_contiguous():
        raise ValueError("token must be contiguous (B,)")
    rows_sb, n_rows = 0, 0
    if rows is not None:
        _check("rows", rows, torch.int64)
        if rows.dim() != 2 or rows.shape[0] != b or rows.stride(1) != 1:
            raise ValueError("rows must be (B, T) with unit inner stride")
        if step is None:
            raise ValueError("rows needs step")
        rows_sb, n_rows = rows.stride(0), rows.shape[1]
    for name, t in (("step", step), ("write_index", write_index), ("pos", pos)):
        if t is not None:
            _check(name, t, torch.int64)
    rc = _lib.load().qf_argmax_step(keys.data_ptr(), n_blocks, b, token.data_ptr(), _ptr(rows),
                                    rows_sb, n_rows, _ptr(step), _ptr(write_index), _ptr(pos),
                                    _stream(keys.device))
    _lib.check(rc, "qf_argmax_step")
