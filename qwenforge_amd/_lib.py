"""ctypes binding of the C ABI in ``include/qf_attn.h``, ``include/qf_step.h``,
``include/qf_paged.h`` and ``include/qf_probe.h``.

The shared object is built in-tree by ``qwenforge_amd.build``.  There is no
fallback: if it is missing or does not load, every op raises.
"""

from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("_qf_attn.so")

_i64, _i32, _f32, _vp = C.c_int64, C.c_int, C.c_float, C.c_void_p

# name -> argument types, in header order.  Every entry point returns int.
SIGNATURES = {
    "qf_decode_attn": [
        _vp, _i64, _i64, _i64,          # q, q_sb, q_sh, q_sg
        _vp, _i64, _i64, _i64,          # k, k_sb, k_sh, k_sn
        _vp, _i64, _i64, _i64,          # v, v_sb, v_sh, v_sn
        _vp, _i64,                      # bias, bias_sb
        _vp, _i64,                      # kv_last, kv_last_sb
        _vp, _vp, _vp, _i32,            # acc, m, l, splits
        _vp,                            # ticket
        _vp, _i64, _i64, _i64,          # out, o_sb, o_sh, o_sg
        _i32, _i32, _i32, _i32, _i32,   # B, KVH, G, D, cap
        _f32, _vp,                      # scale, stream
    ],
    "qf_decode_waves": [_i32, _i32, _i32, _i32, _i32, _i32],   # B, KVH, G, cap, splits, fused
    "qf_decode_attn_noalloc": [
        _vp, _i64, _i64, _i64,          # q, q_sb, q_sh, q_sg
        _vp, _i64, _i64, _i64,          # k, k_sb, k_sh, k_sn
        _vp, _i64, _i64, _i64,          # v, v_sb, v_sh, v_sn
        _vp, _i64,                      # bias, bias_sb
        _vp, _i64,                      # kv_last, kv_last_sb
        _i32,                           # splits
        _vp, _i64, _i64, _i64,          # out, o_sb, o_sh, o_sg
        _i32, _i32, _i32, _i32, _i32,   # B, KVH, G, D, cap
        _f32, _vp,                      # scale, stream
    ],
    "qf_decode_split": [
        _vp, _i64, _i64, _i64,          # q
        _vp, _i64, _i64, _i64,          # k
        _vp, _i64, _i64, _i64,          # v
        _vp, _i64,                      # bias, bias_sb
        _vp, _i64,                      # kv_last, kv_last_sb
        _vp, _vp, _vp, _i32,            # acc, m, l, splits
        _i32, _i32, _i32, _i32, _i32,   # B, KVH, G, D, cap
        _f32, _vp,                      # scale, stream
    ],
    "qf_decode_split_capacity": [
        _vp, _i64, _i64, _i64,          # q
        _vp, _i64, _i64, _i64,          # k
        _vp, _i64, _i64, _i64,          # v
        _vp, _i64,                      # bias, bias_sb
        _vp, _i64,                      # kv_last, kv_last_sb
        _vp, _vp, _vp, _i32,            # acc, m, l, splits
        _i32, _i32, _i32, _i32, _i32,   # B, KVH, G, D, cap
        _f32, _vp,                      # scale, stream
    ],
    "qf_decode_combine": [
        _vp, _vp, _vp, _i32,            # acc, m, l, splits
        _vp, _i64, _i64, _i64,          # out, o_sb, o_sh, o_sg
        _i32, _i32, _i32, _i32,         # B, KVH, G, D
        _vp,                            # stream
    ],
    "qf_prefill_attn": [
        _vp, _i64, _i64, _i64,          # q
        _vp, _i64, _i64, _i64,          # k
        _vp, _i64, _i64, _i64,          # v
        _vp, _vp, _i64, _i64,           # cos, sin, cs_sb, cs_sn
        _vp, _i64, _i64, _i64,          # k_cache
        _vp, _i64, _i64, _i64,          # v_cache
        _i64, _i32,                     # start_pos, cap
        _vp, _i64, _i64, _i64,          # out
        _i32, _i32, _i32, _i32, _i32,   # B, QH, KVH, S, D
        _f32, _vp,                      # scale, stream
    ],
    "qf_prefill_varlen": [
        _vp, _i64, _i64,                # q, q_sh, q_sn
        _vp, _i64, _i64,                # k
        _vp, _i64, _i64,                # v
        _vp, _i32, _i32,                # cu_seqlens, total, max_seqlen
        _vp, _vp, _i64,                 # cos, sin, cs_sn
        _vp, _i64, _i64, _i64,          # k_cache
        _vp, _i64, _i64, _i64,          # v_cache
        _i64, _i32,                     # start_pos, cap
        _vp, _i64, _i64,                # out, o_sh, o_sn
        _i32, _i32, _i32, _i32,         # B, QH, KVH, D
        _f32, _vp,                      # scale, stream
    ],
    "qf_rope_append": [
        _vp, _i64, _i64,                # q, q_sb, q_sh
        _vp, _i64, _i64,                # k
        _vp, _i64, _i64,                # v
        _vp, _vp, _i64,                 # cos, sin, cs_sb
        _vp, _i64, _i64, _i64,          # k_cache
        _vp, _i64, _i64, _i64,          # v_cache
        _vp,                            # write_index
        _vp, _i64, _i64,                # q_out
        _i32, _i32, _i32, _i32, _i32,   # B, QH, KVH, D, cap
        _vp,                            # stream
    ],
    # include/qf_step.h
    "qf_rms_qkv_rope_append": [
        _vp, _i64, _vp,                 # x, x_sb, token
        _vp, _i64,                      # hidden_out, ho_sb
        _vp, _f32,                      # norm_w, eps
        _vp, _i32, _vp,                 # w_qkv, w_layout, bias
        _vp, _vp, _i64,                 # cos, sin, cs_sb
        _vp, _vp,                       # pos, inv_freq
        _vp, _i64, _i64, _i64,          # k_cache
        _vp, _i64, _i64, _i64,          # v_cache
        _vp,                            # write_index
        _vp, _i64, _i64,                # q_out, qo_sb, qo_sh
        _i32, _i32, _i32, _i32, _i32, _i32,  # B, hidden, QH, KVH, D, cap
        _vp,                            # stream
    ],
    "qf_gemv_residual": [
        _vp, _i64, _vp,                 # inp, in_sb, w
        _vp, _i64,                      # hidden, h_sb
        _i32, _i32, _i32,               # B, K, N
        _vp,                            # stream
    ],
    "qf_attn_merge_o_proj": [
        _vp, _vp, _vp, _i32,            # acc, m, l, splits
        _i32, _i32,                     # KVH, G
        _vp, _i32, _vp, _i64,           # w_o, w_layout, hidden, h_sb
        _i32, _i32,                     # B, N
        _vp,                            # stream
    ],
    "qf_rms_gate_up_swiglu": [
        _vp, _i64, _vp, _f32,           # x, x_sb, norm_w, eps
        _vp, _i32, _vp, _i64,           # w_gate_up, w_layout, h_out, ho_sb
        _i32, _i32, _i32,               # B, hidden, I
        _vp,                            # stream
    ],
    "qf_rms_lm_head": [
        _vp, _i64, _vp, _f32,           # x, x_sb, norm_w, eps
        _vp, _i32, _vp, _i64, _vp,      # w_lm, w_layout, logits, lg_sb, keys
        _i32, _i32, _i32, _i32,         # n_blocks, B, hidden, V
        _vp,                            # stream
    ],
    "qf_argmax_step": [
        _vp, _i32, _i32, _vp,           # keys, n_blocks, B, token
        _vp, _i64, _i32,                # rows, rows_sb, n_rows
        _vp, _vp, _vp,                  # step, write_index, pos
        _vp,                            # stream
    ],
    # include/qf_paged.h
    "qf_decode_attn_paged": [
        _vp, _i64, _i64, _i64,          # q, q_sb, q_sh, q_sg
        _vp, _i64, _i64, _i64,          # k_pool, kp_sp, kp_sh, kp_sn
        _vp, _i64, _i64, _i64,          # v_pool, vp_sp, vp_sh, vp_sn
        _vp, _i64, _i32, _i32, _i32,    # block_table, bt_sb, pages_per_row, n_pages, page_size
        _vp, _i64,                      # bias, bias_sb
        _vp, _i64,                      # kv_last, kv_last_sb
        _vp, _vp, _vp, _i32,            # acc, m, l, splits
        _vp,                            # ticket
        _vp, _i64, _i64, _i64,          # out, o_sb, o_sh, o_sg
        _i32, _i32, _i32, _i32,         # B, KVH, G, D
        _f32, _vp,                      # scale, stream
    ],
    "qf_decode_split_paged": [
        _vp, _i64, _i64, _i64,          # q
        _vp, _i64, _i64, _i64,          # k_pool
        _vp, _i64, _i64, _i64,          # v_pool
        _vp, _i64, _i32, _i32, _i32,    # block_table, bt_sb, pages_per_row, n_pages, page_size
        _vp, _i64,                      # bias, bias_sb
        _vp, _i64,                      # kv_last, kv_last_sb
        _vp, _vp, _vp, _i32,            # acc, m, l, splits
        _i32, _i32, _i32, _i32,         # B, KVH, G, D
        _f32, _vp,                      # scale, stream
    ],
    "qf_rope_append_paged": [
        _vp, _i64, _i64,                # q, q_sb, q_sh
        _vp, _i64, _i64,                # k
        _vp, _i64, _i64,                # v
        _vp, _vp, _i64,                 # cos, sin, cs_sb
        _vp, _i64, _i64, _i64,          # k_pool
        _vp, _i64, _i64, _i64,          # v_pool
        _vp, _i64, _i32, _i32, _i32,    # block_table, bt_sb, pages_per_row, n_pages, page_size
        _vp, _i64,                      # slots, slot_sb
        _vp, _i64, _i64,                # q_out
        _i32, _i32, _i32, _i32,         # B, QH, KVH, D
        _vp,                            # stream
    ],
    "qf_prefill_varlen_paged": [
        _vp, _i64, _i64,                # q, q_sh, q_sn
        _vp, _i64, _i64,                # k
        _vp, _i64, _i64,                # v
        _vp, _i32, _i32,                # cu_seqlens, total, max_seqlen
        _vp, _vp, _i64,                 # cos, sin, cs_sn
        _vp, _i64, _i64, _i64,          # k_pool
        _vp, _i64, _i64, _i64,          # v_pool
        _vp, _i64, _i32, _i32, _i32,    # block_table, bt_sb, pages_per_row, n_pages, page_size
        _i64,                           # start_pos
        _vp, _i64, _i64,                # out, o_sh, o_sn
        _i32, _i32, _i32, _i32,         # B, QH, KVH, D
        _f32, _vp,                      # scale, stream
    ],
    "qf_rms_qkv_rope_append_paged": [
        _vp, _i64, _vp,                 # x, x_sb, token
        _vp, _i64,                      # hidden_out, ho_sb
        _vp, _f32,                      # norm_w, eps
        _vp, _i32, _vp,                 # w_qkv, w_layout, bias
        _vp, _vp, _i64,                 # cos, sin, cs_sb
        _vp, _vp,                       # pos, inv_freq
        _vp, _i64, _i64, _i64,          # k_pool
        _vp, _i64, _i64, _i64,          # v_pool
        _vp, _i64, _i32, _i32, _i32,    # block_table, bt_sb, pages_per_row, n_pages, page_size
        _vp, _i64,                      # slots, slot_sb
        _vp, _i64, _i64,                # q_out, qo_sb, qo_sh
        _i32, _i32, _i32, _i32, _i32,   # B, hidden, QH, KVH, D
        _vp,                            # stream
    ],
    "qf_pack_weight": [
        _vp, _i64, _vp,                 # w, w_sb, packed
        _i32, _i32, _i32,               # N, K, layout
        _vp,                            # stream
    ],
    # include/qf_probe.h
    "qf_stream_read": [_vp, _i64, _vp, _i32, _vp],   # src, bytes, sink, workgroups, stream
    "qf_launch_probe": [_vp, _i64, _vp, _vp,          # src, bytes, index, sink
                        _i32, _i32, _i32, _vp],      # workgroups, threads, round_trips, stream
    "qf_decode_split_valu": [
        _vp, _i64, _i64, _i64,          # q
        _vp, _i64, _i64, _i64,          # k
        _vp, _i64, _i64, _i64,          # v
        _vp, _i64,                      # kv_last, kv_last_sb
        _vp, _vp, _vp, _i32,            # acc, m, l, splits
        _i32, _i32, _i32, _i32, _i32,   # B, KVH, G, D, cap
        _f32, _vp,                      # scale, stream
    ],
    "qf_error_string": [_i32],
    "qf_abi_version": [],
}

# Entry points that do not return an int status.
RESTYPES = {"qf_error_string": C.c_char_p}

_lock = threading.Lock()
_lib: C.CDLL | None = None


def load() -> C.CDLL:
    """Load ``_qf_attn.so`` once; raise ``RuntimeError`` if it is unavailable."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m qwenforge_amd.build` "
                "(the HIP kernels have no fallback)"
            )
        lib = C.CDLL(str(LIB_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = RESTYPES.get(name, C.c_int)
        _lib = lib
        return lib


def check(code: int, name: str) -> None:
    """Raise ``RuntimeError`` for a non-zero return code of entry point ``name``."""
    if code != 0:
        msg = load().qf_error_string(code).decode()
        raise RuntimeError(f"{name} failed with code {code}: {msg}")
