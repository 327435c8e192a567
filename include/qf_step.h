/* C ABI of the fused weight-streaming decode-step kernels (gfx950 / MI355X).
 *
 * These replace the per-layer torch op sequence of the reference's graph step
 * _decode_step_static (student_engine.py:876-982) for batches of 1..4 rows.
 * The reference calls torch ops there (F.rms_norm, F.linear, eager RoPE,
 * index_copy_, F.silu, argmax), so each entry point names the op sequence it
 * replaces rather than a reference FFI symbol.  Same conventions as
 * qf_attn.h: fp16 (IEEE half) storage, plain pointers and element strides,
 * the stream as void*, a QF_* / hipError_t return code, no allocation and no
 * synchronisation inside a call (capture-safe).
 *
 * Layouts: activations are row-major (B, width) with a row stride in
 * elements; weights are torch Linear weights, (out_features, in_features)
 * row-major and contiguous.  All activation and weight rows must be 16-byte
 * aligned (pointers 16-byte aligned, strides multiples of 8 elements).
 */
#ifndef QF_STEP_H
#define QF_STEP_H

#include <stdint.h>

#include "qf_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Weight layouts accepted by the projection entry points (w_layout):
 *   QF_W_ROWS   torch Linear layout, (out, in) row-major -- the VALU kernels;
 *   QF_W_TILES  matrix-core tiles written by qf_pack_weight with the row map
 *               the entry point names -- the MFMA kernels (in % 32 == 0). */
#define QF_W_ROWS 0
#define QF_W_TILES 1

/* Row maps of qf_pack_weight. */
#define QF_PACK_PLAIN 0   /* o_proj, down_proj, lm_head */
#define QF_PACK_SWIGLU 1  /* gate_up_weight: gate rows [0, N/2), up rows [N/2, N) */
#define QF_PACK_ROPE 2    /* qkv_weight: 64-row heads, rotate-half pairs (d, d + 32) */

/* Repack a projection weight W (N, K) fp16, row stride w_sb, into matrix-core
 * tiles: tile (rb, kb) of 16 rows x 32 k is 1 KB at (rb * K/32 + kb) * 1 KB,
 * lane l's 16 bytes being W[row(rb, l % 16)][32 kb + 8 (l / 16) .. +7].  The
 * row map (layout) is QF_PACK_PLAIN (row 16 rb + r), QF_PACK_SWIGLU or
 * QF_PACK_ROPE (see decode_step.hip).  No counterpart in the reference: it is
 * the one-time load step that lets every decode-step weight load be a
 * contiguous 1 KB read.  N % 16 == 0 (% 64 for ROPE), K % 32 == 0. */
int qf_pack_weight(const void* w, int64_t w_sb, void* packed, int N, int K, int layout,
                   void* stream);

/* RMSNorm + fused QKV projection (+ bias) + rotate-half RoPE + KV append.
 * Replaces student_engine.py:917-932 (rms_norm, F.linear(normalized,
 * qkv_weight, qkv_bias), split, the eager RoPE of q and k with the per-step
 * cos/sin of :910-915, and the two index_copy_ appends at write_index).
 *
 * x: (B, hidden) rows, row stride x_sb.  When `token` (B int64, device) is
 * non-null, row b is taken from x + token[b] * x_sb instead (x is then the
 * embedding table, :896) and, if `hidden_out` is non-null, the gathered rows
 * are also written to hidden_out (row stride ho_sb) as the residual stream.
 * w_qkv: ((QH + 2*KVH) * 64, hidden) as rows (w_layout QF_W_ROWS) or packed
 * with QF_PACK_ROPE (QF_W_TILES, hidden % 32 == 0); bias: (QH + 2*KVH) * 64
 * or null.
 * RoPE angles come from either cos/sin: (B, 64) fp16 tables, row stride
 * cs_sb (pos and inv_freq NULL), or pos: (B,) int64 positions plus inv_freq:
 * (32,) fp32 (cos and sin NULL), in which case the table entries
 * fp16(cos(float(pos[b]) * inv_freq[i])) (and sin) are formed in the kernel,
 * bit-identical to the torch-built table of :910-915.  Rotated q goes to q_out
 * (B, QH, 64) with strides (qo_sb, qo_sh); rotated k and raw v go to slot
 * write_index[0] of the (B, KVH, cap, 64) caches (skipped when the slot is
 * outside [0, cap)).  Rounding: fp16(acc + bias) per projection output, then
 * the eager RoPE sequence fp16(fp16(x*cos) + fp16(rot(x)*sin)).
 * Supports hidden <= 1024, head_dim 64, B in 1..4. */
int qf_rms_qkv_rope_append(const void* x, int64_t x_sb, const int64_t* token,
                           void* hidden_out, int64_t ho_sb,
                           const void* norm_w, float eps,
                           const void* w_qkv, int w_layout, const void* bias,
                           const void* cos, const void* sin, int64_t cs_sb,
                           const int64_t* pos, const float* inv_freq,
                           void* k_cache, int64_t kc_sb, int64_t kc_sh, int64_t kc_sn,
                           void* v_cache, int64_t vc_sb, int64_t vc_sh, int64_t vc_sn,
                           const int64_t* write_index,
                           void* q_out, int64_t qo_sb, int64_t qo_sh,
                           int B, int hidden, int QH, int KVH, int D, int cap, void* stream);

/* hidden += fp16(inp @ w^T): a bias-free projection added to the residual
 * stream in place.  Replaces `hidden = residual + F.linear(attended, o_weight)`
 * (student_engine.py:973-974) and `hidden = residual + F.linear(gate * up,
 * down_weight)` (:978 with _mlp :666).  inp: (B, K) row stride in_sb; w:
 * (N, K); hidden: (B, N) row stride h_sb.  Rounding: fp16(residual +
 * fp16(acc)).  Supports K <= 8192, B in 1..4. */
int qf_gemv_residual(const void* inp, int64_t in_sb, const void* w,
                     void* hidden, int64_t h_sb, int B, int K, int N, void* stream);

/* Split-K attention merge + o_proj + residual.  Replaces the second decode
 * launch _flash_decode_combine_kernel (student_engine.py:117-162, launched at
 * :860-872) together with `hidden = residual + F.linear(attended, o_weight)`
 * (:973-974): every workgroup merges the partials (acc, m, l) of
 * qf_decode_split for all B x KVH x G query heads, rounds the merged rows to
 * fp16 as the combine does (fp16(A * (1/L))) and applies the projection.
 * acc: (B, KVH, splits, G, 64) fp32, m/l: (B, KVH, splits, G) fp32 (m in
 * natural-log units), all contiguous; w_o: (N, KVH*G*64) as rows (w_layout
 * QF_W_ROWS) or packed with QF_PACK_PLAIN (QF_W_TILES: N % 16 == 0, hidden
 * 8-byte aligned with h_sb % 4 == 0); hidden: (B, N) row stride h_sb,
 * updated in place.  Supports KVH*G*64 <= 1024, B in 1..4. */
int qf_attn_merge_o_proj(const float* acc, const float* m, const float* l, int splits,
                         int KVH, int G, const void* w_o, int w_layout, void* hidden,
                         int64_t h_sb, int B, int N, void* stream);

/* RMSNorm + gate/up projection + SwiGLU.  Replaces `normalized =
 * rms_norm(hidden, post_norm)` (:976-977) and the first two lines of _mlp
 * (:664-665) plus the product `gate * up` (:666): h = fp16(fp16(silu(g)) * u)
 * with g = fp16(acc_gate), u = fp16(acc_up).  w_gate_up: (2*I, hidden) with
 * the gate rows first (the reference's fused layout, :520-527) as rows
 * (QF_W_ROWS) or packed with QF_PACK_SWIGLU (QF_W_TILES, I % 8 == 0,
 * hidden % 32 == 0); h_out: (B, I) row stride ho_sb.  Supports hidden <= 1024,
 * B in 1..4. */
int qf_rms_gate_up_swiglu(const void* x, int64_t x_sb, const void* norm_w, float eps,
                          const void* w_gate_up, int w_layout, void* h_out, int64_t ho_sb,
                          int B, int hidden, int I, void* stream);

/* Final RMSNorm + lm_head projection + per-block argmax.  Replaces
 * `rms_norm(hidden, final_norm)` and `F.linear(hidden, lm_head)` (:980-981)
 * and the first half of `torch.argmax(logits, dim=-1)` (:982).  Writes fp16
 * logits (B, V) with row stride lg_sb and, per batch row b and block j <
 * n_blocks, keys[b * n_blocks + j] = the block's best (logit, index) packed
 * so that the largest key is the largest logit with the smallest index
 * (torch.argmax's first-maximum rule).  keys: B * n_blocks uint64 (device).
 * w_lm: (V, hidden) as rows (w_layout QF_W_ROWS) or packed with
 * QF_PACK_PLAIN (QF_W_TILES: V % 16 == 0, hidden % 32 == 0, logits 8-byte
 * aligned with lg_sb % 4 == 0).  Supports hidden <= 1024, B in 1..4,
 * 1 <= n_blocks <= 65535. */
int qf_rms_lm_head(const void* x, int64_t x_sb, const void* norm_w, float eps,
                   const void* w_lm, int w_layout, void* logits, int64_t lg_sb, uint64_t* keys,
                   int n_blocks, int B, int hidden, int V, void* stream);

/* Reduces the per-block keys of qf_rms_lm_head to the argmax token and does
 * the step's slot bookkeeping on the device: token[b] = argmax;
 * rows[b * rows_sb + step[0]] = token[b] (when step[0] < n_rows); then
 * write_index[0] += 1, pos[b] += 1 and step[0] += 1.  Replaces the argmax of
 * :982 and the host-side updates between replays (student_engine.py:1126-1132:
 * token store, write_index.fill_, static_pos += 1).  Any of rows/write_index/
 * pos/step may be null to skip that update (rows needs step). */
int qf_argmax_step(const uint64_t* keys, int n_blocks, int B, int64_t* token,
                   int64_t* rows, int64_t rows_sb, int n_rows, int64_t* step,
                   int64_t* write_index, int64_t* pos, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QF_STEP_H */
