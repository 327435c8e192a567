/*
 * qf_paged.h -- paged KV-cache variants of the attention-path entry points.
 *
 * The reference keeps one dense (B, KVH, cap, D) cache per layer and pads
 * ragged batches up to the longest row (student_engine.py:1162-1204,
 * :1263-1319); block-level KV management ("PagedAttention & Continuous
 * Batching") is on its roadmap (README.md:144) with no kernel behind it.
 * These entry points are that layout for this library's kernels: the same
 * mathematics and rounding as the dense entry points in qf_attn.h / qf_step.h,
 * with every cache replaced by a page pool and a block table:
 *
 *   k_pool, v_pool   (n_pages, KVH, page_size, D) fp16, strides in elements:
 *                    *_sp (page), *_sh (kv head), *_sn (slot within the page);
 *                    D contiguous.
 *   block_table      int32 (B, pages_per_row), row stride bt_sb >= pages_per_row:
 *                    logical page j of batch row b is physical page
 *                    block_table[b * bt_sb + j].
 *   logical slot s of row b  ->  pool[block_table[b][s / page_size], h, s % page_size]
 *
 * page_size is a power of two in [64, 4096], so a 32-key decode tile and a
 * 64-key prefill tile never straddle a page; a row's logical capacity is
 * pages_per_row * page_size.  Page ids outside [0, n_pages) are a caller
 * error: appends skip such a slot and reads clamp to the pool (in bounds,
 * values unspecified).  Rows hold no padding holes: each row's length is its
 * own (kv_last per row for decode, cu_seqlens for prefill, a per-row slot for
 * appends), which is what lets a batch admit and retire rows independently.
 *
 * Conventions are those of qf_attn.h (device pointers, element strides,
 * void* stream, QF_OK / QF_ERR_* / hipError_t returns, no allocation, no
 * synchronisation).
 */
#ifndef QF_PAGED_H
#define QF_PAGED_H

#include <stdint.h>

#include "qf_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Split-K decode attention over paged caches: qf_decode_attn
 * (student_engine.py:834-874 semantics) with k/v read through the block
 * table.  q, bias, kv_last, the scratch (acc, m, l, ticket) and out are as in
 * qf_decode_attn; cap = pages_per_row * page_size.  kv_last per row
 * (kv_last_sb = 1) is the usual way to bound each row's keys.
 */
int qf_decode_attn_paged(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sg,
                         const void* k_pool, int64_t kp_sp, int64_t kp_sh, int64_t kp_sn,
                         const void* v_pool, int64_t vp_sp, int64_t vp_sh, int64_t vp_sn,
                         const int32_t* block_table, int64_t bt_sb, int pages_per_row,
                         int n_pages, int page_size,
                         const void* bias, int64_t bias_sb,
                         const int64_t* kv_last, int64_t kv_last_sb,
                         float* acc, float* m, float* l, int splits,
                         int32_t* ticket,
                         void* out, int64_t o_sb, int64_t o_sh, int64_t o_sg,
                         int B, int KVH, int G, int D, float scale, void* stream);

/*
 * Split phase only, over paged caches (qf_decode_split semantics, the
 * _flash_decode_split_kernel launch SE:854-865): writes the partials
 * (acc, m, l) for a later merge (qf_decode_combine or qf_attn_merge_o_proj).
 */
int qf_decode_split_paged(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sg,
                          const void* k_pool, int64_t kp_sp, int64_t kp_sh, int64_t kp_sn,
                          const void* v_pool, int64_t vp_sp, int64_t vp_sh, int64_t vp_sn,
                          const int32_t* block_table, int64_t bt_sb, int pages_per_row,
                          int n_pages, int page_size,
                          const void* bias, int64_t bias_sb,
                          const int64_t* kv_last, int64_t kv_last_sb,
                          float* acc, float* m, float* l, int splits,
                          int B, int KVH, int G, int D, float scale, void* stream);

/*
 * One-token RoPE + append into paged caches: qf_rope_append (the eager RoPE
 * SE:927-928 and index_copy_ appends SE:931-932) with a slot per row, read on
 * the device: row b's new K/V go to logical slot slots[b * slot_sb] (a slot
 * outside [0, pages_per_row * page_size) writes nothing; q_out is always
 * written).
 */
int qf_rope_append_paged(const void* q, int64_t q_sb, int64_t q_sh,
                         const void* k, int64_t k_sb, int64_t k_sh,
                         const void* v, int64_t v_sb, int64_t v_sh,
                         const void* cos, const void* sin, int64_t cs_sb,
                         void* k_pool, int64_t kp_sp, int64_t kp_sh, int64_t kp_sn,
                         void* v_pool, int64_t vp_sp, int64_t vp_sh, int64_t vp_sn,
                         const int32_t* block_table, int64_t bt_sb, int pages_per_row,
                         int n_pages, int page_size,
                         const int64_t* slots, int64_t slot_sb,
                         void* q_out, int64_t qo_sb, int64_t qo_sh,
                         int B, int QH, int KVH, int D, void* stream);

/*
 * Ragged causal prefill into paged caches: qf_prefill_varlen (rows packed
 * along the token axis, _prefill_ragged SE:1162-1204 in one launch) with token
 * i of row b appended at logical slot start_pos + i of row b, then attended
 * from the pages.  start_pos must be a multiple of 64 and
 * start_pos + max_seqlen <= pages_per_row * page_size.  cos/sin (per-token
 * tables) are optional; without them K is stored as given.
 */
int qf_prefill_varlen_paged(const void* q, int64_t q_sh, int64_t q_sn,
                            const void* k, int64_t k_sh, int64_t k_sn,
                            const void* v, int64_t v_sh, int64_t v_sn,
                            const int32_t* cu_seqlens, int total, int max_seqlen,
                            const void* cos, const void* sin, int64_t cs_sn,
                            void* k_pool, int64_t kp_sp, int64_t kp_sh, int64_t kp_sn,
                            void* v_pool, int64_t vp_sp, int64_t vp_sh, int64_t vp_sn,
                            const int32_t* block_table, int64_t bt_sb, int pages_per_row,
                            int n_pages, int page_size, int64_t start_pos,
                            void* out, int64_t o_sh, int64_t o_sn,
                            int B, int QH, int KVH, int D, float scale, void* stream);

/*
 * The fused decode-step QKV projection (qf_rms_qkv_rope_append in qf_step.h:
 * rms_norm + QKV linear + RoPE + append, SE:917-932) appending into paged
 * caches at a per-row slot slots[b * slot_sb] read on the device.  RoPE
 * from cos/sin tables or from pos + inv_freq, as there.
 */
int qf_rms_qkv_rope_append_paged(const void* x, int64_t x_sb, const int64_t* token,
                                 void* hidden_out, int64_t ho_sb,
                                 const void* norm_w, float eps,
                                 const void* w_qkv, int w_layout, const void* bias,
                                 const void* cos, const void* sin, int64_t cs_sb,
                                 const int64_t* pos, const float* inv_freq,
                                 void* k_pool, int64_t kp_sp, int64_t kp_sh, int64_t kp_sn,
                                 void* v_pool, int64_t vp_sp, int64_t vp_sh, int64_t vp_sn,
                                 const int32_t* block_table, int64_t bt_sb, int pages_per_row,
                                 int n_pages, int page_size,
                                 const int64_t* slots, int64_t slot_sb,
                                 void* q_out, int64_t qo_sb, int64_t qo_sh,
                                 int B, int hidden, int QH, int KVH, int D, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QF_PAGED_H */
