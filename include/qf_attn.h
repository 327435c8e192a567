/*
 * qf_attn.h -- C ABI of the MI355X (gfx950) attention hot path of QwenForge.
 *
 * Three hand-written HIP kernels replace the reference engine's Triton
 * kernels and torch ops on the attention path of student_engine.py:
 *
 *   qf_decode_attn    split-K flash-decoding GQA attention over the KV cache
 *                     (replaces _flash_decode_split_kernel SE:32-115,
 *                      _flash_decode_combine_kernel SE:117-162 and their
 *                      launcher _flash_decode_attention SE:834-874; also the
 *                      math twin SE:968-972)
 *   qf_prefill_attn   causal GQA flash-prefill, optionally with rotate-half
 *                     RoPE applied in registers and the KV-cache append fused
 *                     (replaces _gqa_flash_prefill_kernel SE:164-251 behind
 *                      student_qwen::gqa_flash_prefill SE:254-292, the eager
 *                      RoPE SE:767 / SE:542-554 and the slice append
 *                      SE:715-716)
 *   qf_rope_append    one-token RoPE on q/k plus the KV-cache append at a
 *                     device-resident slot (replaces SE:927-932)
 *
 * Conventions (all entry points):
 *   - Pointers are device pointers owned by the caller; the library keeps none.
 *   - Tensors are fp16 unless stated; strides are in ELEMENTS; the innermost
 *     (head-dim) stride is 1 and is not passed.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).  All
 *     work is enqueued on it; nothing is allocated and nothing synchronises,
 *     so every call is legal inside hipGraph stream capture.
 *   - Return value: 0 on success; a negative QF_ERR_* code for a rejected
 *     argument (nothing launched); a positive hipError_t from the launch.
 *     Nothing throws across the ABI.
 *   - Supported shapes: head_dim D == 64, 1 <= G <= 16 query heads per kv
 *     head.  Anything else returns QF_ERR_UNSUPPORTED.
 *   - Reentrant.  The only global state is the per-GPU address of
 *     qf_decode_attn_noalloc's static scratch, looked up once under a mutex.
 */
#ifndef QF_ATTN_H
#define QF_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QF_OK 0
#define QF_ERR_INVALID_ARG (-1)
#define QF_ERR_UNSUPPORTED (-2)
#define QF_ERR_SCRATCH_LIMIT (-3)

/* Bytes of split partials (acc, m, l) the no-allocation decode entry point
 * holds per GPU: B*KVH*splits*G*(D+2)*4 must not exceed this. */
#define QF_NOALLOC_PARTIAL_BYTES (4 << 20)

/* Human-readable text for a return code of any qf_* entry point. */
const char* qf_error_string(int code);

/* ABI version (major * 100 + minor): 301.  301 adds qf_decode_split_capacity
 * (nothing else changes).  300, from 200: qf_attn_merge_o_proj and
 * qf_rms_lm_head (qf_step.h) take w_layout after the weight pointer, and the
 * qf_decode_attn ticket holds one int32 counter per (b, kv head) instead of
 * one in total. */
int qf_abi_version(void);

/*
 * Split-K flash-decoding attention for one new token per sequence.
 *
 * Replaces StudentEngine._flash_decode_attention (student_engine.py:834-874),
 * i.e. the launches of _flash_decode_split_kernel (:854-865) and
 * _flash_decode_combine_kernel (:866-873), keeping their data contract:
 *
 *   q      (B, KVH, G, D)   `grouped` query, strides q_sb, q_sh, q_sg
 *   k, v   (B, KVH, cap, D) caches; K and V take separate strides
 *   bias   (B, cap) additive fp16 bias (0 valid / fp16-min empty), stride
 *          bias_sb; NULL = no bias
 *   kv_last  NULL, or device int64 holding the last slot (inclusive) that can
 *          be valid in each row; row b reads kv_last[b * kv_last_sb]
 *          (kv_last_sb = 0 shares one value, e.g. the engine's write_index).
 *          Slots beyond it are skipped instead of read; NULL reads all of cap
 *          exactly like the reference.
 *   acc    fp32 (B, KVH, S, G, D) contiguous; m, l fp32 (B, KVH, S, G)
 *          contiguous: per-split partials (S = `splits`) with the reference's
 *          meaning (unnormalised sum p*v, running max in natural-log units,
 *          sum p).  Split s covers [s*split_len, min(+split_len, upper)) with
 *          split_len = ceil(upper / S) rounded up to a multiple of 32.
 *          With splits = 1 one workgroup per (b, kv head) covers every slot,
 *          merges its waves in LDS and writes `out` itself: acc, m, l and the
 *          ticket are not read or written.
 *   ticket NULL: the merge runs as a second kernel (reference two-launch
 *          shape).  Non-NULL: int32[B*KVH], one counter per (b, kv head),
 *          zero-filled once by the caller; the merge runs inside the same
 *          launch: every workgroup of a (b, h) stores its partial, waits for
 *          the stores to complete and increments the counter, and the
 *          workgroup that completes the count (splits increments) merges all
 *          `splits` partials, writes the output and re-arms the counter to 0,
 *          so the same ticket serves every later call.  Calls that share a
 *          ticket or the partials must not overlap in time.
 *   out    (B, KVH, G, D) fp16, strides o_sb, o_sh, o_sg.
 *   scale  the score scale, D**-0.5 in the reference.
 */
int qf_decode_attn(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sg,
                   const void* k, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                   const void* v, int64_t v_sb, int64_t v_sh, int64_t v_sn,
                   const void* bias, int64_t bias_sb,
                   const int64_t* kv_last, int64_t kv_last_sb,
                   float* acc, float* m, float* l, int splits,
                   int32_t* ticket,
                   void* out, int64_t o_sb, int64_t o_sh, int64_t o_sg,
                   int B, int KVH, int G, int D, int cap, float scale,
                   void* stream);

/*
 * Launch plan of the decode split kernel (host only, no GPU work): the
 * wave64 count per workgroup qf_decode_attn / qf_decode_split launch with
 * for these arguments (`fused` = a ticket is passed), or QF_ERR_INVALID_ARG.
 * The kernel is decode_split_kernel<waves, bias, merge mode, paged>; tools
 * use this to name the kernel a measurement covers.
 */
int qf_decode_waves(int B, int KVH, int G, int cap, int splits, int fused);

/*
 * qf_decode_attn without caller scratch.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under hipGraph
 * capture, tight serving loops, harnesses that forbid hipMalloc).
 *
 * Arguments and results are qf_decode_attn's minus acc/m/l/ticket: the
 * per-split partials and the merge counters live in a static device array of
 * the library, one copy per GPU (QF_NOALLOC_PARTIAL_BYTES of partials plus
 * 256 KiB of counters, held until the process ends).  The merge is the one
 * qf_decode_attn picks for the same split count with a caller ticket for
 * 2..32 splits and without one above 32, so the output equals
 * qf_decode_attn's bit for bit.
 *
 *   - Returns QF_ERR_SCRATCH_LIMIT (nothing launched) when
 *     B*KVH*splits*G*(D+2)*4 > QF_NOALLOC_PARTIAL_BYTES.
 *   - The first call on a device looks the array up with
 *     hipGetSymbolAddress and zeroes its counters with a fill kernel on
 *     `stream`; nothing is allocated, ever.
 *   - Every call on one GPU shares that GPU's array: calls that overlap in
 *     time on one GPU (different streams, or concurrent graph replays) race
 *     and must be serialised by the caller.
 */
int qf_decode_attn_noalloc(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sg,
                           const void* k, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                           const void* v, int64_t v_sb, int64_t v_sh, int64_t v_sn,
                           const void* bias, int64_t bias_sb,
                           const int64_t* kv_last, int64_t kv_last_sb,
                           int splits,
                           void* out, int64_t o_sb, int64_t o_sh, int64_t o_sg,
                           int B, int KVH, int G, int D, int cap, float scale,
                           void* stream);

/*
 * The two launches of the reference's decode, separately (SE:854-865 and
 * SE:866-873): qf_decode_split writes the per-split partials (acc, m, l) with
 * the contract of qf_decode_attn; qf_decode_combine merges `splits` partials
 * of every (b, kv head) into `out`.  qf_decode_attn with ticket == NULL is
 * exactly split followed by combine.
 */
int qf_decode_split(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sg,
                    const void* k, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                    const void* v, int64_t v_sb, int64_t v_sh, int64_t v_sn,
                    const void* bias, int64_t bias_sb,
                    const int64_t* kv_last, int64_t kv_last_sb,
                    float* acc, float* m, float* l, int splits,
                    int B, int KVH, int G, int D, int cap, float scale,
                    void* stream);

/*
 * qf_decode_split over the reference's split ranges: split s covers
 * [s*split_len, min(+split_len, cap)) with split_len = ceil(cap / S) rounded
 * up to a multiple of 32, as _flash_decode_attention computes it
 * (student_engine.py:851), and kv_last (optional) only masks: slots past it
 * are read and given zero weight.  The ranges then need no device load, so
 * the first K/V loads do not wait for kv_last.  For callers whose rows fill
 * most of the capacity, such as a decode engine's per-layer caches (the
 * slots past kv_last are read for nothing).  Partials have
 * qf_decode_split's layout and meaning; a split past kv_last holds the empty
 * state (m = -inf, l = 0, acc = 0), which every merge drops.
 */
int qf_decode_split_capacity(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sg,
                             const void* k, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                             const void* v, int64_t v_sb, int64_t v_sh, int64_t v_sn,
                             const void* bias, int64_t bias_sb,
                             const int64_t* kv_last, int64_t kv_last_sb,
                             float* acc, float* m, float* l, int splits,
                             int B, int KVH, int G, int D, int cap, float scale,
                             void* stream);

int qf_decode_combine(const float* acc, const float* m, const float* l, int splits,
                      void* out, int64_t o_sb, int64_t o_sh, int64_t o_sg,
                      int B, int KVH, int G, int D, void* stream);

/*
 * Causal GQA flash-prefill.
 *
 * Replaces _gqa_flash_prefill_kernel (student_engine.py:164-251) as launched
 * by student_qwen::gqa_flash_prefill (:254-280): query head h reads kv head
 * h / (QH/KVH); key j is visible to query i iff j <= i.  V has its own
 * strides (the reference reuses K's, :208-209).
 *
 *   q (B, QH, S, D), k/v (B, KVH, S, D) -> out (B, QH, S, D) fp16.
 *
 * Optional fusions (pass NULL to disable):
 *   cos, sin (B, S, D) fp16 tables, strides cs_sb (0 = shared by the batch)
 *          and cs_sn: rotate-half RoPE is applied to q and k in registers with
 *          the eager fp16 rounding of SE:927-928 / SE:552-553
 *          (fp16(fp16(x*cos) + fp16(rotate_half(x)*sin))).
 *   k_cache, v_cache (B, KVH, cap, D): the post-RoPE k and the raw v of token
 *          i are written to slot start_pos + i (the slice copy of
 *          SE:715-716); both or neither.  Requires start_pos + S <= cap.
 *
 * Needs no scratch memory: one workgroup per 64-row query tile, the key
 * range split over its two halves of waves and merged in LDS.
 */
int qf_prefill_attn(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sn,
                    const void* k, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                    const void* v, int64_t v_sb, int64_t v_sh, int64_t v_sn,
                    const void* cos, const void* sin, int64_t cs_sb, int64_t cs_sn,
                    void* k_cache, int64_t kc_sb, int64_t kc_sh, int64_t kc_sn,
                    void* v_cache, int64_t vc_sb, int64_t vc_sh, int64_t vc_sn,
                    int64_t start_pos, int cap,
                    void* out, int64_t o_sb, int64_t o_sh, int64_t o_sn,
                    int B, int QH, int KVH, int S, int D, float scale,
                    void* stream);


/*
 * Ragged (variable-length) causal prefill of B packed rows, with the same
 * optional RoPE and cache-append fusions.  Replaces _prefill_ragged
 * (student_engine.py:1162-1204), which runs _prefill once per row and copies
 * each row's K/V into cache[row, :, :len] -- here one launch covers every row.
 *
 *   q (T, QH, D), k/v (T, KVH, D), out (T, QH, D): the B rows packed along
 *          the token axis (strides *_sh per head, *_sn per token); row b is
 *          tokens [cu_seqlens[b], cu_seqlens[b+1]) (int32 device array of
 *          B+1 entries, cu_seqlens[0] = 0, total = T = cu_seqlens[B]).
 *   max_seqlen  the longest row (sizes the grid; rows are clamped to it and
 *          to [0, total), so no cu content reads or writes out of bounds).
 *   cos, sin (T, D): per-token tables (each row's positions 0..len-1),
 *          token stride cs_sn.  RoPE requires the cache (both or neither).
 *   k_cache, v_cache (B, KVH, cap, D): token i of row b goes to slot
 *          start_pos + i of row b.  Requires start_pos + max_seqlen <= cap.
 */
int qf_prefill_varlen(const void* q, int64_t q_sh, int64_t q_sn,
                      const void* k, int64_t k_sh, int64_t k_sn,
                      const void* v, int64_t v_sh, int64_t v_sn,
                      const int32_t* cu_seqlens, int total, int max_seqlen,
                      const void* cos, const void* sin, int64_t cs_sn,
                      void* k_cache, int64_t kc_sb, int64_t kc_sh, int64_t kc_sn,
                      void* v_cache, int64_t vc_sb, int64_t vc_sh, int64_t vc_sn,
                      int64_t start_pos, int cap,
                      void* out, int64_t o_sh, int64_t o_sn,
                      int B, int QH, int KVH, int D, float scale, void* stream);

/*
 * One-token RoPE + KV-cache append (decode).
 *
 * Replaces the eager RoPE of the graph step (student_engine.py:927-928, with
 * the per-step cos/sin of :912-915 passed in) and the two index_copy_ calls
 * (:931-932):
 *
 *   q (B, QH, D), k/v (B, KVH, D)  the new token (head strides *_sh)
 *   cos, sin (B, D) fp16, row stride cs_sb
 *   k_cache[b, h, slot] = rope(k[b, h]);  v_cache[b, h, slot] = v[b, h]
 *   q_out[b, h] = rope(q[b, h])             (B, QH, D), strides qo_sb, qo_sh
 *
 * slot = write_index[0], read on the device (so a captured graph picks up the
 * value current at each replay).  A slot outside [0, cap) writes nothing to
 * the caches (q_out is still written).
 */
int qf_rope_append(const void* q, int64_t q_sb, int64_t q_sh,
                   const void* k, int64_t k_sb, int64_t k_sh,
                   const void* v, int64_t v_sb, int64_t v_sh,
                   const void* cos, const void* sin, int64_t cs_sb,
                   void* k_cache, int64_t kc_sb, int64_t kc_sh, int64_t kc_sn,
                   void* v_cache, int64_t vc_sb, int64_t vc_sh, int64_t vc_sn,
                   const int64_t* write_index,
                   void* q_out, int64_t qo_sb, int64_t qo_sh,
                   int B, int QH, int KVH, int D, int cap,
                   void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QF_ATTN_H */
