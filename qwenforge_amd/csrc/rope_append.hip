// One-token rotate-half RoPE + KV-cache append for gfx950 (MI355X).
//
// Replaces the graph step's eager RoPE (student_engine.py:927-928, cos/sin
// from :912-915 passed in) and its two index_copy_ calls (:931-932).  The
// slot is read from device memory, so a captured hipGraph writes the slot
// that is current at each replay, exactly like index_copy_ with the
// write_index tensor.  Rounding follows the eager fp16 sequence bit for bit.
//
// One workgroup per batch row; each work item is one 8-wide chunk pair
// (dims c..c+7 and c+32..c+39) of one head, so both halves of every
// rotate-half pair are in the same thread.
#include "qf_common.h"
#include "../../include/qf_attn.h"
#include "../../include/qf_paged.h"

namespace qf {
namespace rope_append {

struct Args {
  const f16* q;
  int64_t q_sb, q_sh;
  const f16* k;
  int64_t k_sb, k_sh;
  const f16* v;
  int64_t v_sb, v_sh;
  const f16* cos;
  const f16* sin;
  int64_t cs_sb;
  f16* kc;
  int64_t kc_sb, kc_sh, kc_sn;
  f16* vc;
  int64_t vc_sb, vc_sh, vc_sn;
  const int64_t* write_index;
  f16* q_out;
  int64_t qo_sb, qo_sh;
  int QH, KVH, cap;
  // Paged caches: kc/vc are page pools with page strides kc_sb/vc_sb; row b
  // appends at logical slot slots[b * slot_sb], in page
  // table[b * t_sb + (slot >> log2p)].  cap = pages per row << log2p.
  const int32_t* table;
  int64_t t_sb;
  int log2p, n_pages;
  const int64_t* slots;
  int64_t slot_sb;
};
static_assert(covers_lines(sizeof(Args), {offsetof(Args, q), offsetof(Args, cos),
                                          offsetof(Args, write_index), offsetof(Args, cap)}),
              "touch_arg_lines fields cover every line");

template <bool kPaged>
__global__ __launch_bounds__(256) void rope_append_kernel(Args a) {
  const int b = touch_arg_lines((int)blockIdx.x, a.q, a.cos, a.write_index, a.cap);
  // Element offsets of row b's destination slot (kv head 0) in the caches.
  int64_t kro, vro;
  bool in_range;
  if (kPaged) {
    const int64_t slot = a.slots[b * a.slot_sb];
    in_range = slot >= 0 && slot < a.cap;
    const int64_t sl = in_range ? slot : 0;  // branch-free table read
    const int page = a.table[b * a.t_sb + (sl >> a.log2p)];
    in_range = in_range && page >= 0 && page < a.n_pages;
    const int64_t row = sl & ((1 << a.log2p) - 1);
    kro = (int64_t)page * a.kc_sb + row * a.kc_sn;
    vro = (int64_t)page * a.vc_sb + row * a.vc_sn;
  } else {
    const int64_t slot = a.write_index[0];
    in_range = slot >= 0 && slot < a.cap;
    kro = b * a.kc_sb + slot * a.kc_sn;
    vro = b * a.vc_sb + slot * a.vc_sn;
  }
  const int n_rope = (a.QH + a.KVH) * 4;  // chunk pairs to rotate
  const int n_items = n_rope + a.KVH * 8;  // + 8-wide V chunks to copy
  for (int it = threadIdx.x; it < n_items; it += blockDim.x) {
    if (it < n_rope) {
      const int head = it >> 2, c = it & 3;
      const f16* cp = a.cos + b * a.cs_sb + 8 * c;
      const f16* sp = a.sin + b * a.cs_sb + 8 * c;
      if (head < a.QH) {
        const f16* src = a.q + b * a.q_sb + head * a.q_sh + 8 * c;
        f16x8 lo = load16(src), hi = load16(src + 32);
        rope_pair(lo, hi, load16(cp), load16(sp), load16(cp + 32), load16(sp + 32));
        f16* dst = a.q_out + b * a.qo_sb + head * a.qo_sh + 8 * c;
        store16(dst, lo);
        store16(dst + 32, hi);
      } else {
        const int h = head - a.QH;
        const f16* src = a.k + b * a.k_sb + h * a.k_sh + 8 * c;
        f16x8 lo = load16(src), hi = load16(src + 32);
        rope_pair(lo, hi, load16(cp), load16(sp), load16(cp + 32), load16(sp + 32));
        if (in_range) {
          f16* dst = a.kc + kro + h * a.kc_sh + 8 * c;
          store16(dst, lo);
          store16(dst + 32, hi);
        }
      }
    } else {
      const int j = it - n_rope;
      const int h = j >> 3, c = j & 7;
      if (in_range)
        store16(a.vc + vro + h * a.vc_sh + 8 * c,
                load16(a.v + b * a.v_sb + h * a.v_sh + 8 * c));
    }
  }
}

}  // namespace rope_append
}  // namespace qf

using namespace qf;

static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

extern "C" int qf_rope_append(const void* q, int64_t q_sb, int64_t q_sh,
                              const void* k, int64_t k_sb, int64_t k_sh,
                              const void* v, int64_t v_sb, int64_t v_sh,
                              const void* cos, const void* sin, int64_t cs_sb,
                              void* k_cache, int64_t kc_sb, int64_t kc_sh, int64_t kc_sn,
                              void* v_cache, int64_t vc_sb, int64_t vc_sh, int64_t vc_sn,
                              const int64_t* write_index,
                              void* q_out, int64_t qo_sb, int64_t qo_sh,
                              int B, int QH, int KVH, int D, int cap,
                              void* stream) {
  if (D != 64) return QF_ERR_UNSUPPORTED;
  if (!q || !k || !v || !cos || !sin || !k_cache || !v_cache || !write_index || !q_out)
    return QF_ERR_INVALID_ARG;
  if (B < 1 || QH < 1 || KVH < 1 || cap < 1 || B > 65535) return QF_ERR_INVALID_ARG;
  if (!al16(q) || !al16(k) || !al16(v) || !al16(cos) || !al16(sin) || !al16(k_cache) ||
      !al16(v_cache) || !al16(q_out))
    return QF_ERR_INVALID_ARG;
  if ((q_sb | q_sh | k_sb | k_sh | v_sb | v_sh | cs_sb | kc_sb | kc_sh | kc_sn | vc_sb | vc_sh |
       vc_sn | qo_sb | qo_sh) & 7)
    return QF_ERR_INVALID_ARG;

  rope_append::Args a;
  a.q = static_cast<const f16*>(q); a.q_sb = q_sb; a.q_sh = q_sh;
  a.k = static_cast<const f16*>(k); a.k_sb = k_sb; a.k_sh = k_sh;
  a.v = static_cast<const f16*>(v); a.v_sb = v_sb; a.v_sh = v_sh;
  a.cos = static_cast<const f16*>(cos); a.sin = static_cast<const f16*>(sin); a.cs_sb = cs_sb;
  a.kc = static_cast<f16*>(k_cache); a.kc_sb = kc_sb; a.kc_sh = kc_sh; a.kc_sn = kc_sn;
  a.vc = static_cast<f16*>(v_cache); a.vc_sb = vc_sb; a.vc_sh = vc_sh; a.vc_sn = vc_sn;
  a.write_index = write_index;
  a.q_out = static_cast<f16*>(q_out); a.qo_sb = qo_sb; a.qo_sh = qo_sh;
  a.QH = QH; a.KVH = KVH; a.cap = cap;
  a.table = nullptr; a.t_sb = 0; a.log2p = 0; a.n_pages = 0; a.slots = nullptr; a.slot_sb = 0;
  hipLaunchKernelGGL(rope_append::rope_append_kernel<false>, dim3(B), dim3(128), 0,
                     static_cast<hipStream_t>(stream), a);
  return (int)hipGetLastError();
}

extern "C" int qf_rope_append_paged(const void* q, int64_t q_sb, int64_t q_sh,
                                    const void* k, int64_t k_sb, int64_t k_sh,
                                    const void* v, int64_t v_sb, int64_t v_sh,
                                    const void* cos, const void* sin, int64_t cs_sb,
                                    void* k_pool, int64_t kp_sp, int64_t kp_sh, int64_t kp_sn,
                                    void* v_pool, int64_t vp_sp, int64_t vp_sh, int64_t vp_sn,
                                    const int32_t* block_table, int64_t bt_sb, int pages_per_row,
                                    int n_pages, int page_size,
                                    const int64_t* slots, int64_t slot_sb,
                                    void* q_out, int64_t qo_sb, int64_t qo_sh,
                                    int B, int QH, int KVH, int D, void* stream) {
  const int l2 = page_log2(page_size, pages_per_row, n_pages);
  if (D != 64 || l2 < 0) return QF_ERR_UNSUPPORTED;
  if (!q || !k || !v || !cos || !sin || !k_pool || !v_pool || !block_table || !slots || !q_out)
    return QF_ERR_INVALID_ARG;
  if (B < 1 || QH < 1 || KVH < 1 || B > 65535 || bt_sb < pages_per_row) return QF_ERR_INVALID_ARG;
  if (!al16(q) || !al16(k) || !al16(v) || !al16(cos) || !al16(sin) || !al16(k_pool) ||
      !al16(v_pool) || !al16(q_out))
    return QF_ERR_INVALID_ARG;
  if ((q_sb | q_sh | k_sb | k_sh | v_sb | v_sh | cs_sb | kp_sp | kp_sh | kp_sn | vp_sp | vp_sh |
       vp_sn | qo_sb | qo_sh) & 7)
    return QF_ERR_INVALID_ARG;

  rope_append::Args a;
  a.q = static_cast<const f16*>(q); a.q_sb = q_sb; a.q_sh = q_sh;
  a.k = static_cast<const f16*>(k); a.k_sb = k_sb; a.k_sh = k_sh;
  a.v = static_cast<const f16*>(v); a.v_sb = v_sb; a.v_sh = v_sh;
  a.cos = static_cast<const f16*>(cos); a.sin = static_cast<const f16*>(sin); a.cs_sb = cs_sb;
  a.kc = static_cast<f16*>(k_pool); a.kc_sb = kp_sp; a.kc_sh = kp_sh; a.kc_sn = kp_sn;
  a.vc = static_cast<f16*>(v_pool); a.vc_sb = vp_sp; a.vc_sh = vp_sh; a.vc_sn = vp_sn;
  a.write_index = nullptr;
  a.q_out = static_cast<f16*>(q_out); a.qo_sb = qo_sb; a.qo_sh = qo_sh;
  a.QH = QH; a.KVH = KVH; a.cap = pages_per_row * page_size;
  a.table = block_table; a.t_sb = bt_sb; a.log2p = l2; a.n_pages = n_pages;
  a.slots = slots; a.slot_sb = slot_sb;
  hipLaunchKernelGGL(rope_append::rope_append_kernel<true>, dim3(B), dim3(128), 0,
                     static_cast<hipStream_t>(stream), a);
  return (int)hipGetLastError();
}
