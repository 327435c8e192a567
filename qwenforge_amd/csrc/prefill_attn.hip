// Causal GQA flash-prefill for gfx950 (MI355X), with rotate-half RoPE and the
// KV-cache append optionally fused in.
//
// Replaces _gqa_flash_prefill_kernel (student_engine.py:164-251) as launched by
// the student_qwen::gqa_flash_prefill custom op (:254-280), plus the eager
// RoPE in front of it (:767, :542-554) and the slice append of the cached
// prefill (:715-716).
//
// One workgroup = 64 query rows of one query head (four wave64s x 16 rows);
// query tiles are launched heaviest-first (the last rows see the most keys).
// Per 64-key tile the workgroup cooperatively
//   - loads K with 16-byte loads, applies RoPE in registers (both halves of a
//     rotate-half pair are loaded by the same thread), stores the rotated rows
//     to LDS in natural [key][d] layout,
//   - loads V and stores it transposed ([d][key]) to LDS,
//   - on the diagonal tile of the group's first query head, also writes the
//     rotated K and raw V into the cache (each key tile is written exactly
//     once per (b, kv head)).
// Each wave then computes S^T = K Q^T and O^T += V^T P^T with
// v_mfma_f32_16x16x32_f16 and an online softmax in the log2 domain; Q is
// rotated in registers once at the start.
#include "qf_common.h"
#include "../../include/qf_attn.h"

namespace qf {

namespace prefill {

constexpr int kD = 64;
constexpr int kBM = 64;        // query rows per workgroup
constexpr int kBN = 64;        // keys per tile
constexpr int kWaves = 4;
constexpr int kKStride = 72;   // LDS row stride (halves) of the K tile
constexpr int kVtStride = 72;  // LDS row stride (halves) of the V^T tile

struct Args {
  const f16* q;
  int64_t q_sb, q_sh, q_sn;
  const f16* k;
  int64_t k_sb, k_sh, k_sn;
  const f16* v;
  int64_t v_sb, v_sh, v_sn;
  const f16* cos;
  const f16* sin;
  int64_t cs_sb, cs_sn;
  f16* kc;
  int64_t kc_sb, kc_sh, kc_sn;
  f16* vc;
  int64_t vc_sb, vc_sh, vc_sn;
  int64_t start_pos;
  f16* out;
  int64_t o_sb, o_sh, o_sn;
  int B, QH, KVH, G, S;
  float scale_log2;
};

template <bool kRope, bool kAppend>
__global__ __launch_bounds__(kWaves * 64) void prefill_kernel(Args a) {
  __shared__ __attribute__((aligned(16))) f16 ks[kBN][kKStride];
  __shared__ __attribute__((aligned(16))) f16 vts[kD][kVtStride];

  const int n_mtiles = gridDim.x;
  const int mt = n_mtiles - 1 - blockIdx.x;  // heaviest tiles first
  const int bq = blockIdx.y;
  const int b = bq / a.QH, hq = bq % a.QH;
  const int hk = hq / a.G;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int S = a.S;

  // ---- Q^T operand (16 rows per wave), rotated in registers.
  const int qrow = mt * kBM + w * 16 + col;
  f16x8 qf[2];
  {
    const int qr = qrow < S ? qrow : S - 1;
    const f16* qp = a.q + b * a.q_sb + hq * a.q_sh + (int64_t)qr * a.q_sn + 8 * grp;
    qf[0] = load16(qp);
    qf[1] = load16(qp + 32);
    if (kRope) {
      const int64_t co = b * a.cs_sb + (int64_t)qr * a.cs_sn + 8 * grp;
      rope_pair(qf[0], qf[1], load16(a.cos + co), load16(a.sin + co), load16(a.cos + co + 32),
                load16(a.sin + co + 32));
    }
  }

  float m_run = kNegInf, l_run = 0.f;
  f32x4 o[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const f16* kb = a.k + b * a.k_sb + hk * a.k_sh;
  const f16* vb = a.v + b * a.v_sb + hk * a.v_sh;
  const bool writer = kAppend && (hq % a.G == 0);
  const int key_end = (mt + 1) * kBM < S ? (mt + 1) * kBM : S;
  const int n_ktiles = (key_end + kBN - 1) / kBN;

  // Loader mapping: thread -> (key row, 8-wide chunk pair c / c+4 for K,
  // 16-wide slice for V).
  const int ld_key = tid >> 2, ld_c = tid & 3;

  for (int kt = 0; kt < n_ktiles; ++kt) {
    const int key0 = kt * kBN;
    {
      const int key = key0 + ld_key;
      const int kc = key < S ? key : S - 1;
      f16x8 klo = load16(kb + (int64_t)kc * a.k_sn + 8 * ld_c);
      f16x8 khi = load16(kb + (int64_t)kc * a.k_sn + 32 + 8 * ld_c);
      if (kRope) {
        const int64_t co = b * a.cs_sb + (int64_t)kc * a.cs_sn + 8 * ld_c;
        rope_pair(klo, khi, load16(a.cos + co), load16(a.sin + co), load16(a.cos + co + 32),
                  load16(a.sin + co + 32));
      }
      *reinterpret_cast<f16x8*>(&ks[ld_key][8 * ld_c]) = klo;
      *reinterpret_cast<f16x8*>(&ks[ld_key][32 + 8 * ld_c]) = khi;
      const f16x8 v0 = load16(vb + (int64_t)kc * a.v_sn + 16 * ld_c);
      const f16x8 v1 = load16(vb + (int64_t)kc * a.v_sn + 16 * ld_c + 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        vts[16 * ld_c + e][ld_key] = v0[e];
        vts[16 * ld_c + 8 + e][ld_key] = v1[e];
      }
      if (writer && kt == mt && key < S) {
        const int64_t slot = a.start_pos + key;
        f16* kd = a.kc + b * a.kc_sb + hk * a.kc_sh + slot * a.kc_sn;
        f16* vd = a.vc + b * a.vc_sb + hk * a.vc_sh + slot * a.vc_sn;
        store16(kd + 8 * ld_c, klo);
        store16(kd + 32 + 8 * ld_c, khi);
        store16(vd + 16 * ld_c, v0);
        store16(vd + 16 * ld_c + 8, v1);
      }
    }
    __syncthreads();

    // Two 32-key chunks per tile.
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      f32x4 c[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int krow = 32 * ch + 8 * (col >> 2) + 4 * j + (col & 3);
        const f16x8 a0 = *reinterpret_cast<const f16x8*>(&ks[krow][8 * grp]);
        const f16x8 a1 = *reinterpret_cast<const f16x8*>(&ks[krow][32 + 8 * grp]);
        c[j] = f32x4{0.f, 0.f, 0.f, 0.f};
        c[j] = mfma16x16x32(a0, qf[0], c[j]);
        c[j] = mfma16x16x32(a1, qf[1], c[j]);
      }
      float sc[8];
      const int kbase = key0 + 32 * ch + 8 * grp;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int key = kbase + jj;
        const float x = (jj < 4 ? c[0][jj] : c[1][jj - 4]) * a.scale_log2;
        sc[jj] = (key <= qrow && key < S) ? x : kNegInf;
      }
      float mx = sc[0];
#pragma unroll
      for (int jj = 1; jj < 8; ++jj) mx = fmaxf(mx, sc[jj]);
      mx = col_max(mx);
      const float m_new = fmaxf(m_run, mx);
      const float safe_m = (m_new == kNegInf) ? 0.f : m_new;
      const float resc = (m_new == kNegInf) ? 1.f : fast_exp2(m_run - m_new);
      float psum = 0.f;
      f16x8 pb;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const float p = (sc[jj] == kNegInf) ? 0.f : fast_exp2(sc[jj] - safe_m);
        psum += p;
        pb[jj] = (f16)p;
      }
      l_run = l_run * resc + psum;
      m_run = m_new;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const f16x8 va = *reinterpret_cast<const f16x8*>(&vts[16 * t + col][32 * ch + 8 * grp]);
        o[t] = mfma16x16x32(va, pb, o[t] * resc);
      }
    }
    __syncthreads();
  }

  l_run = col_sum(l_run);
  if (qrow < S) {
    const float inv = 1.f / l_run;
    f16* op = a.out + b * a.o_sb + hq * a.o_sh + (int64_t)qrow * a.o_sn;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      f16x4 r;
#pragma unroll
      for (int i = 0; i < 4; ++i) r[i] = (f16)(o[t][i] * inv);
      *reinterpret_cast<f16x4*>(op + 16 * t + 4 * grp) = r;
    }
  }
}

}  // namespace prefill
}  // namespace qf

using namespace qf;

static bool aligned16p(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

extern "C" int qf_prefill_attn(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sn,
                               const void* k, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                               const void* v, int64_t v_sb, int64_t v_sh, int64_t v_sn,
                               const void* cos, const void* sin, int64_t cs_sb, int64_t cs_sn,
                               void* k_cache, int64_t kc_sb, int64_t kc_sh, int64_t kc_sn,
                               void* v_cache, int64_t vc_sb, int64_t vc_sh, int64_t vc_sn,
                               int64_t start_pos, int cap,
                               void* out, int64_t o_sb, int64_t o_sh, int64_t o_sn,
                               int B, int QH, int KVH, int S, int D, float scale,
                               void* stream) {
  using namespace qf::prefill;
  if (D != kD) return QF_ERR_UNSUPPORTED;
  if (!q || !k || !v || !out) return QF_ERR_INVALID_ARG;
  if (B < 1 || KVH < 1 || QH < KVH || QH % KVH != 0 || S < 1) return QF_ERR_INVALID_ARG;
  if ((int64_t)B * QH > 65535) return QF_ERR_INVALID_ARG;
  const bool rope = cos != nullptr || sin != nullptr;
  if (rope && (!cos || !sin)) return QF_ERR_INVALID_ARG;
  const bool append = k_cache != nullptr || v_cache != nullptr;
  if (append && (!k_cache || !v_cache)) return QF_ERR_INVALID_ARG;
  if (append && (start_pos < 0 || start_pos + S > cap)) return QF_ERR_INVALID_ARG;
  if (!aligned16p(q) || !aligned16p(k) || !aligned16p(v)) return QF_ERR_INVALID_ARG;
  if ((q_sb | q_sh | q_sn | k_sb | k_sh | k_sn | v_sb | v_sh | v_sn) & 7) return QF_ERR_INVALID_ARG;
  if ((reinterpret_cast<uintptr_t>(out) & 7u) || ((o_sb | o_sh | o_sn) & 3)) return QF_ERR_INVALID_ARG;
  if (rope && (!aligned16p(cos) || !aligned16p(sin) || ((cs_sb | cs_sn) & 7))) return QF_ERR_INVALID_ARG;
  if (append && (!aligned16p(k_cache) || !aligned16p(v_cache) ||
                 ((kc_sb | kc_sh | kc_sn | vc_sb | vc_sh | vc_sn) & 7)))
    return QF_ERR_INVALID_ARG;

  Args a;
  a.q = static_cast<const f16*>(q);
  a.q_sb = q_sb; a.q_sh = q_sh; a.q_sn = q_sn;
  a.k = static_cast<const f16*>(k);
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_sn = k_sn;
  a.v = static_cast<const f16*>(v);
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_sn = v_sn;
  a.cos = static_cast<const f16*>(cos);
  a.sin = static_cast<const f16*>(sin);
  a.cs_sb = cs_sb; a.cs_sn = cs_sn;
  a.kc = static_cast<f16*>(k_cache);
  a.kc_sb = kc_sb; a.kc_sh = kc_sh; a.kc_sn = kc_sn;
  a.vc = static_cast<f16*>(v_cache);
  a.vc_sb = vc_sb; a.vc_sh = vc_sh; a.vc_sn = vc_sn;
  a.start_pos = start_pos;
  a.out = static_cast<f16*>(out);
  a.o_sb = o_sb; a.o_sh = o_sh; a.o_sn = o_sn;
  a.B = B; a.QH = QH; a.KVH = KVH; a.G = QH / KVH; a.S = S;
  a.scale_log2 = scale * kLog2e;

  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid((S + kBM - 1) / kBM, B * QH), block(kWaves * 64);
  if (rope && append) hipLaunchKernelGGL((prefill_kernel<true, true>), grid, block, 0, st, a);
  else if (rope) hipLaunchKernelGGL((prefill_kernel<true, false>), grid, block, 0, st, a);
  else if (append) hipLaunchKernelGGL((prefill_kernel<false, true>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((prefill_kernel<false, false>), grid, block, 0, st, a);
  return (int)hipGetLastError();
}
