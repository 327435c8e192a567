// VALU dot-product form of the decode split kernel, kept for one purpose: to
// measure, beside the matrix-core kernel (decode_attn.hip), whether packing a
// GQA group's query heads into one 16-column MFMA tile beats plain VALU dot
// products.  It is not on the hot path; qf_decode_split_valu (qf_probe.h)
// writes the same partials (acc, m, l) as qf_decode_split, so the library's
// combine launch merges either.
//
// Layout of the work (one workgroup of kNW waves per (split, b, kv head), the
// waves interleaved over 64-key tiles, the next tile's loads issued before
// the current tile is computed, all K/V loads non-temporal like the MFMA
// kernel's):
//   q.k   lane = key: the lane holds its key's K row (eight 16-byte loads)
//         and runs v_dot2_f32_f16 against the G query rows, read from LDS as
//         broadcasts;
//   softmax  per query, the tile maximum is a wave reduction (DPP within
//         rows of 16 lanes, then gfx950 permlane swaps across rows); the
//         running sum stays per lane until the end;
//   p.V   lane = (key half, dim pair): V rows are loaded coalesced (8 lanes
//         per 128-byte row) into LDS, the probabilities (rounded to fp16, as
//         the MFMA kernel feeds them) go to LDS as one 16-byte row per key,
//         and each lane accumulates its two dims over its 32 keys with fp32
//         FMAs; the two key halves add up through a permlane swap.
#include "qf_common.h"
#include "../../include/qf_attn.h"
#include "../../include/qf_probe.h"

namespace qf {
namespace valu {

constexpr int kNW = 4;        // waves per workgroup
constexpr int kG = 7;         // query heads per kv head (Qwen2.5-0.5B)
constexpr int kD = 64;
constexpr int kKT = 64;       // keys per wave tile (one per lane)
constexpr int kVs = kD + 2;   // LDS row stride (halves) of a V tile: 132 bytes

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

struct Args {
  const f16* q;
  int64_t q_sb, q_sh, q_sg;
  const f16* k;
  int64_t k_sb, k_sh, k_sn;
  const f16* v;
  int64_t v_sb, v_sh, v_sn;
  const int64_t* kv_last;
  int64_t kv_last_sb;
  float* acc;
  float* m;
  float* l;
  int KVH, cap, splits;
  float scale_log2;
};
static_assert(covers_lines(sizeof(Args), {offsetof(Args, q), offsetof(Args, v), offsetof(Args, KVH)}),
              "touch_arg_lines fields cover every line");

__device__ __forceinline__ float dpp_f(float x, int ctrl) {
  // Row-local lane shuffle; ctrl is a compile-time DPP control.
  switch (ctrl) {
    case 0xB1: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
    case 0x4E: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));
    case 0x141: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false));
    default: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false));
  }
}

// Maximum over the 64 lanes: quad_perm [1,0,3,2], [2,3,0,1], row half
// mirror and row mirror leave every lane of a 16-lane row with the row's
// maximum; the permlane swaps then combine rows l ^ 16 and l ^ 32.
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp_f(x, 0xB1));
  x = fmaxf(x, dpp_f(x, 0x4E));
  x = fmaxf(x, dpp_f(x, 0x141));
  x = fmaxf(x, dpp_f(x, 0x140));
  float a, b;
  xor16_pair(x, a, b);
  xor32_pair(fmaxf(a, b), a, b);
  return fmaxf(a, b);
}

__device__ __forceinline__ float wave_sum(float x) {
  x += dpp_f(x, 0xB1);
  x += dpp_f(x, 0x4E);
  x += dpp_f(x, 0x141);
  x += dpp_f(x, 0x140);
  float a, b;
  xor16_pair(x, a, b);
  xor32_pair(a + b, a, b);
  return a + b;
}

struct Tile {
  f16x8 k[8];   // the lane's key row
  f16x8 v[8];   // 8 coalesced 16-byte pieces: rows t0 + 8i + lane / 8, dims 8 * (lane % 8)
};

__device__ __forceinline__ void load_tile(Tile& t, const f16* kb, const f16* vb, int64_t k_sn,
                                          int64_t v_sn, int t0, int last, int lane) {
  int key = t0 + lane;
  key = key < last ? key : last;
#pragma unroll
  for (int c = 0; c < 8; ++c) t.k[c] = load16_nt(kb + (int64_t)key * k_sn + 8 * c);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int r = t0 + 8 * i + (lane >> 3);
    r = r < last ? r : last;
    t.v[i] = load16_nt(vb + (int64_t)r * v_sn + 8 * (lane & 7));
  }
}

__global__ __launch_bounds__(kNW * 64) void decode_split_valu_kernel(Args a) {
  __shared__ __attribute__((aligned(16))) f16 qs[kG][kD];
  __shared__ __attribute__((aligned(16))) f16 vs[kNW][kKT][kVs];
  __shared__ __attribute__((aligned(16))) f16 ps[kNW][kKT][8];
  __shared__ float mo[kNW][kG][kD];
  __shared__ float mm[kNW][kG], ml[kNW][kG];

  const int KVH = touch_arg_lines(a.KVH, a.q, a.v, a.acc);
  const int s = blockIdx.x, bh = blockIdx.y, b = bh / KVH, h = bh % KVH;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  for (int i = tid; i < kG * 8; i += kNW * 64) {
    const int q = i / 8, c = i % 8;
    *reinterpret_cast<f16x8*>(&qs[q][8 * c]) =
        load16(a.q + b * a.q_sb + h * a.q_sh + q * a.q_sg + 8 * c);
  }
  int upper = a.cap;
  if (a.kv_last != nullptr) {
    const int64_t last = a.kv_last[(int64_t)b * a.kv_last_sb];
    upper = (int)(last + 1 < 0 ? 0 : (last + 1 > a.cap ? a.cap : last + 1));
  }
  int split_len = (upper + a.splits - 1) / a.splits;
  split_len = (split_len + 31) / 32 * 32;
  const int lo = s * split_len;
  const int hi = lo + split_len < upper ? lo + split_len : upper;
  __syncthreads();

  float m_run[kG], l_run[kG], o[kG][2];
#pragma unroll
  for (int q = 0; q < kG; ++q) {
    m_run[q] = kNegInf;
    l_run[q] = 0.f;
    o[q][0] = o[q][1] = 0.f;
  }
  const f16* kb = a.k + b * a.k_sb + h * a.k_sh;
  const f16* vb = a.v + b * a.v_sb + h * a.v_sh;
  const int last = hi - 1;
  const int half = lane >> 5, dp = lane & 31;  // p.V roles

  const auto consume = [&](const Tile& t, int t0) __attribute__((always_inline)) {
    // V rows into this wave's LDS tile.
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 8 * i + (lane >> 3);
      f16* dst = &vs[w][r][8 * (lane & 7)];
      // 132-byte rows: 4-byte aligned only, so write as four dwords.
      const u32x4 x = __builtin_bit_cast(u32x4, t.v[i]);
#pragma unroll
      for (int e = 0; e < 4; ++e) reinterpret_cast<uint32_t*>(dst)[e] = x[e];
    }
    const bool valid = t0 + lane < hi;
    f16x8 pr;
#pragma unroll
    for (int q = 0; q < kG; ++q) {
      float d = 0.f;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const f16x8 qq = *reinterpret_cast<const f16x8*>(&qs[q][8 * c]);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          d = __builtin_amdgcn_fdot2(f16x2{t.k[c][2 * e], t.k[c][2 * e + 1]},
                                     f16x2{qq[2 * e], qq[2 * e + 1]}, d, false);
      }
      const float sc = valid ? d * a.scale_log2 : kNegInf;
      const float mt = wave_max(sc);
      const float mn = fmaxf(m_run[q], mt);
      const float safe = (mn == kNegInf) ? 0.f : mn;
      const float resc = (m_run[q] == kNegInf) ? 0.f : fast_exp2(m_run[q] - safe);
      const float p = (sc == kNegInf) ? 0.f : fast_exp2(sc - safe);
      l_run[q] = l_run[q] * resc + p;
      o[q][0] *= resc;
      o[q][1] *= resc;
      m_run[q] = mn;
      pr[q] = (f16)p;
    }
    pr[7] = (f16)0.f;
    *reinterpret_cast<f16x8*>(&ps[w][lane][0]) = pr;
    __builtin_amdgcn_wave_barrier();
    // p.V: lane (half, dp) takes keys 32 * half .. +31, dims 2dp, 2dp + 1.
#pragma unroll 8
    for (int kk = 0; kk < 32; ++kk) {
      const int key = 32 * half + kk;
      const f16x2 vv = *reinterpret_cast<const f16x2*>(&vs[w][key][2 * dp]);
      const f16x8 pp = *reinterpret_cast<const f16x8*>(&ps[w][key][0]);
      const float v0 = (float)vv[0], v1 = (float)vv[1];
#pragma unroll
      for (int q = 0; q < kG; ++q) {
        o[q][0] += (float)pp[q] * v0;
        o[q][1] += (float)pp[q] * v1;
      }
    }
    __builtin_amdgcn_wave_barrier();
  };

  constexpr int kStep = kNW * kKT;
  int t0 = lo + w * kKT;
  const int n = t0 < hi ? (hi - t0 + kStep - 1) / kStep : 0;
  if (n > 0) {
    Tile ta, tb;
    load_tile(ta, kb, vb, a.k_sn, a.v_sn, t0, last, lane);
    int i = 0;
    for (; i + 2 < n; i += 2, t0 += 2 * kStep) {
      load_tile(tb, kb, vb, a.k_sn, a.v_sn, t0 + kStep, last, lane);
      __builtin_amdgcn_sched_barrier(0);
      consume(ta, t0);
      load_tile(ta, kb, vb, a.k_sn, a.v_sn, t0 + 2 * kStep, last, lane);
      __builtin_amdgcn_sched_barrier(0);
      consume(tb, t0 + kStep);
    }
    if (i + 2 == n) {
      load_tile(tb, kb, vb, a.k_sn, a.v_sn, t0 + kStep, last, lane);
      __builtin_amdgcn_sched_barrier(0);
      consume(ta, t0);
      consume(tb, t0 + kStep);
    } else {
      consume(ta, t0);
    }
  }

  // The two key halves of each dim pair, then the wave's sums.
#pragma unroll
  for (int q = 0; q < kG; ++q) {
    float x0, y0, x1, y1;
    xor32_pair(o[q][0], x0, y0);
    xor32_pair(o[q][1], x1, y1);
    o[q][0] = x0 + y0;
    o[q][1] = x1 + y1;
    l_run[q] = wave_sum(l_run[q]);
  }
  if (half == 0) {
#pragma unroll
    for (int q = 0; q < kG; ++q) {
      mo[w][q][2 * dp] = o[q][0];
      mo[w][q][2 * dp + 1] = o[q][1];
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int q = 0; q < kG; ++q) {
      mm[w][q] = m_run[q];
      ml[w][q] = l_run[q];
    }
  }
  __syncthreads();
  const int64_t part = (int64_t)bh * a.splits + s;
  for (int e = tid; e < kG * kD; e += kNW * 64) {
    const int q = e / kD, d = e % kD;
    float M = kNegInf;
#pragma unroll
    for (int ww = 0; ww < kNW; ++ww) M = fmaxf(M, mm[ww][q]);
    const float safe = (M == kNegInf) ? 0.f : M;
    float so = 0.f, sl = 0.f;
#pragma unroll
    for (int ww = 0; ww < kNW; ++ww) {
      const float wt = (mm[ww][q] == kNegInf) ? 0.f : fast_exp2(mm[ww][q] - safe);
      so += wt * mo[ww][q][d];
      sl += wt * ml[ww][q];
    }
    a.acc[(part * kG + q) * kD + d] = so;
    if (d == 0) {
      a.m[part * kG + q] = (M == kNegInf) ? kNegInf : M * kLn2;
      a.l[part * kG + q] = sl;
    }
  }
}

}  // namespace valu
}  // namespace qf

extern "C" int qf_decode_split_valu(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sg,
                                    const void* k, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                                    const void* v, int64_t v_sb, int64_t v_sh, int64_t v_sn,
                                    const int64_t* kv_last, int64_t kv_last_sb,
                                    float* acc, float* m, float* l, int splits,
                                    int B, int KVH, int G, int D, int cap, float scale,
                                    void* stream) {
  using namespace qf::valu;
  if (G != kG || D != kD) return QF_ERR_UNSUPPORTED;
  if (!q || !k || !v || !acc || !m || !l || cap < 1) return QF_ERR_INVALID_ARG;
  if (B < 1 || KVH < 1 || splits < 1 || splits > 65535 || B * (int64_t)KVH > 65535)
    return QF_ERR_INVALID_ARG;
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if (!a16(q) || !a16(k) || !a16(v)) return QF_ERR_INVALID_ARG;
  if ((q_sb | q_sh | q_sg | k_sb | k_sh | k_sn | v_sb | v_sh | v_sn) & 7) return QF_ERR_INVALID_ARG;
  Args a{static_cast<const qf::f16*>(q), q_sb, q_sh, q_sg,
         static_cast<const qf::f16*>(k), k_sb, k_sh, k_sn,
         static_cast<const qf::f16*>(v), v_sb, v_sh, v_sn,
         kv_last, kv_last_sb, acc, m, l, KVH, cap, splits, scale * qf::kLog2e};
  hipLaunchKernelGGL(decode_split_valu_kernel, dim3(splits, B * KVH), dim3(kNW * 64), 0,
                     static_cast<hipStream_t>(stream), a);
  return (int)hipGetLastError();
}
