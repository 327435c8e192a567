// Fused weight-streaming decode-step kernels for gfx950 (MI355X).
//
// At decode batch sizes (B <= 4) every projection of the step is a
// matrix-vector product whose cost is streaming the weight matrix from HBM
// once; the arithmetic is a few fp16 dot products per loaded byte.  The
// kernels here therefore share one shape:
//
//   * a workgroup of four wave64s; each wave owns whole weight rows (1, 2 or 4
//     of them) and issues every 16-byte load of those rows up front, so a
//     wave keeps 2-10 KB of independent loads in flight;
//   * while the loads fly, the workgroup stages the B activation rows into
//     LDS, applying the RMSNorm prologue where the reference has one (the sum
//     of squares is a workgroup reduction; the row is tiny and L2-resident);
//   * the lanes of a wave stride over a row's 16-byte chunks, each chunk
//     meets the matching LDS chunk of every batch row in four v_dot2_f32_f16,
//     and a butterfly over the 64 lanes leaves each row total in every lane;
//   * the epilogue fuses what follows the projection in the reference:
//     bias + RoPE + KV append (QKV), SwiGLU (gate/up), residual add (o_proj,
//     down), and a per-block argmax key (lm_head).
//
// Replaces the torch op sequence of _decode_step_static
// (student_engine.py:896-982); see include/qf_step.h for the per-entry-point
// mapping and rounding.
#include "qf_common.h"
#include "../../include/qf_step.h"

namespace qf {
namespace step {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kNW = 4;          // waves per workgroup
constexpr int kNT = kNW * 64;   // threads per workgroup
constexpr int kMaxB = 4;        // batch rows per launch
constexpr int kMaxNormK = 1024; // widest normalised (hidden) row: one chunk per thread
constexpr int kMaxK = 8192;     // widest projection input (down_proj: intermediate)
constexpr int kHeadDim = 64;

__device__ __forceinline__ float dot8(f16x8 w, f16x8 x, float acc) {
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(w, w, 0, 1),
                               __builtin_shufflevector(x, x, 0, 1), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(w, w, 2, 3),
                               __builtin_shufflevector(x, x, 2, 3), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(w, w, 4, 5),
                               __builtin_shufflevector(x, x, 4, 5), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(w, w, 6, 7),
                               __builtin_shufflevector(x, x, 6, 7), acc, false);
  return acc;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ f16x8 zero8() {
  f16x8 z;
#pragma unroll
  for (int e = 0; e < 8; ++e) z[e] = (f16)0.f;
  return z;
}

// The NS 16-byte chunks of one weight row that lane `lane` multiplies:
// chunk 64*s + lane, s < NS (chunks past the row are zero).
template <int NS>
__device__ __forceinline__ void load_row(const f16* __restrict__ w, int C, f16x8 (&r)[NS],
                                         int lane) {
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int c = 64 * s + lane;
    r[s] = c < C ? load16(w + 8 * c) : zero8();
  }
}

// acc[b] += partial dot of the lane's chunks of a row with staged row b.
template <int NS, int NB>
__device__ __forceinline__ void dot_row(const f16x8 (&r)[NS], const f16* xs, int K, int C,
                                        float (&acc)[NB], int lane) {
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int c = 64 * s + lane;
    if (c < C) {
#pragma unroll
      for (int b = 0; b < NB; ++b)
        acc[b] = dot8(r[s], *reinterpret_cast<const f16x8*>(xs + b * K + 8 * c), acc[b]);
    }
  }
}

// Stages NB activation rows into LDS xs[b * K ..], RMS-normalised as torch's
// fused RMSNorm kernel does for fp16 (fp32 math, one rounding):
//   y = fp16((x * rsqrt(mean(x^2) + eps)) * w)     (student_engine.py:530-535 form)
// K <= kMaxNormK, so each thread owns at most one chunk per row.  When
// `raw_out` is non-null the unnormalised rows are also copied there.
template <int NB>
__device__ __forceinline__ void stage_rms(const f16* const (&rows)[NB], int K,
                                          const f16* __restrict__ nw, float eps, f16* xs,
                                          float* red, f16* raw_out, int64_t raw_sb) {
  const int C = K / 8;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  f16x8 xv[NB];
  float ss[NB];
  const bool own = tid < C;
  const f16x8 g = own ? load16(nw + 8 * tid) : zero8();
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    xv[b] = own ? load16(rows[b] + 8 * tid) : zero8();
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += (float)xv[b][e] * (float)xv[b][e];
    ss[b] = wave_sum(s);
    if (lane == 0) red[w * NB + b] = ss[b];
  }
  if (raw_out != nullptr && own) {
#pragma unroll
    for (int b = 0; b < NB; ++b) store16(raw_out + b * raw_sb + 8 * tid, xv[b]);
  }
  __syncthreads();
  if (own) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      float tot = 0.f;
#pragma unroll
      for (int ww = 0; ww < kNW; ++ww) tot += red[ww * NB + b];
      const float rstd = rsqrtf(tot / (float)K + eps);
      f16x8 y;
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = (f16)(((float)xv[b][e] * rstd) * (float)g[e]);
      store16(xs + b * K + 8 * tid, y);
    }
  }
  __syncthreads();
}

// Stages NB rows (row stride sb) into LDS unchanged.
template <int NB>
__device__ __forceinline__ void stage_plain(const f16* __restrict__ x, int64_t sb, int K,
                                            f16* xs) {
  const int C = K / 8;
  for (int i = threadIdx.x; i < NB * C; i += kNT) {
    const int b = i / C, c = i % C;
    store16(xs + b * K + 8 * c, load16(x + b * sb + 8 * c));
  }
  __syncthreads();
}

// Eager rotate-half RoPE of one (d, d+32) pair with the reference's fp16
// rounding (student_engine.py:927-928): lo' = fp16(fp16(lo*cos_lo) -
// fp16(hi*sin_lo)), hi' = fp16(fp16(hi*cos_hi) + fp16(lo*sin_hi)).
__device__ __forceinline__ void rope1(float lo, float hi, float cl, float sl, float ch, float sh,
                                      f16& out_lo, f16& out_hi) {
#pragma clang fp contract(off)
  const float a = round16(lo * cl);
  const float b = round16(hi * sl);
  const float c = round16(hi * ch);
  const float d = round16(lo * sh);
  out_lo = (f16)(a - b);
  out_hi = (f16)(c + d);
}

// ---------------------------------------------------------------------------
struct QkvArgs {
  const f16* x;
  int64_t x_sb;
  const int64_t* token;
  f16* hidden_out;
  int64_t ho_sb;
  const f16* norm_w;
  float eps;
  const f16* w;
  const f16* bias;
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
  int K, QH, KVH, cap, n_pairs;
};

// One wave per (head, d) rotate-half pair: rows head*64 + d and head*64 + d + 32.
template <int NB>
__global__ __launch_bounds__(kNT) void rms_qkv_rope_append_kernel(QkvArgs a) {
  constexpr int NS = kMaxNormK / 8 / 64;  // 2
  __shared__ __attribute__((aligned(16))) f16 xs[NB * kMaxNormK];
  __shared__ float red[kNW * NB];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int K = a.K, C = K / 8;
  const int p = blockIdx.x * kNW + w;
  const bool valid = p < a.n_pairs;
  const int head = p / (kHeadDim / 2), dd = p % (kHeadDim / 2);
  const int r0 = head * kHeadDim + dd, r1 = r0 + kHeadDim / 2;

  f16x8 w0[NS], w1[NS];
  if (valid) {
    load_row<NS>(a.w + (int64_t)r0 * K, C, w0, lane);
    load_row<NS>(a.w + (int64_t)r1 * K, C, w1, lane);
  }
  const f16* rows[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
    rows[b] = a.x + (a.token != nullptr ? a.token[b] : (int64_t)b) * a.x_sb;
  f16* raw = (a.token != nullptr && blockIdx.x == 0) ? a.hidden_out : nullptr;
  stage_rms<NB>(rows, K, a.norm_w, a.eps, xs, red, raw, a.ho_sb);
  if (!valid) return;

  float s0[NB], s1[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) s0[b] = s1[b] = 0.f;
  dot_row<NS, NB>(w0, xs, K, C, s0, lane);
  dot_row<NS, NB>(w1, xs, K, C, s1, lane);
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    s0[b] = wave_sum(s0[b]);
    s1[b] = wave_sum(s1[b]);
  }
  if (lane >= NB) return;
  // Lane b finishes batch row b.
  const int b = lane;
  float v0 = s0[0], v1 = s1[0];
#pragma unroll
  for (int bb = 1; bb < NB; ++bb)
    if (b == bb) { v0 = s0[bb]; v1 = s1[bb]; }
  const float bias0 = a.bias != nullptr ? (float)a.bias[r0] : 0.f;
  const float bias1 = a.bias != nullptr ? (float)a.bias[r1] : 0.f;
  const float lo = (float)(f16)(v0 + bias0), hi = (float)(f16)(v1 + bias1);
  const int64_t slot = a.write_index[0];
  const bool in_range = slot >= 0 && slot < a.cap;
  if (head < a.QH + a.KVH) {
    const f16* cp = a.cos + b * a.cs_sb;
    const f16* sp = a.sin + b * a.cs_sb;
    f16 olo, ohi;
    rope1(lo, hi, (float)cp[dd], (float)sp[dd], (float)cp[dd + 32], (float)sp[dd + 32], olo, ohi);
    if (head < a.QH) {
      f16* q = a.q_out + b * a.qo_sb + head * a.qo_sh;
      q[dd] = olo;
      q[dd + 32] = ohi;
    } else if (in_range) {
      f16* k = a.kc + b * a.kc_sb + (head - a.QH) * a.kc_sh + slot * a.kc_sn;
      k[dd] = olo;
      k[dd + 32] = ohi;
    }
  } else if (in_range) {
    f16* v = a.vc + b * a.vc_sb + (head - a.QH - a.KVH) * a.vc_sh + slot * a.vc_sn;
    v[dd] = (f16)lo;
    v[dd + 32] = (f16)hi;
  }
}

// ---------------------------------------------------------------------------
struct GemvArgs {
  const f16* inp;
  int64_t in_sb;
  const f16* w;
  f16* hidden;
  int64_t h_sb;
  int K, N;
};

// Each wave owns RW consecutive rows; hidden[b][n] = fp16(hidden + fp16(acc)).
template <int NB, int NS, int RW>
__global__ __launch_bounds__(kNT) void gemv_residual_kernel(GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) f16 xs_dyn[];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int K = a.K, C = K / 8;
  const int n0 = (blockIdx.x * kNW + w) * RW;
  f16x8 wr[RW][NS];
#pragma unroll
  for (int r = 0; r < RW; ++r)
    if (n0 + r < a.N) load_row<NS>(a.w + (int64_t)(n0 + r) * K, C, wr[r], lane);
  stage_plain<NB>(a.inp, a.in_sb, K, xs_dyn);
  if (n0 >= a.N) return;
  float acc[RW][NB];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[r][b] = 0.f;
    if (n0 + r < a.N) dot_row<NS, NB>(wr[r], xs_dyn, K, C, acc[r], lane);
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[r][b] = wave_sum(acc[r][b]);
  }
  // Lane r*NB + b finishes (row n0 + r, batch row b).
  if (lane >= RW * NB) return;
  const int r = lane / NB, b = lane % NB;
  float v = acc[0][0];
#pragma unroll
  for (int rr = 0; rr < RW; ++rr)
#pragma unroll
    for (int bb = 0; bb < NB; ++bb)
      if (r == rr && b == bb) v = acc[rr][bb];
  const int n = n0 + r;
  if (n >= a.N) return;
  f16* h = a.hidden + b * a.h_sb + n;
  *h = (f16)((float)*h + (float)(f16)v);
}

// ---------------------------------------------------------------------------
struct GateUpArgs {
  const f16* x;
  int64_t x_sb;
  const f16* norm_w;
  float eps;
  const f16* w;
  f16* h;
  int64_t h_sb;
  int K, I;
};

// Each wave owns PW SwiGLU pairs (gate row j, up row I + j).
template <int NB, int PW>
__global__ __launch_bounds__(kNT) void rms_gate_up_swiglu_kernel(GateUpArgs a) {
  constexpr int NS = kMaxNormK / 8 / 64;
  __shared__ __attribute__((aligned(16))) f16 xs[NB * kMaxNormK];
  __shared__ float red[kNW * NB];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int K = a.K, C = K / 8;
  const int j0 = (blockIdx.x * kNW + w) * PW;
  f16x8 wg[PW][NS], wu[PW][NS];
#pragma unroll
  for (int pp = 0; pp < PW; ++pp) {
    if (j0 + pp < a.I) {
      load_row<NS>(a.w + (int64_t)(j0 + pp) * K, C, wg[pp], lane);
      load_row<NS>(a.w + (int64_t)(a.I + j0 + pp) * K, C, wu[pp], lane);
    }
  }
  const f16* rows[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) rows[b] = a.x + b * a.x_sb;
  stage_rms<NB>(rows, K, a.norm_w, a.eps, xs, red, nullptr, 0);
  if (j0 >= a.I) return;
  float ag[PW][NB], au[PW][NB];
#pragma unroll
  for (int pp = 0; pp < PW; ++pp) {
#pragma unroll
    for (int b = 0; b < NB; ++b) ag[pp][b] = au[pp][b] = 0.f;
    if (j0 + pp < a.I) {
      dot_row<NS, NB>(wg[pp], xs, K, C, ag[pp], lane);
      dot_row<NS, NB>(wu[pp], xs, K, C, au[pp], lane);
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      ag[pp][b] = wave_sum(ag[pp][b]);
      au[pp][b] = wave_sum(au[pp][b]);
    }
  }
  if (lane >= PW * NB) return;
  const int pp = lane / NB, b = lane % NB;
  float g = ag[0][0], u = au[0][0];
#pragma unroll
  for (int q = 0; q < PW; ++q)
#pragma unroll
    for (int bb = 0; bb < NB; ++bb)
      if (pp == q && b == bb) { g = ag[q][bb]; u = au[q][bb]; }
  const int j = j0 + pp;
  if (j >= a.I) return;
  // F.silu on the fp16 gate (fp32 math, one rounding), then the fp16 product.
  const float g16 = (float)(f16)g, u16 = (float)(f16)u;
  const float s16 = (float)(f16)(g16 / (1.f + expf(-g16)));
  a.h[b * a.h_sb + j] = (f16)(s16 * u16);
}

// ---------------------------------------------------------------------------
struct LmArgs {
  const f16* x;
  int64_t x_sb;
  const f16* norm_w;
  float eps;
  const f16* w;
  f16* logits;
  int64_t lg_sb;
  uint64_t* keys;
  int K, V;
};

// Orderable key of an fp16 logit at `index`: larger logit first, then the
// smaller index (torch.argmax returns the first maximum).
__device__ __forceinline__ uint64_t argmax_key(f16 v, int index) {
  const unsigned short bits = __builtin_bit_cast(unsigned short, v);
  const unsigned ord = (bits & 0x8000u) ? (~bits & 0xFFFFu) : (bits | 0x8000u);
  return ((uint64_t)ord << 32) | (uint64_t)(0xFFFFFFFFu - (unsigned)index);
}

// Grid-stride over groups of RW rows per wave, next group's loads in flight
// while the current one is reduced.
template <int NB>
__global__ __launch_bounds__(kNT) void rms_lm_head_kernel(LmArgs a) {
  constexpr int NS = kMaxNormK / 8 / 64;
  constexpr int RW = 4;
  __shared__ __attribute__((aligned(16))) f16 xs[NB * kMaxNormK];
  __shared__ float red[kNW * NB];
  __shared__ uint64_t wkeys[kNW][NB];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int K = a.K, C = K / 8;
  const int groups = (a.V + RW - 1) / RW;
  const int stride = gridDim.x * kNW;
  int g = blockIdx.x * kNW + w;

  f16x8 cur[RW][NS], nxt[RW][NS];
  auto load_group = [&](int grp, f16x8 (&buf)[RW][NS]) {
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int n = grp * RW + r;
      if (n < a.V) load_row<NS>(a.w + (int64_t)n * K, C, buf[r], lane);
      else {
#pragma unroll
        for (int s = 0; s < NS; ++s) buf[r][s] = zero8();
      }
    }
  };
  if (g < groups) load_group(g, cur);
  const f16* rows[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) rows[b] = a.x + b * a.x_sb;
  stage_rms<NB>(rows, K, a.norm_w, a.eps, xs, red, nullptr, 0);

  uint64_t best[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) best[b] = 0;
  for (; g < groups; g += stride) {
    if (g + stride < groups) load_group(g + stride, nxt);
    float acc[RW][NB];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[r][b] = 0.f;
      dot_row<NS, NB>(cur[r], xs, K, C, acc[r], lane);
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[r][b] = wave_sum(acc[r][b]);
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int n = g * RW + r;
      if (n < a.V) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const f16 lg = (f16)acc[r][b];
          const uint64_t key = argmax_key(lg, n);
          best[b] = key > best[b] ? key : best[b];
          if (lane == r * NB + b) a.logits[b * a.lg_sb + n] = lg;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int s = 0; s < NS; ++s) cur[r][s] = nxt[r][s];
  }
  if (lane == 0) {
#pragma unroll
    for (int b = 0; b < NB; ++b) wkeys[w][b] = best[b];
  }
  __syncthreads();
  if (threadIdx.x < NB) {
    const int b = threadIdx.x;
    uint64_t k = wkeys[0][b];
#pragma unroll
    for (int ww = 1; ww < kNW; ++ww) k = wkeys[ww][b] > k ? wkeys[ww][b] : k;
    a.keys[(int64_t)b * gridDim.x + blockIdx.x] = k;
  }
}

// ---------------------------------------------------------------------------
struct FinArgs {
  const uint64_t* keys;
  int n_blocks, B;
  int64_t* token;
  int64_t* rows;
  int64_t rows_sb;
  int n_rows;
  int64_t* step;
  int64_t* write_index;
  int64_t* pos;
};

__global__ __launch_bounds__(256) void argmax_step_kernel(FinArgs a) {
  __shared__ uint64_t part[256];
  __shared__ int64_t chosen[kMaxB];
  for (int b = 0; b < a.B; ++b) {
    uint64_t k = 0;
    for (int j = threadIdx.x; j < a.n_blocks; j += 256) {
      const uint64_t v = a.keys[(int64_t)b * a.n_blocks + j];
      k = v > k ? v : k;
    }
    part[threadIdx.x] = k;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
      if (threadIdx.x < o) {
        const uint64_t v = part[threadIdx.x + o];
        if (v > part[threadIdx.x]) part[threadIdx.x] = v;
      }
      __syncthreads();
    }
    if (threadIdx.x == 0) chosen[b] = (int64_t)(0xFFFFFFFFu - (unsigned)(part[0] & 0xFFFFFFFFu));
    __syncthreads();
  }
  if (threadIdx.x != 0) return;
  const int64_t s = a.step != nullptr ? a.step[0] : 0;
  for (int b = 0; b < a.B; ++b) {
    a.token[b] = chosen[b];
    if (a.rows != nullptr && a.step != nullptr && s >= 0 && s < a.n_rows)
      a.rows[b * a.rows_sb + s] = chosen[b];
    if (a.pos != nullptr) a.pos[b] += 1;
  }
  if (a.write_index != nullptr) a.write_index[0] += 1;
  if (a.step != nullptr) a.step[0] = s + 1;
}

}  // namespace step
}  // namespace qf

using namespace qf;
using namespace qf::step;

static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Launches KERNEL<B, ...> for B in 1..4 (grid, block, shm, st, a in scope).
#define QF_DISPATCH_B(B, KERNEL, ...)                                                      \
  switch (B) {                                                                             \
    case 1: hipLaunchKernelGGL((KERNEL<1, ##__VA_ARGS__>), grid, block, shm, st, a); break; \
    case 2: hipLaunchKernelGGL((KERNEL<2, ##__VA_ARGS__>), grid, block, shm, st, a); break; \
    case 3: hipLaunchKernelGGL((KERNEL<3, ##__VA_ARGS__>), grid, block, shm, st, a); break; \
    default: hipLaunchKernelGGL((KERNEL<4, ##__VA_ARGS__>), grid, block, shm, st, a); break; \
  }

extern "C" int qf_rms_qkv_rope_append(const void* x, int64_t x_sb, const int64_t* token,
                                      void* hidden_out, int64_t ho_sb,
                                      const void* norm_w, float eps,
                                      const void* w_qkv, const void* bias,
                                      const void* cos, const void* sin, int64_t cs_sb,
                                      void* k_cache, int64_t kc_sb, int64_t kc_sh, int64_t kc_sn,
                                      void* v_cache, int64_t vc_sb, int64_t vc_sh, int64_t vc_sn,
                                      const int64_t* write_index,
                                      void* q_out, int64_t qo_sb, int64_t qo_sh,
                                      int B, int hidden, int QH, int KVH, int D, int cap,
                                      void* stream) {
  if (D != kHeadDim) return QF_ERR_UNSUPPORTED;
  if (B < 1 || B > kMaxB || hidden < 8 || hidden > kMaxNormK || hidden % 8) return QF_ERR_UNSUPPORTED;
  if (!x || !norm_w || !w_qkv || !cos || !sin || !k_cache || !v_cache || !write_index || !q_out)
    return QF_ERR_INVALID_ARG;
  if (QH < 1 || KVH < 1 || cap < 1) return QF_ERR_INVALID_ARG;
  if (token != nullptr && hidden_out != nullptr && (!al16(hidden_out) || (ho_sb & 7)))
    return QF_ERR_INVALID_ARG;
  if (!al16(x) || !al16(norm_w) || !al16(w_qkv) || (x_sb & 7)) return QF_ERR_INVALID_ARG;
  QkvArgs a;
  a.x = static_cast<const f16*>(x); a.x_sb = x_sb; a.token = token;
  a.hidden_out = static_cast<f16*>(hidden_out); a.ho_sb = ho_sb;
  a.norm_w = static_cast<const f16*>(norm_w); a.eps = eps;
  a.w = static_cast<const f16*>(w_qkv); a.bias = static_cast<const f16*>(bias);
  a.cos = static_cast<const f16*>(cos); a.sin = static_cast<const f16*>(sin); a.cs_sb = cs_sb;
  a.kc = static_cast<f16*>(k_cache); a.kc_sb = kc_sb; a.kc_sh = kc_sh; a.kc_sn = kc_sn;
  a.vc = static_cast<f16*>(v_cache); a.vc_sb = vc_sb; a.vc_sh = vc_sh; a.vc_sn = vc_sn;
  a.write_index = write_index;
  a.q_out = static_cast<f16*>(q_out); a.qo_sb = qo_sb; a.qo_sh = qo_sh;
  a.K = hidden; a.QH = QH; a.KVH = KVH; a.cap = cap;
  a.n_pairs = (QH + 2 * KVH) * (kHeadDim / 2);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((a.n_pairs + kNW - 1) / kNW), block(kNT);
  const size_t shm = 0;
  QF_DISPATCH_B(B, rms_qkv_rope_append_kernel)
  return (int)hipGetLastError();
}

extern "C" int qf_gemv_residual(const void* inp, int64_t in_sb, const void* w, void* hidden,
                                int64_t h_sb, int B, int K, int N, void* stream) {
  if (B < 1 || B > kMaxB || K < 8 || K > kMaxK || K % 8) return QF_ERR_UNSUPPORTED;
  if (!inp || !w || !hidden || N < 1) return QF_ERR_INVALID_ARG;
  if (!al16(inp) || !al16(w) || (in_sb & 7)) return QF_ERR_INVALID_ARG;
  GemvArgs a;
  a.inp = static_cast<const f16*>(inp); a.in_sb = in_sb;
  a.w = static_cast<const f16*>(w);
  a.hidden = static_cast<f16*>(hidden); a.h_sb = h_sb;
  a.K = K; a.N = N;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t shm = (size_t)B * K * sizeof(f16);
  const dim3 block(kNT);
  const int C = K / 8;
  if (C <= 128) {
    // Short rows (o_proj): two rows per wave.
    const dim3 grid((N + kNW * 2 - 1) / (kNW * 2));
    QF_DISPATCH_B(B, gemv_residual_kernel, 2, 2)
  } else {
    // Long rows (down_proj): one row per wave, the whole row in flight.
    const dim3 grid((N + kNW - 1) / kNW);
    QF_DISPATCH_B(B, gemv_residual_kernel, 16, 1)
  }
  return (int)hipGetLastError();
}

extern "C" int qf_rms_gate_up_swiglu(const void* x, int64_t x_sb, const void* norm_w, float eps,
                                     const void* w_gate_up, void* h_out, int64_t ho_sb,
                                     int B, int hidden, int I, void* stream) {
  if (B < 1 || B > kMaxB || hidden < 8 || hidden > kMaxNormK || hidden % 8) return QF_ERR_UNSUPPORTED;
  if (!x || !norm_w || !w_gate_up || !h_out || I < 1) return QF_ERR_INVALID_ARG;
  if (!al16(x) || !al16(norm_w) || !al16(w_gate_up) || (x_sb & 7)) return QF_ERR_INVALID_ARG;
  GateUpArgs a;
  a.x = static_cast<const f16*>(x); a.x_sb = x_sb;
  a.norm_w = static_cast<const f16*>(norm_w); a.eps = eps;
  a.w = static_cast<const f16*>(w_gate_up);
  a.h = static_cast<f16*>(h_out); a.h_sb = ho_sb;
  a.K = hidden; a.I = I;
  hipStream_t st = static_cast<hipStream_t>(stream);
  constexpr int PW = 2;
  const dim3 grid((I + kNW * PW - 1) / (kNW * PW)), block(kNT);
  const size_t shm = 0;
  QF_DISPATCH_B(B, rms_gate_up_swiglu_kernel, PW)
  return (int)hipGetLastError();
}

extern "C" int qf_rms_lm_head(const void* x, int64_t x_sb, const void* norm_w, float eps,
                              const void* w_lm, void* logits, int64_t lg_sb, uint64_t* keys,
                              int n_blocks, int B, int hidden, int V, void* stream) {
  if (B < 1 || B > kMaxB || hidden < 8 || hidden > kMaxNormK || hidden % 8) return QF_ERR_UNSUPPORTED;
  if (!x || !norm_w || !w_lm || !logits || !keys || V < 1) return QF_ERR_INVALID_ARG;
  if (n_blocks < 1 || n_blocks > 65535) return QF_ERR_INVALID_ARG;
  if (!al16(x) || !al16(norm_w) || !al16(w_lm) || (x_sb & 7)) return QF_ERR_INVALID_ARG;
  LmArgs a;
  a.x = static_cast<const f16*>(x); a.x_sb = x_sb;
  a.norm_w = static_cast<const f16*>(norm_w); a.eps = eps;
  a.w = static_cast<const f16*>(w_lm);
  a.logits = static_cast<f16*>(logits); a.lg_sb = lg_sb;
  a.keys = keys;
  a.K = hidden; a.V = V;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(n_blocks), block(kNT);
  const size_t shm = 0;
  QF_DISPATCH_B(B, rms_lm_head_kernel)
  return (int)hipGetLastError();
}

extern "C" int qf_argmax_step(const uint64_t* keys, int n_blocks, int B, int64_t* token,
                              int64_t* rows, int64_t rows_sb, int n_rows, int64_t* step,
                              int64_t* write_index, int64_t* pos, void* stream) {
  if (B < 1 || B > kMaxB) return QF_ERR_UNSUPPORTED;
  if (!keys || !token || n_blocks < 1) return QF_ERR_INVALID_ARG;
  if (rows != nullptr && step == nullptr) return QF_ERR_INVALID_ARG;
  FinArgs a;
  a.keys = keys; a.n_blocks = n_blocks; a.B = B;
  a.token = token; a.rows = rows; a.rows_sb = rows_sb; a.n_rows = n_rows;
  a.step = step; a.write_index = write_index; a.pos = pos;
  hipLaunchKernelGGL(argmax_step_kernel, dim3(1), dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return (int)hipGetLastError();
}
