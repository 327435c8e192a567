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
// The down projection departs from this shape: its rows are long (K = 4864),
// so each row is split between the two waves of its own workgroup, and each
// lane loads the activation chunks it needs straight into registers.
//
// Replaces the torch op sequence of _decode_step_static
// (student_engine.py:896-982); see include/qf_step.h for the per-entry-point
// mapping and rounding.
#include "qf_common.h"
#include "../../include/qf_step.h"
#include "../../include/qf_paged.h"

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

// Sum over the 64 lanes with DPP moves (no LDS traffic): butterflies inside
// each 16-lane row, then row broadcasts leave the total in lane 63, which is
// read back as a wave-uniform value.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ float dpp_add(float v) {
  const int moved = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, kRowMask, 0xF,
                                                false);
  return v + __builtin_bit_cast(float, moved);
}

__device__ __forceinline__ float wave_sum(float v) {
  v = dpp_add<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]: quad sums
  v = dpp_add<0x141, 0xF>(v);  // row_half_mirror: 8-lane sums
  v = dpp_add<0x140, 0xF>(v);  // row_mirror: 16-lane row sums
  v = dpp_add<0x142, 0xA>(v);  // row_bcast:15 into rows 1, 3
  v = dpp_add<0x143, 0xC>(v);  // row_bcast:31 into rows 2, 3: lane 63 holds the total
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ f16x8 zero8() {
  f16x8 z;
#pragma unroll
  for (int e = 0; e < 8; ++e) z[e] = (f16)0.f;
  return z;
}

// The NS 16-byte chunks of one weight row that lane `lane` multiplies:
// chunk 64*s + lane, s < NS.  Lanes past the row's C chunks load its last
// chunk (never used), so no load sits behind a branch and every load of a
// wave is in flight at once.  A step reads each weight once, so the loads
// are non-temporal (with the tile loads below, config 5 0.578 -> 0.526 ms
// per step at B=1 and 0.726 -> 0.670 at B=4).
template <int NS>
__device__ __forceinline__ void load_row(const f16* __restrict__ w, int C, f16x8 (&r)[NS],
                                         int lane) {
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int c = min(64 * s + lane, C - 1);
    r[s] = load16_nt(w + 8 * c);
  }
}

// acc[b] += partial dot of the lane's chunks of a row with staged row b.
template <int NS, int NB>
__device__ __forceinline__ void dot_row(const f16x8 (&r)[NS], const f16* xs, int K, int C,
                                        float (&acc)[NB], int lane) {
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int c0 = 64 * s + lane;
    const bool in = c0 < C;
    const int c = in ? c0 : C - 1;
    const f16x8 wv = in ? r[s] : zero8();
#pragma unroll
    for (int b = 0; b < NB; ++b)
      acc[b] = dot8(wv, *reinterpret_cast<const f16x8*>(xs + b * K + 8 * c), acc[b]);
  }
}

// RMS-normalised staging of NB activation rows into LDS xs[b * K ..], as
// torch's fused RMSNorm kernel computes it for fp16 (fp32 math, one rounding):
//   y = fp16((x * rsqrt(mean(x^2) + eps)) * w)     (student_engine.py:530-535 form)
// Split in two so the caller can issue its weight loads in between: the
// activation loads go first and are waited for alone.  K <= kMaxNormK, so
// thread t < C owns chunk t of every row.
template <int NB>
struct RmsStage {
  f16x8 x[NB];
  f16x8 g;
};

template <int NB>
__device__ __forceinline__ void rms_load(RmsStage<NB>& st, const f16* const (&rows)[NB], int K,
                                         const f16* __restrict__ nw) {
  const int c = min((int)threadIdx.x, K / 8 - 1);
  st.g = load16(nw + 8 * c);
#pragma unroll
  for (int b = 0; b < NB; ++b) st.x[b] = load16(rows[b] + 8 * c);
}

template <int NB>
__device__ __forceinline__ void rms_finish(const RmsStage<NB>& st, int K, float eps, f16* xs,
                                           float* red, f16* raw_out, int64_t raw_sb) {
  const int C = K / 8;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const bool own = tid < C;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += (float)st.x[b][e] * (float)st.x[b][e];
    s = wave_sum(own ? s : 0.f);
    if (lane == 0) red[w * NB + b] = s;
  }
  if (raw_out != nullptr && own) {
#pragma unroll
    for (int b = 0; b < NB; ++b) store16(raw_out + b * raw_sb + 8 * tid, st.x[b]);
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
      for (int e = 0; e < 8; ++e) y[e] = (f16)(((float)st.x[b][e] * rstd) * (float)st.g[e]);
      store16(xs + b * K + 8 * tid, y);
    }
  }
  __syncthreads();
}

// Plain staging of NB rows (row stride sb, K = 8C) into LDS, likewise split:
// thread t holds chunks t + kNT*i of the flattened (NB x C) chunk grid.
template <int XP>
__device__ __forceinline__ void plain_load(f16x8 (&v)[XP], const f16* __restrict__ x, int64_t sb,
                                           int C, int NB) {
  const int total = NB * C;
#pragma unroll
  for (int i = 0; i < XP; ++i) {
    const int idx = min((int)threadIdx.x + kNT * i, total - 1);
    const int b = idx / C, c = idx - b * C;
    v[i] = load16(x + b * sb + 8 * c);
  }
}

template <int XP>
__device__ __forceinline__ void plain_finish(const f16x8 (&v)[XP], int C, int NB, f16* xs) {
  const int total = NB * C;
#pragma unroll
  for (int i = 0; i < XP; ++i) {
    const int idx = threadIdx.x + kNT * i;
    if (idx < total) store16(xs + 8 * idx, v[i]);  // xs[b][c] at 8 * (b * C + c)
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
  // Positions mode (cos == nullptr): row b's angle for frequency i is
  // float(pos[b]) * inv_freq[i], and cos/sin are evaluated here in fp32 and
  // rounded to fp16 -- bit-identical to the torch table (SE:910-915) that
  // table mode reads.
  const int64_t* pos;
  const float* inv_freq;
  f16* kc;
  int64_t kc_sb, kc_sh, kc_sn;
  f16* vc;
  int64_t vc_sb, vc_sh, vc_sn;
  const int64_t* write_index;
  f16* q_out;
  int64_t qo_sb, qo_sh;
  int K, QH, KVH, cap, n_pairs;
  // Paged caches: kc/vc are page pools (page strides kc_sb/vc_sb); row b
  // appends at logical slot slots[b * slot_sb], in page
  // table[b * t_sb + (slot >> log2p)].  cap = pages per row << log2p.
  const int32_t* table;
  int64_t t_sb;
  int log2p, n_pages;
  const int64_t* slots;
  int64_t slot_sb;
};
static_assert(covers_lines(sizeof(QkvArgs), {offsetof(QkvArgs, x), offsetof(QkvArgs, bias),
                                             offsetof(QkvArgs, write_index), offsetof(QkvArgs, K),
                                             offsetof(QkvArgs, slots)}),
              "touch_arg_lines fields cover every line");

// One wave per (head, d) rotate-half pair: rows head*64 + d and head*64 + d + 32.
template <int NB, bool kPaged, bool kPos>
__global__ __launch_bounds__(kNT) void rms_qkv_rope_append_kernel(QkvArgs a) {
  constexpr int NS = kMaxNormK / 8 / 64;  // 2
  __shared__ __attribute__((aligned(16))) f16 xs[NB * kMaxNormK];
  __shared__ float red[kNW * NB];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int K = touch_arg_lines(a.K, a.x, a.bias, a.write_index, a.slots), C = K / 8;
  const int p_raw = blockIdx.x * kNW + w;
  const bool valid = p_raw < a.n_pairs;
  const int p = valid ? p_raw : a.n_pairs - 1;  // spare waves load a real pair, store nothing
  const int head = p / (kHeadDim / 2), dd = p % (kHeadDim / 2);
  const int r0 = head * kHeadDim + dd, r1 = r0 + kHeadDim / 2;

  const f16* rows[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
    rows[b] = a.x + (a.token != nullptr ? a.token[b] : (int64_t)b) * a.x_sb;
  RmsStage<NB> st;
  rms_load<NB>(st, rows, K, a.norm_w);
  // Epilogue operands, loaded now so their latency hides under the weights':
  // lane b < NB finishes batch row b.
  const int be = lane < NB ? lane : 0;
  const int64_t slot = kPaged ? a.slots[be * a.slot_sb] : a.write_index[0];
  // Branch-free bias: without one, a weight element is read and dropped (a
  // guarded load would wait for completion before the weights go out).
  const bool has_bias = a.bias != nullptr;
  const f16* bsrc = has_bias ? a.bias : a.w;
  const float braw0 = (float)bsrc[r0], braw1 = (float)bsrc[r1];
  const float bias0 = has_bias ? braw0 : 0.f;
  const float bias1 = has_bias ? braw1 : 0.f;
  float cos_lo, sin_lo, cos_hi, sin_hi;
  float ang = 0.f;
  if (kPos) {
    // Both halves of a rotate-half pair share frequency dd (emb = cat(f, f)).
    ang = (float)a.pos[be] * a.inv_freq[dd];
  } else {
    const f16* cp = a.cos + be * a.cs_sb;
    const f16* sp = a.sin + be * a.cs_sb;
    cos_lo = (float)cp[dd];
    sin_lo = (float)sp[dd];
    cos_hi = (float)cp[dd + 32];
    sin_hi = (float)sp[dd + 32];
  }
  f16x8 w0[NS], w1[NS];
  load_row<NS>(a.w + (int64_t)r0 * K, C, w0, lane);
  load_row<NS>(a.w + (int64_t)r1 * K, C, w1, lane);
  // Element offsets of the destination slot (kv head 0); the page lookup
  // (paged caches) depends on the slot, so it is issued after the weights.
  bool in_range = slot >= 0 && slot < a.cap;
  int64_t kro, vro;
  if (kPaged) {
    const int64_t sl = in_range ? slot : 0;  // branch-free table read
    const int page = a.table[be * a.t_sb + (sl >> a.log2p)];
    in_range = in_range && page >= 0 && page < a.n_pages;
    const int64_t row = sl & ((1 << a.log2p) - 1);
    kro = (int64_t)page * a.kc_sb + row * a.kc_sn;
    vro = (int64_t)page * a.vc_sb + row * a.vc_sn;
  } else {
    kro = be * a.kc_sb + slot * a.kc_sn;
    vro = be * a.vc_sb + slot * a.vc_sn;
  }
  if (kPos) {
    // Evaluated while the weight rows are in flight (the angle's loads were
    // issued before them).
    cos_lo = cos_hi = (float)(f16)cosf(ang);
    sin_lo = sin_hi = (float)(f16)sinf(ang);
  }
  f16* raw = (a.token != nullptr && blockIdx.x == 0) ? a.hidden_out : nullptr;
  rms_finish<NB>(st, K, a.eps, xs, red, raw, a.ho_sb);
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
  const float lo = (float)(f16)(v0 + bias0), hi = (float)(f16)(v1 + bias1);
  if (head < a.QH + a.KVH) {
    f16 olo, ohi;
    rope1(lo, hi, cos_lo, sin_lo, cos_hi, sin_hi, olo, ohi);
    if (head < a.QH) {
      f16* q = a.q_out + b * a.qo_sb + head * a.qo_sh;
      q[dd] = olo;
      q[dd + 32] = ohi;
    } else if (in_range) {
      f16* k = a.kc + kro + (head - a.QH) * a.kc_sh;
      k[dd] = olo;
      k[dd + 32] = ohi;
    }
  } else if (in_range) {
    f16* v = a.vc + vro + (head - a.QH - a.KVH) * a.vc_sh;
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
template <int NB, int NS, int RW, int XP>
__global__ __launch_bounds__(kNT) void gemv_residual_kernel(GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) f16 xs_dyn[];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int K = a.K, C = K / 8;
  const int n0 = (blockIdx.x * kNW + w) * RW;
  // Lane r*NB + b finishes (row n0 + r, batch row b).
  const int re = lane < RW * NB ? lane / NB : 0, be = lane < RW * NB ? lane % NB : 0;
  f16* hp = a.hidden + be * a.h_sb + min(n0 + re, a.N - 1);
  f16x8 xv[XP];
  plain_load<XP>(xv, a.inp, a.in_sb, C, NB);
  f16x8 wr[RW][NS];
#pragma unroll
  for (int r = 0; r < RW; ++r) load_row<NS>(a.w + (int64_t)min(n0 + r, a.N - 1) * K, C, wr[r], lane);
  // Last, as in the long-row kernel: loads retire in issue order.
  const float resid = (float)*hp;
  plain_finish<XP>(xv, C, NB, xs_dyn);
  if (n0 >= a.N) return;
  float acc[RW][NB];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[r][b] = 0.f;
    dot_row<NS, NB>(wr[r], xs_dyn, K, C, acc[r], lane);
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
  if (n0 + r >= a.N) return;
  *hp = (f16)(resid + (float)(f16)v);
}

// Long rows (down_proj): RPW rows per workgroup, each split between KP waves
// (contiguous parts of ceil(C / KP) chunks, whose sums meet in LDS and are
// added in part order).  Nothing is staged: each lane loads the activation
// chunks it multiplies straight into registers (L2 hits, issued right after
// its weight loads), so no barrier stands between the loads and the dot
// products.  Measured on MI355X at K = 4864, N = 896, weights past the MALL,
// against one row per wave of a four-wave workgroup with the activation
// staged through LDS: KP = 2, RPW = 1 takes B=1 3.81-3.86 vs 4.35 us, B=2
// 4.32 vs 4.81, B=4 5.02-5.11 vs 5.42 (RPW = 4 with the activation staged:
// 4.03-4.09 / 4.45-4.51 / 5.46-5.51).  Rounding: fp16(residual + fp16(acc)).
template <int NB, int NS, int KP, int RPW>
__global__ __launch_bounds__(KP * RPW * 64) void gemv_residual_direct_kernel(GemvArgs a) {
  __shared__ float red[KP][RPW][NB];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int rw = w % RPW, part = w / RPW;
  const int K = a.K, C = K / 8, Cp = (C + KP - 1) / KP;
  const int c0 = part * Cp, c1 = min(c0 + Cp, C);
  const int n0 = blockIdx.x * RPW + rw;
  const int nr = min(n0, a.N - 1);
  const int be = lane < NB ? lane : 0;
  f16* hp = a.hidden + be * a.h_sb + nr;
  const f16* wrow = a.w + (int64_t)nr * K;
  f16x8 wr[NS], xr[NB][NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) wr[s] = load16_nt(wrow + 8 * min(c0 + 64 * s + lane, c1 - 1));
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int c = min(c0 + 64 * s + lane, c1 - 1);
#pragma unroll
    for (int b = 0; b < NB; ++b) xr[b][s] = load16(a.inp + b * a.in_sb + 8 * c);
  }
  // The residual goes out last.  Vector loads retire in issue order, so a
  // slow residual load ahead of the weights would hold up every weight and
  // activation load behind it.  Measured on MI355X, outputs bit-identical:
  // calls in a row on weights past the MALL, each reading rows the previous
  // call had just written, B=1 3.77 -> 3.65 us, B=2 4.26 -> 3.99, B=3 4.68
  // -> 4.36, B=4 5.07 -> 4.76; inside the decode step, where the gate/up
  // launch has just read those rows into L2, no change.
  const float resid = (float)*hp;
  float acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = 0.f;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const bool in = c0 + 64 * s + lane < c1;
    const f16x8 wv = in ? wr[s] : zero8();
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = dot8(wv, xr[b][s], acc[b]);
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = wave_sum(acc[b]);
  if (KP > 1) {
    if (lane == 0) {
#pragma unroll
      for (int b = 0; b < NB; ++b) red[part][rw][b] = acc[b];
    }
    __syncthreads();
  }
  if (part != 0 || n0 >= a.N || lane >= NB) return;
  float v = 0.f;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (lane == b) {
      v = acc[b];
#pragma unroll
      for (int p = 1; p < KP; ++p) v += red[p][rw][b];
    }
  }
  *hp = (f16)(resid + (float)(f16)v);
}

// ---------------------------------------------------------------------------
// o_proj with the split-K attention merge as its staging prologue.  Every
// workgroup merges the decode kernel's partials (acc, m, l in the reference's
// scratch layout, student_engine.py:117-162 algebra) for all B x KVH x G
// query heads itself -- a few tens of KB of L2-resident reads -- instead of a
// separate combine launch writing the fp16 attention output first.  The
// merged row is rounded to fp16 exactly as the combine kernel rounds it
// (out = fp16(A * (1 / L))), then hidden += fp16(att @ w_o^T).
struct MergeArgs {
  const float* acc;
  const float* m;
  const float* l;
  int splits, KVH, G;
  const f16* w;
  f16* hidden;
  int64_t h_sb;
  int K, N;
};
static_assert(covers_lines(sizeof(MergeArgs), {offsetof(MergeArgs, acc), offsetof(MergeArgs, K)}),
              "touch_arg_lines fields cover every line");

// The merge prologue shared by the o_proj kernels: every workgroup folds
// all B x KVH x G x 64 merged attention values into LDS xs (fp16, the
// combine's rounding).  `issue` runs right after the first batch of partial
// loads goes out and issues the caller's weight (and residual) loads, so the
// L2-resident partials land first and the merge runs while the weights are in
// flight.  Ends with a workgroup barrier.
template <int NB, typename Issue>
__device__ __forceinline__ void merge_partials(const MergeArgs& a, f16* xs, Issue&& issue) {
  // Splits folded per batch: the engine's split counts (8 at one row, 4 at
  // more) in one batch, so the merge is one round trip.
  constexpr int kSB = NB == 1 ? 8 : 4;
  // Item = (b, h, g, 4 dims); xs offset of item `it` is 4 * it because
  // hidden index (h * G + g) * 64 + d matches the (B, KVH, G, D) output layout.
  // Thread t owns items t + kNT*i (i < NB covers NB * KVH * G * 16 <= NB * kNT
  // items); each batch loads kSB splits of every owned item at once.
  const int S = a.splits, G = a.G;
  const int items = NB * a.KVH * G * 16;
  float M[NB], L[NB];
  f32x4 A[NB];
  int64_t ml0[NB], acc0[NB];  // split-0 index into m/l, and into acc as f32x4 slots
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int it = min((int)threadIdx.x + kNT * i, items - 1);
    const int d4 = it & 15, bhg = it >> 4;
    const int g = bhg % G, bh = bhg / G;
    ml0[i] = (int64_t)bh * S * G + g;  // split s adds s * G
    acc0[i] = ml0[i] * 16 + d4;        // split s adds s * G * 16
    M[i] = kNegInf;
    L[i] = 0.f;
    A[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  float mv[NB][kSB], lv[NB][kSB];
  f32x4 av[NB][kSB];
  const auto load_batch = [&](int s0) {
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int u = 0; u < kSB; ++u) {
        const int64_t off = (int64_t)min(s0 + u, S - 1) * G;
        mv[i][u] = a.m[ml0[i] + off];
        lv[i][u] = a.l[ml0[i] + off];
        av[i][u] = reinterpret_cast<const f32x4*>(a.acc)[acc0[i] + off * 16];
      }
  };
  const auto fold_batch = [&](int s0) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      float mc = M[i];
#pragma unroll
      for (int u = 0; u < kSB; ++u)
        if (s0 + u < S) mc = fmaxf(mc, mv[i][u]);
      const float safe = (mc == kNegInf) ? 0.f : mc;
      const float r = (M[i] == kNegInf) ? 0.f : fast_exp2((M[i] - safe) * kLog2e);
      L[i] *= r;
      A[i] *= r;
#pragma unroll
      for (int u = 0; u < kSB; ++u) {
        const float wt = (s0 + u >= S || mv[i][u] == kNegInf) ? 0.f
                                                               : fast_exp2((mv[i][u] - safe) * kLog2e);
        L[i] += wt * lv[i][u];
        A[i] += wt * av[i][u];
      }
      M[i] = mc;
    }
  };
  // The first batch of partials goes out before the weight rows: the partials
  // are L2-resident and land first, so the merge runs while the weights are
  // in flight (a wait for loads issued after the weights would wait for the
  // weights too).
  load_batch(0);
  issue();
  // Keep the loads above in flight together (left alone, the scheduler sinks
  // them next to their uses).
  __builtin_amdgcn_sched_barrier(0);
  fold_batch(0);
  for (int s0 = kSB; s0 < S; s0 += kSB) {
    load_batch(s0);
    fold_batch(s0);
  }
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int it = threadIdx.x + kNT * i;
    if (it < items) {
      const float inv = 1.f / L[i];
      f16x4 o;
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] = (f16)(A[i][c] * inv);
      *reinterpret_cast<f16x4*>(xs + 4 * it) = o;
    }
  }
  __syncthreads();
}

template <int NB, int RW>
__global__ __launch_bounds__(kNT) void attn_merge_gemv_residual_kernel(MergeArgs a) {
  constexpr int NS = kMaxNormK / 8 / 64;
  __shared__ __attribute__((aligned(16))) f16 xs[NB * kMaxNormK];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int K = touch_arg_lines(a.K, a.acc), C = K / 8;
  const int n0 = (blockIdx.x * kNW + w) * RW;
  f16x8 wr[RW][NS];
  const int re = lane < RW * NB ? lane / NB : 0, be = lane < RW * NB ? lane % NB : 0;
  f16* hp = a.hidden + be * a.h_sb + min(n0 + re, a.N - 1);
  float resid;
  merge_partials<NB>(a, xs, [&] {
#pragma unroll
    for (int r = 0; r < RW; ++r) load_row<NS>(a.w + (int64_t)min(n0 + r, a.N - 1) * K, C, wr[r], lane);
    resid = (float)*hp;
  });
  if (n0 >= a.N) return;
  float acc[RW][NB];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[r][b] = 0.f;
    dot_row<NS, NB>(wr[r], xs, K, C, acc[r], lane);
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[r][b] = wave_sum(acc[r][b]);
  }
  if (lane >= RW * NB) return;
  const int r = lane / NB, b = lane % NB;
  float v = acc[0][0];
#pragma unroll
  for (int rr = 0; rr < RW; ++rr)
#pragma unroll
    for (int bb = 0; bb < NB; ++bb)
      if (r == rr && b == bb) v = acc[rr][bb];
  if (n0 + r >= a.N) return;
  *hp = (f16)(resid + (float)(f16)v);
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
  const f16* rows[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) rows[b] = a.x + b * a.x_sb;
  RmsStage<NB> st;
  rms_load<NB>(st, rows, K, a.norm_w);
  f16x8 wg[PW][NS], wu[PW][NS];
#pragma unroll
  for (int pp = 0; pp < PW; ++pp) {
    const int j = min(j0 + pp, a.I - 1);
    load_row<NS>(a.w + (int64_t)j * K, C, wg[pp], lane);
    load_row<NS>(a.w + (int64_t)(a.I + j) * K, C, wu[pp], lane);
  }
  rms_finish<NB>(st, K, a.eps, xs, red, nullptr, 0);
  if (j0 >= a.I) return;
  float ag[PW][NB], au[PW][NB];
#pragma unroll
  for (int pp = 0; pp < PW; ++pp) {
#pragma unroll
    for (int b = 0; b < NB; ++b) ag[pp][b] = au[pp][b] = 0.f;
    dot_row<NS, NB>(wg[pp], xs, K, C, ag[pp], lane);
    dot_row<NS, NB>(wu[pp], xs, K, C, au[pp], lane);
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
// Matrix-core forms (weights packed by qf_pack_weight).  The NB batch rows
// are the columns of a v_mfma_f32_16x16x32_f16 (columns >= NB are zero) and
// 16 weight rows its A operand, so the k-reduction happens inside the matrix
// core: no cross-lane sums, and one 16-byte LDS activation read per lane per
// 32 k (the VALU form reads NB per weight row).  A packed tile (row block rb,
// k block kb) is the 1 KB A operand in lane order -- lane l's 16 bytes are
// row r = l % 16, k = 32 kb + 8 (l / 16) .. +7 -- so every weight load of a
// wave is one contiguous 1 KB read.  Tiles are stored rb-major.
__device__ __forceinline__ f16x8 tile_load(const f16* __restrict__ w, int nkb, int rb, int kb,
                                           int lane) {
  return load16_nt(w + (((int64_t)rb * nkb + kb) * 64 + lane) * 8);
}

// B operand of k block kb for lane l: staged activation row l % 16 at
// k = 32 kb + 8 (l / 16), zero for columns >= NB.
template <int NB>
__device__ __forceinline__ f16x8 act_operand(const f16* xs, int K, int kb, int lane) {
  const int col = lane & 15;
  const f16x8 v = *reinterpret_cast<const f16x8*>(xs + min(col, NB - 1) * K + 32 * kb +
                                                   8 * (lane >> 4));
  return col < NB ? v : zero8();
}

// The MFMA k blocks of one wave: blocks [kb0, kb0 + n) (n <= NBLK) of a
// row block, with the tile loads issued by the caller beforehand.
template <int NB, int NBLK>
__device__ __forceinline__ f32x4 tile_mfma(const f16x8 (&wa)[NBLK], const f16* xs, int K, int kb0,
                                           int n, int lane) {
  // Every B operand is read from LDS before the first MFMA, so the LDS
  // latency is paid once, not once per block.
  f16x8 xb[NBLK];
#pragma unroll
  for (int t = 0; t < NBLK; ++t) xb[t] = t < n ? act_operand<NB>(xs, K, kb0 + t, lane) : zero8();
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < NBLK; ++t) {
    if (t & 1) acc1 = mfma16x16x32(wa[t], xb[t], acc1);
    else acc0 = mfma16x16x32(wa[t], xb[t], acc0);
  }
  return acc0 + acc1;
}

// Gate/up + SwiGLU.  Packing QF_PACK_SWIGLU puts, in row block rb, MFMA
// row r = 4g + i on gate row 8 rb + 2g + (i & 1) for i < 2 and on the
// matching up row (+ I) for i >= 2, so C registers t (gate) and t + 2 (up)
// of lane l are one SwiGLU pair: lane l finishes outputs 8 rb + 2 (l >> 4)
// + {0, 1} of batch row l & 15.  KS waves split a row block's k range and
// add their partial tiles in LDS.
constexpr int kGuKS = 4;                             // k splits per row block
constexpr int kGuBlk = kMaxNormK / 32 / kGuKS;       // k blocks per wave (max)

template <int NB>
__global__ __launch_bounds__(kNT) void rms_gate_up_swiglu_mfma_kernel(GateUpArgs a) {
  __shared__ __attribute__((aligned(16))) f16 xs[NB * kMaxNormK];
  __shared__ float red[kNW * NB];
  __shared__ f32x4 part[kNW][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int K = a.K, nkb = K / 32;
  const int per = (nkb + kGuKS - 1) / kGuKS;
  const int kp = w % kGuKS;
  const int nrb = a.I / 8;
  const int rb = min((int)blockIdx.x * (kNW / kGuKS) + w / kGuKS, nrb - 1);
  const int kb0 = kp * per, n = min(per, nkb - kb0);
  const f16* rows[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) rows[b] = a.x + b * a.x_sb;
  RmsStage<NB> st;
  rms_load<NB>(st, rows, K, a.norm_w);
  f16x8 wa[kGuBlk];
#pragma unroll
  for (int t = 0; t < kGuBlk; ++t) wa[t] = tile_load(a.w, nkb, rb, min(kb0 + t, nkb - 1), lane);
  rms_finish<NB>(st, K, a.eps, xs, red, nullptr, 0);
  f32x4 acc = tile_mfma<NB, kGuBlk>(wa, xs, K, kb0, n, lane);
  if (kp != 0) part[w][lane] = acc;
  __syncthreads();
  if (kp != 0) return;
#pragma unroll
  for (int s = 1; s < kGuKS; ++s) acc += part[w + s][lane];
  const int col = lane & 15;
  const int jb = ((int)blockIdx.x * (kNW / kGuKS) + w / kGuKS) * 8 + 2 * (lane >> 4);
  if (col >= NB || jb >= a.I) return;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    // F.silu on the fp16 gate (fp32 math, one rounding), then the fp16 product.
    const float g16 = (float)(f16)acc[t], u16 = (float)(f16)acc[t + 2];
    const float s16 = (float)(f16)(g16 / (1.f + expf(-g16)));
    a.h[col * a.h_sb + jb + t] = (f16)(s16 * u16);
  }
}

// Merge + o_proj on matrix-core tiles (packed with QF_PACK_PLAIN), for 2-4
// rows: merge_partials, then one 16-row block per workgroup, its k range split
// between the four waves (kOpKS) whose partial tiles are added in LDS; the
// batch rows are the MFMA columns, so a wave spends one MFMA per 1 KB of
// weights where the row kernel spends four v_dot2 per batch row and 16
// bytes, plus a 64-lane butterfly per row and batch row.  Lane l finishes
// rows 16 rb + 4 (l / 16) + i of batch row l % 16: fp16(residual + fp16(acc)).
// Measured on MI355X at hidden 896 (8 splits at B=1, 4 above), weights past
// the MALL, row kernel / this one: B=1 2.79 / 3.07 us, B=2 3.31 / 3.14, B=3
// 3.90 / 3.48, B=4 4.50 / 3.93.
constexpr int kOpKS = 4;
constexpr int kOpBlk = kMaxNormK / 32 / kOpKS;

template <int NB>
__global__ __launch_bounds__(kNT) void attn_merge_o_proj_mfma_kernel(MergeArgs a) {
  static_assert(kNW / kOpKS == 1, "one row block per workgroup");
  __shared__ __attribute__((aligned(16))) f16 xs[NB * kMaxNormK];
  __shared__ f32x4 part[kNW][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int K = touch_arg_lines(a.K, a.acc), nkb = K / 32;
  const int per = (nkb + kOpKS - 1) / kOpKS;
  const int kp = w % kOpKS;
  const int rb = blockIdx.x;
  const int kb0 = kp * per, n = min(per, nkb - kb0);
  const int col = lane & 15, q = lane >> 4;
  f16* hp = a.hidden + min(col, NB - 1) * a.h_sb + 16 * rb + 4 * q;
  f16x8 wa[kOpBlk];
  f16x4 res;
  merge_partials<NB>(a, xs, [&] {
#pragma unroll
    for (int t = 0; t < kOpBlk; ++t) wa[t] = tile_load(a.w, nkb, rb, min(kb0 + t, nkb - 1), lane);
    res = *reinterpret_cast<const f16x4*>(hp);
  });
  f32x4 acc = tile_mfma<NB, kOpBlk>(wa, xs, K, kb0, n, lane);
  if (kp != 0) part[w][lane] = acc;
  __syncthreads();
  if (kp != 0 || col >= NB) return;
#pragma unroll
  for (int s = 1; s < kOpKS; ++s) acc += part[w + s][lane];
  f16x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = (f16)((float)res[i] + (float)(f16)acc[i]);
  *reinterpret_cast<f16x4*>(hp) = o;
}

// QKV + bias + RoPE + KV append.  Packing QF_PACK_ROPE makes row block
// rb = 4 head + c hold, in MFMA row r = 4g + i, row 64 head + d (i < 2) and
// row 64 head + d + 32 (i >= 2) with d = 8c + 2g + (i & 1): lane l's C
// registers t and t + 2 are the rotate-half pair of d = 8c + 2 (l >> 4) + t
// for batch row l & 15, so bias, RoPE and the append run in the lane.
constexpr int kQkvKS = 4;
constexpr int kQkvBlk = kMaxNormK / 32 / kQkvKS;

template <int NB, bool kPaged, bool kPos>
__global__ __launch_bounds__(kNT) void rms_qkv_rope_append_mfma_kernel(QkvArgs a) {
  __shared__ __attribute__((aligned(16))) f16 xs[NB * kMaxNormK];
  __shared__ float red[kNW * NB];
  __shared__ f32x4 part[kNW][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int K = touch_arg_lines(a.K, a.x, a.bias, a.write_index, a.slots), nkb = K / 32;
  const int per = (nkb + kQkvKS - 1) / kQkvKS;
  const int kp = w % kQkvKS;
  const int nrb = (a.QH + 2 * a.KVH) * 4;
  const int rb = min((int)blockIdx.x * (kNW / kQkvKS) + w / kQkvKS, nrb - 1);
  const int kb0 = kp * per, n = min(per, nkb - kb0);
  const f16* rows[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
    rows[b] = a.x + (a.token != nullptr ? a.token[b] : (int64_t)b) * a.x_sb;
  RmsStage<NB> st;
  rms_load<NB>(st, rows, K, a.norm_w);
  // Epilogue operands, loaded now so their latency hides under the weights'.
  const int col = lane & 15, q = lane >> 4;
  const int be = min(col, NB - 1);
  const int head = rb >> 2;
  const int d0 = 8 * (rb & 3) + 2 * q;  // this lane's pair dims d0, d0 + 1 (and + 32)
  const int64_t slot = kPaged ? a.slots[be * a.slot_sb] : a.write_index[0];
  // Branch-free bias: without one, a weight element is read and dropped.
  const bool has_bias = a.bias != nullptr;
  const f16* bsrc = (has_bias ? a.bias : a.w) + 64 * head + d0;
  float bias[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const float lo = (float)bsrc[t], hi = (float)bsrc[t + 32];
    bias[t][0] = has_bias ? lo : 0.f;
    bias[t][1] = has_bias ? hi : 0.f;
  }
  float cs[2][4];  // per dim: cos_lo, sin_lo, cos_hi, sin_hi
  float ang[2] = {0.f, 0.f};
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    if (kPos) {
      ang[t] = (float)a.pos[be] * a.inv_freq[d0 + t];
    } else {
      const f16* cp = a.cos + be * a.cs_sb + d0 + t;
      const f16* sp = a.sin + be * a.cs_sb + d0 + t;
      cs[t][0] = (float)cp[0];
      cs[t][1] = (float)sp[0];
      cs[t][2] = (float)cp[32];
      cs[t][3] = (float)sp[32];
    }
  }
  f16x8 wa[kQkvBlk];
#pragma unroll
  for (int t = 0; t < kQkvBlk; ++t) wa[t] = tile_load(a.w, nkb, rb, min(kb0 + t, nkb - 1), lane);
  // Destination slot offsets (kv head 0); the page lookup depends on the
  // slot, so it is issued after the weights.
  bool in_range = slot >= 0 && slot < a.cap;
  int64_t kro, vro;
  if (kPaged) {
    const int64_t sl = in_range ? slot : 0;
    const int page = a.table[be * a.t_sb + (sl >> a.log2p)];
    in_range = in_range && page >= 0 && page < a.n_pages;
    const int64_t prow = sl & ((1 << a.log2p) - 1);
    kro = (int64_t)page * a.kc_sb + prow * a.kc_sn;
    vro = (int64_t)page * a.vc_sb + prow * a.vc_sn;
  } else {
    kro = be * a.kc_sb + slot * a.kc_sn;
    vro = be * a.vc_sb + slot * a.vc_sn;
  }
  if (kPos) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      cs[t][0] = cs[t][2] = (float)(f16)cosf(ang[t]);
      cs[t][1] = cs[t][3] = (float)(f16)sinf(ang[t]);
    }
  }
  f16* raw = (a.token != nullptr && blockIdx.x == 0) ? a.hidden_out : nullptr;
  rms_finish<NB>(st, K, a.eps, xs, red, raw, a.ho_sb);
  f32x4 acc = tile_mfma<NB, kQkvBlk>(wa, xs, K, kb0, n, lane);
  if (kp != 0) part[w][lane] = acc;
  __syncthreads();
  if (kp != 0) return;
#pragma unroll
  for (int s = 1; s < kQkvKS; ++s) acc += part[w + s][lane];
  const int rb_raw = (int)blockIdx.x * (kNW / kQkvKS) + w / kQkvKS;
  if (col >= NB || rb_raw >= nrb) return;
  const int b = col;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int d = d0 + t;
    const float lo = (float)(f16)(acc[t] + bias[t][0]);
    const float hi = (float)(f16)(acc[t + 2] + bias[t][1]);
    if (head < a.QH + a.KVH) {
      f16 olo, ohi;
      rope1(lo, hi, cs[t][0], cs[t][1], cs[t][2], cs[t][3], olo, ohi);
      if (head < a.QH) {
        f16* qo = a.q_out + b * a.qo_sb + head * a.qo_sh;
        qo[d] = olo;
        qo[d + 32] = ohi;
      } else if (in_range) {
        f16* kd = a.kc + kro + (head - a.QH) * a.kc_sh;
        kd[d] = olo;
        kd[d + 32] = ohi;
      }
    } else if (in_range) {
      f16* vd = a.vc + vro + (head - a.QH - a.KVH) * a.vc_sh;
      vd[d] = (f16)lo;
      vd[d + 32] = (f16)hi;
    }
  }
}

// ---------------------------------------------------------------------------
// Weight packing (one pass at load time): tile (rb, kb), lane l, 16 bytes =
// W[row(rb, l % 16)][32 kb + 8 (l / 16) ..].  Row maps: plain rows 16 rb + r;
// QF_PACK_SWIGLU as above; QF_PACK_ROPE puts row block rb = 4 head + c on
// rows 64 head + 8c + 2g + (i & 1) (+ 32 for i >= 2), pairing each
// rotate-half (d, d + 32) in one lane's C registers.
__device__ __forceinline__ int pack_row(int layout, int N, int rb, int r) {
  const int g = r >> 2, i = r & 3;
  if (layout == QF_PACK_SWIGLU) {
    const int j = 8 * rb + 2 * g + (i & 1);
    return (i & 2) ? N / 2 + j : j;
  }
  if (layout == QF_PACK_ROPE) {
    const int head = rb >> 2, c = rb & 3;
    return 64 * head + 8 * c + 2 * g + (i & 1) + ((i & 2) ? 32 : 0);
  }
  return 16 * rb + r;
}

__global__ __launch_bounds__(256) void pack_weight_kernel(const f16* __restrict__ w, int64_t w_sb,
                                                          f16* __restrict__ out, int N, int K,
                                                          int layout) {
  const int nkb = K / 32;
  const int64_t chunk = (int64_t)blockIdx.x * 256 + threadIdx.x;  // one 16-byte chunk
  const int64_t total = (int64_t)(N / 16) * nkb * 64;
  if (chunk >= total) return;
  const int lane = (int)(chunk & 63);
  const int64_t tile = chunk >> 6;
  const int rb = (int)(tile / nkb), kb = (int)(tile % nkb);
  const int row = pack_row(layout, N, rb, lane & 15);
  store16(out + chunk * 8, load16(w + row * w_sb + 32 * kb + 8 * (lane >> 4)));
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
    for (int r = 0; r < RW; ++r)
      load_row<NS>(a.w + (int64_t)min(grp * RW + r, a.V - 1) * K, C, buf[r], lane);
  };
  const f16* rows[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) rows[b] = a.x + b * a.x_sb;
  RmsStage<NB> st;
  rms_load<NB>(st, rows, K, a.norm_w);
  load_group(min(g, groups - 1), cur);
  rms_finish<NB>(st, K, a.eps, xs, red, nullptr, 0);

  uint64_t best[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) best[b] = 0;
  for (; g < groups; g += stride) {
    load_group(min(g + stride, groups - 1), nxt);  // past the end: a real row, unused
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

// lm_head on matrix-core tiles (packed with QF_PACK_PLAIN: 16 vocab rows per
// row block, its K/32 tiles one contiguous run), for 2-4 batch rows: the
// batch rows are the MFMA columns, so a wave spends one MFMA and one 16-byte
// LDS read per 1 KB of weights, where the VALU form spends four v_dot2 and an
// LDS read per batch row and 16 bytes, plus a 64-lane butterfly per row and
// batch row.  Each wave takes whole row blocks (grid-stride), in stages of
// kLmKC tiles with the next stage's loads always in flight (past the end it
// reloads a real tile, unused); an f32x4 accumulator holds rows 4 (l / 16) + i
// of batch row l % 16.  Logits and keys as rms_lm_head_kernel.  Measured on
// MI355X at vocab 151936, K = 896, weights past the MALL: 45.6-45.8 us at
// every batch, against the row kernel's 43.2 (B=1), 44.8 (B=2) and 51.1 (B=4);
// stages of 7 or 14 tiles took 46.8 / 50.4.
constexpr int kLmKC = 8;

template <int NB>
__global__ __launch_bounds__(kNT) void rms_lm_head_mfma_kernel(LmArgs a) {
  __shared__ __attribute__((aligned(16))) f16 xs[NB * kMaxNormK];
  __shared__ float red[kNW * NB];
  __shared__ uint64_t wkeys[kNW][NB];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int K = a.K, nkb = K / 32;
  const int nch = (nkb + kLmKC - 1) / kLmKC;
  const int nrb = a.V / 16;
  const int stride = gridDim.x * kNW;
  const int rb0 = blockIdx.x * kNW + w;
  const int mine = rb0 < nrb ? (nrb - 1 - rb0) / stride + 1 : 0;
  const int items = mine * nch;
  auto load_stage = [&](int i, f16x8 (&buf)[kLmKC]) {
    const int ii = min(i, max(items - 1, 0));
    const int rb = min(rb0 + (ii / nch) * stride, nrb - 1), ch = ii % nch;
#pragma unroll
    for (int t = 0; t < kLmKC; ++t) buf[t] = tile_load(a.w, nkb, rb, min(ch * kLmKC + t, nkb - 1), lane);
  };
  const f16* rows[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) rows[b] = a.x + b * a.x_sb;
  RmsStage<NB> st;
  rms_load<NB>(st, rows, K, a.norm_w);
  f16x8 cur[kLmKC], nxt[kLmKC];
  load_stage(0, cur);
  rms_finish<NB>(st, K, a.eps, xs, red, nullptr, 0);

  const int col = lane & 15, q = lane >> 4;
  uint64_t best = 0;
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  for (int i = 0; i < items; ++i) {
    load_stage(i + 1, nxt);
    const int ch = i % nch;
    const int n = min(kLmKC, nkb - ch * kLmKC);
    // A stage past the row's last k block multiplies zeros (its tiles are
    // re-read real ones), so the MFMA sequence has no branch.
    f16x8 xb[kLmKC];
#pragma unroll
    for (int t = 0; t < kLmKC; ++t) xb[t] = t < n ? act_operand<NB>(xs, K, ch * kLmKC + t, lane) : zero8();
#pragma unroll
    for (int t = 0; t < kLmKC; ++t) {
      if (t & 1) acc1 = mfma16x16x32(cur[t], xb[t], acc1);
      else acc0 = mfma16x16x32(cur[t], xb[t], acc0);
    }
    if (ch == nch - 1) {
      const f32x4 acc = acc0 + acc1;
      const int n0 = 16 * (rb0 + (i / nch) * stride) + 4 * q;
      if (col < NB) {
        f16x4 lg;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          lg[e] = (f16)acc[e];
          const uint64_t key = argmax_key(lg[e], n0 + e);
          best = key > best ? key : best;
        }
        *reinterpret_cast<f16x4*>(a.logits + col * a.lg_sb + n0) = lg;
      }
      acc0 = f32x4{0.f, 0.f, 0.f, 0.f};
      acc1 = acc0;
    }
#pragma unroll
    for (int t = 0; t < kLmKC; ++t) cur[t] = nxt[t];
  }
  // Best key of each batch row: over the four lanes of its column, then the
  // waves.
#pragma unroll
  for (int off = 16; off < 64; off <<= 1) {
    const unsigned lo = __shfl_xor((unsigned)best, off), hi = __shfl_xor((unsigned)(best >> 32), off);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    best = o > best ? o : best;
  }
  if (lane < NB) wkeys[w][lane] = best;
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
  __shared__ uint64_t part[kMaxB][256];
  const int tid = threadIdx.x;
  // Every load is issued before any wait: the keys, the step counter and
  // (thread b) row b's position.  The optional counters are read branch-free
  // (a missing one reads a key and is dropped): a guarded load would wait for
  // completion before the key loads go out.
  const int64_t* keys64 = reinterpret_cast<const int64_t*>(a.keys);
  const int64_t s_raw = (a.step != nullptr ? a.step : keys64)[0];
  const int64_t p_raw = (a.pos != nullptr ? a.pos : keys64)[min(tid, a.B - 1)];
  const int64_t w_raw = (a.write_index != nullptr ? a.write_index : keys64)[0];
  const int64_t s = a.step != nullptr ? s_raw : 0;
  const int64_t p = a.pos != nullptr ? p_raw : 0;
  const int64_t wi = a.write_index != nullptr ? w_raw : 0;
  // Four keys per row per thread and round, all rows' loads issued together
  // (indices past n_blocks re-read the last key).
  uint64_t k[kMaxB];
#pragma unroll
  for (int b = 0; b < kMaxB; ++b) k[b] = 0;
  const int rows = a.B;
  for (int j0 = tid; j0 < a.n_blocks; j0 += 4 * 256) {
    uint64_t v[kMaxB][4];
#pragma unroll
    for (int b = 0; b < kMaxB; ++b)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int j = min(j0 + 256 * u, a.n_blocks - 1);
        v[b][u] = a.keys[(int64_t)min(b, rows - 1) * a.n_blocks + j];
      }
#pragma unroll
    for (int b = 0; b < kMaxB; ++b)
#pragma unroll
      for (int u = 0; u < 4; ++u) k[b] = v[b][u] > k[b] ? v[b][u] : k[b];
  }
#pragma unroll
  for (int b = 0; b < kMaxB; ++b) part[b][tid] = k[b];
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (tid < o) {
#pragma unroll
      for (int b = 0; b < kMaxB; ++b) {
        const uint64_t v = part[b][tid + o];
        if (v > part[b][tid]) part[b][tid] = v;
      }
    }
    __syncthreads();
  }
  if (tid < a.B) {
    const int64_t tok = (int64_t)(0xFFFFFFFFu - (unsigned)(part[tid][0] & 0xFFFFFFFFu));
    a.token[tid] = tok;
    if (a.rows != nullptr && s >= 0 && s < a.n_rows) a.rows[tid * a.rows_sb + s] = tok;
    if (a.pos != nullptr) a.pos[tid] = p + 1;
  }
  if (tid == 0) {
    if (a.write_index != nullptr) a.write_index[0] = wi + 1;
    if (a.step != nullptr) a.step[0] = s + 1;
  }
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

extern "C" int qf_pack_weight(const void* w, int64_t w_sb, void* packed, int N, int K, int layout,
                              void* stream) {
  if (layout != QF_PACK_PLAIN && layout != QF_PACK_SWIGLU && layout != QF_PACK_ROPE)
    return QF_ERR_INVALID_ARG;
  if (N < 16 || N % 16 || K < 32 || K % 32) return QF_ERR_UNSUPPORTED;
  if (layout == QF_PACK_ROPE && N % 64) return QF_ERR_UNSUPPORTED;
  if (!w || !packed || w_sb < K || (w_sb & 7) || !al16(w) || !al16(packed)) return QF_ERR_INVALID_ARG;
  const int64_t chunks = (int64_t)N * K / 8;
  if ((chunks + 255) / 256 > 0x7fffffff) return QF_ERR_INVALID_ARG;
  hipLaunchKernelGGL(pack_weight_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const f16*>(w), w_sb,
                     static_cast<f16*>(packed), N, K, layout);
  return (int)hipGetLastError();
}

// RoPE source of the QKV entry points: 0 = cos/sin tables, 1 = positions +
// inv_freq, -1 = neither or a mix.
static int rope_source(const void* cos, const void* sin, const int64_t* pos, const float* inv_freq) {
  if (cos && sin && !pos && !inv_freq) return 0;
  if (!cos && !sin && pos && inv_freq) return 1;
  return -1;
}

extern "C" int qf_rms_qkv_rope_append(const void* x, int64_t x_sb, const int64_t* token,
                                      void* hidden_out, int64_t ho_sb,
                                      const void* norm_w, float eps,
                                      const void* w_qkv, int w_layout, const void* bias,
                                      const void* cos, const void* sin, int64_t cs_sb,
                                      const int64_t* pos, const float* inv_freq,
                                      void* k_cache, int64_t kc_sb, int64_t kc_sh, int64_t kc_sn,
                                      void* v_cache, int64_t vc_sb, int64_t vc_sh, int64_t vc_sn,
                                      const int64_t* write_index,
                                      void* q_out, int64_t qo_sb, int64_t qo_sh,
                                      int B, int hidden, int QH, int KVH, int D, int cap,
                                      void* stream) {
  if (w_layout != QF_W_ROWS && w_layout != QF_W_TILES) return QF_ERR_INVALID_ARG;
  if (D != kHeadDim) return QF_ERR_UNSUPPORTED;
  if (B < 1 || B > kMaxB || hidden < 8 || hidden > kMaxNormK || hidden % 8) return QF_ERR_UNSUPPORTED;
  if (!x || !norm_w || !w_qkv || !k_cache || !v_cache || !write_index || !q_out)
    return QF_ERR_INVALID_ARG;
  const int rope_mode = rope_source(cos, sin, pos, inv_freq);
  if (rope_mode < 0) return QF_ERR_INVALID_ARG;
  if (QH < 1 || KVH < 1 || cap < 1) return QF_ERR_INVALID_ARG;
  if (token != nullptr && hidden_out != nullptr && (!al16(hidden_out) || (ho_sb & 7)))
    return QF_ERR_INVALID_ARG;
  if (!al16(x) || !al16(norm_w) || !al16(w_qkv) || (x_sb & 7)) return QF_ERR_INVALID_ARG;
  QkvArgs a;
  a.table = nullptr; a.t_sb = 0; a.log2p = 0; a.n_pages = 0; a.slots = nullptr; a.slot_sb = 0;
  a.x = static_cast<const f16*>(x); a.x_sb = x_sb; a.token = token;
  a.hidden_out = static_cast<f16*>(hidden_out); a.ho_sb = ho_sb;
  a.norm_w = static_cast<const f16*>(norm_w); a.eps = eps;
  a.w = static_cast<const f16*>(w_qkv); a.bias = static_cast<const f16*>(bias);
  a.cos = static_cast<const f16*>(cos); a.sin = static_cast<const f16*>(sin); a.cs_sb = cs_sb;
  a.pos = pos; a.inv_freq = inv_freq;
  a.kc = static_cast<f16*>(k_cache); a.kc_sb = kc_sb; a.kc_sh = kc_sh; a.kc_sn = kc_sn;
  a.vc = static_cast<f16*>(v_cache); a.vc_sb = vc_sb; a.vc_sh = vc_sh; a.vc_sn = vc_sn;
  a.write_index = write_index;
  a.q_out = static_cast<f16*>(q_out); a.qo_sb = qo_sb; a.qo_sh = qo_sh;
  a.K = hidden; a.QH = QH; a.KVH = KVH; a.cap = cap;
  a.n_pairs = (QH + 2 * KVH) * (kHeadDim / 2);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((a.n_pairs + kNW - 1) / kNW), block(kNT);
  const size_t shm = 0;
  if (w_layout == QF_W_TILES) {
    if (hidden % 32) return QF_ERR_UNSUPPORTED;
    const dim3 tgrid(((QH + 2 * KVH) * 4 + kNW / kQkvKS - 1) / (kNW / kQkvKS));
    const dim3& grid = tgrid;
    if (rope_mode == 1) {
      QF_DISPATCH_B(B, rms_qkv_rope_append_mfma_kernel, false, true)
    } else {
      QF_DISPATCH_B(B, rms_qkv_rope_append_mfma_kernel, false, false)
    }
  } else if (rope_mode == 1) {
    QF_DISPATCH_B(B, rms_qkv_rope_append_kernel, false, true)
  } else {
    QF_DISPATCH_B(B, rms_qkv_rope_append_kernel, false, false)
  }
  return (int)hipGetLastError();
}

extern "C" int qf_rms_qkv_rope_append_paged(const void* x, int64_t x_sb, const int64_t* token,
                                            void* hidden_out, int64_t ho_sb,
                                            const void* norm_w, float eps,
                                            const void* w_qkv, int w_layout, const void* bias,
                                            const void* cos, const void* sin, int64_t cs_sb,
                                            const int64_t* pos, const float* inv_freq,
                                            void* k_pool, int64_t kp_sp, int64_t kp_sh, int64_t kp_sn,
                                            void* v_pool, int64_t vp_sp, int64_t vp_sh, int64_t vp_sn,
                                            const int32_t* block_table, int64_t bt_sb,
                                            int pages_per_row, int n_pages, int page_size,
                                            const int64_t* slots, int64_t slot_sb,
                                            void* q_out, int64_t qo_sb, int64_t qo_sh,
                                            int B, int hidden, int QH, int KVH, int D,
                                            void* stream) {
  if (w_layout != QF_W_ROWS && w_layout != QF_W_TILES) return QF_ERR_INVALID_ARG;
  const int l2 = page_log2(page_size, pages_per_row, n_pages);
  if (D != kHeadDim || l2 < 0) return QF_ERR_UNSUPPORTED;
  if (B < 1 || B > kMaxB || hidden < 8 || hidden > kMaxNormK || hidden % 8) return QF_ERR_UNSUPPORTED;
  if (!x || !norm_w || !w_qkv || !k_pool || !v_pool || !block_table || !slots || !q_out)
    return QF_ERR_INVALID_ARG;
  const int rope_mode = rope_source(cos, sin, pos, inv_freq);
  if (rope_mode < 0) return QF_ERR_INVALID_ARG;
  if (QH < 1 || KVH < 1 || bt_sb < pages_per_row) return QF_ERR_INVALID_ARG;
  if (token != nullptr && hidden_out != nullptr && (!al16(hidden_out) || (ho_sb & 7)))
    return QF_ERR_INVALID_ARG;
  if (!al16(x) || !al16(norm_w) || !al16(w_qkv) || (x_sb & 7)) return QF_ERR_INVALID_ARG;
  QkvArgs a;
  a.x = static_cast<const f16*>(x); a.x_sb = x_sb; a.token = token;
  a.hidden_out = static_cast<f16*>(hidden_out); a.ho_sb = ho_sb;
  a.norm_w = static_cast<const f16*>(norm_w); a.eps = eps;
  a.w = static_cast<const f16*>(w_qkv); a.bias = static_cast<const f16*>(bias);
  a.cos = static_cast<const f16*>(cos); a.sin = static_cast<const f16*>(sin); a.cs_sb = cs_sb;
  a.pos = pos; a.inv_freq = inv_freq;
  a.kc = static_cast<f16*>(k_pool); a.kc_sb = kp_sp; a.kc_sh = kp_sh; a.kc_sn = kp_sn;
  a.vc = static_cast<f16*>(v_pool); a.vc_sb = vp_sp; a.vc_sh = vp_sh; a.vc_sn = vp_sn;
  a.write_index = nullptr;
  a.q_out = static_cast<f16*>(q_out); a.qo_sb = qo_sb; a.qo_sh = qo_sh;
  a.K = hidden; a.QH = QH; a.KVH = KVH; a.cap = pages_per_row * page_size;
  a.n_pairs = (QH + 2 * KVH) * (kHeadDim / 2);
  a.table = block_table; a.t_sb = bt_sb; a.log2p = l2; a.n_pages = n_pages;
  a.slots = slots; a.slot_sb = slot_sb;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((a.n_pairs + kNW - 1) / kNW), block(kNT);
  const size_t shm = 0;
  if (w_layout == QF_W_TILES) {
    if (hidden % 32) return QF_ERR_UNSUPPORTED;
    const dim3 tgrid(((QH + 2 * KVH) * 4 + kNW / kQkvKS - 1) / (kNW / kQkvKS));
    const dim3& grid = tgrid;
    if (rope_mode == 1) {
      QF_DISPATCH_B(B, rms_qkv_rope_append_mfma_kernel, true, true)
    } else {
      QF_DISPATCH_B(B, rms_qkv_rope_append_mfma_kernel, true, false)
    }
  } else if (rope_mode == 1) {
    QF_DISPATCH_B(B, rms_qkv_rope_append_kernel, true, true)
  } else {
    QF_DISPATCH_B(B, rms_qkv_rope_append_kernel, true, false)
  }
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
    // Short rows (o_proj): two rows per wave; the B x K input is at most two
    // chunks per thread.
    const dim3 grid((N + kNW * 2 - 1) / (kNW * 2));
    if (B * C <= kNT) { QF_DISPATCH_B(B, gemv_residual_kernel, 2, 2, 1) }
    else { QF_DISPATCH_B(B, gemv_residual_kernel, 2, 2, 2) }
  } else {
    // Long rows (down_proj): gemv_residual_direct_kernel, one row per
    // workgroup split between two waves, nothing staged in LDS; 5 chunk
    // rounds per wave up to K = 5120 (K = 4864: 4.75), 8 up to kMaxK.
    constexpr int kKP = 2, kRPW = 1;
    const dim3 gridd((N + kRPW - 1) / kRPW), blockd(kKP * kRPW * 64);
    const dim3& grid = gridd;
    const dim3& block = blockd;
    const size_t shm = 0;
    if ((C + kKP - 1) / kKP <= 5 * 64) { QF_DISPATCH_B(B, gemv_residual_direct_kernel, 5, kKP, kRPW) }
    else { QF_DISPATCH_B(B, gemv_residual_direct_kernel, 8, kKP, kRPW) }
  }
  return (int)hipGetLastError();
}

extern "C" int qf_attn_merge_o_proj(const float* acc, const float* m, const float* l, int splits,
                                    int KVH, int G, const void* w_o, int w_layout, void* hidden,
                                    int64_t h_sb, int B, int N, void* stream) {
  const int K = KVH * G * kHeadDim;
  if (w_layout != QF_W_ROWS && w_layout != QF_W_TILES) return QF_ERR_INVALID_ARG;
  if (B < 1 || B > kMaxB || G < 1 || KVH < 1 || K > kMaxNormK || KVH * G * 16 > kNT)
    return QF_ERR_UNSUPPORTED;
  if (!acc || !m || !l || !w_o || !hidden || N < 1 || splits < 1) return QF_ERR_INVALID_ARG;
  if (!al16(acc) || !al16(w_o)) return QF_ERR_INVALID_ARG;
  // Matrix-core form: whole 16-row blocks, 8-byte residual loads and stores.
  if (w_layout == QF_W_TILES && N % 16) return QF_ERR_UNSUPPORTED;
  if (w_layout == QF_W_TILES && ((reinterpret_cast<uintptr_t>(hidden) & 7) || (h_sb & 3)))
    return QF_ERR_INVALID_ARG;
  MergeArgs a;
  a.acc = acc; a.m = m; a.l = l;
  a.splits = splits; a.KVH = KVH; a.G = G;
  a.w = static_cast<const f16*>(w_o);
  a.hidden = static_cast<f16*>(hidden); a.h_sb = h_sb;
  a.K = K; a.N = N;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // Every workgroup re-reads all partials, so batched calls use fewer, wider
  // workgroups (measured on MI355X: B=1 best at 2 rows per wave, B=4 at 4).
  const size_t shm = 0;
  if (w_layout == QF_W_TILES) {
    const dim3 grid(N / 16), block(kNT);
    QF_DISPATCH_B(B, attn_merge_o_proj_mfma_kernel)
    return (int)hipGetLastError();
  }
  const int RW = B == 1 ? 2 : 4;
  const dim3 grid((N + kNW * RW - 1) / (kNW * RW)), block(kNT);
  if (RW == 2) { QF_DISPATCH_B(B, attn_merge_gemv_residual_kernel, 2) }
  else { QF_DISPATCH_B(B, attn_merge_gemv_residual_kernel, 4) }
  return (int)hipGetLastError();
}

extern "C" int qf_rms_gate_up_swiglu(const void* x, int64_t x_sb, const void* norm_w, float eps,
                                     const void* w_gate_up, int w_layout, void* h_out,
                                     int64_t ho_sb, int B, int hidden, int I, void* stream) {
  if (w_layout != QF_W_ROWS && w_layout != QF_W_TILES) return QF_ERR_INVALID_ARG;
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
  const dim3 block(kNT);
  const size_t shm = 0;
  if (w_layout == QF_W_TILES) {
    // 8 SwiGLU pairs per row block, kNW / kGuKS row blocks per workgroup.
    if (hidden % 32 || I % 8) return QF_ERR_UNSUPPORTED;
    const dim3 grid((I / 8 + kNW / kGuKS - 1) / (kNW / kGuKS));
    QF_DISPATCH_B(B, rms_gate_up_swiglu_mfma_kernel)
  } else {
    constexpr int PW = 2;
    const dim3 grid((I + kNW * PW - 1) / (kNW * PW));
    QF_DISPATCH_B(B, rms_gate_up_swiglu_kernel, PW)
  }
  return (int)hipGetLastError();
}

extern "C" int qf_rms_lm_head(const void* x, int64_t x_sb, const void* norm_w, float eps,
                              const void* w_lm, int w_layout, void* logits, int64_t lg_sb,
                              uint64_t* keys, int n_blocks, int B, int hidden, int V, void* stream) {
  if (w_layout != QF_W_ROWS && w_layout != QF_W_TILES) return QF_ERR_INVALID_ARG;
  if (B < 1 || B > kMaxB || hidden < 8 || hidden > kMaxNormK || hidden % 8) return QF_ERR_UNSUPPORTED;
  if (!x || !norm_w || !w_lm || !logits || !keys || V < 1) return QF_ERR_INVALID_ARG;
  // Matrix-core form: whole 16-row blocks, 8-byte logit stores.
  if (w_layout == QF_W_TILES && (hidden % 32 || V % 16)) return QF_ERR_UNSUPPORTED;
  if (w_layout == QF_W_TILES && ((reinterpret_cast<uintptr_t>(logits) & 7) || (lg_sb & 3)))
    return QF_ERR_INVALID_ARG;
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
  if (w_layout == QF_W_TILES) { QF_DISPATCH_B(B, rms_lm_head_mfma_kernel) }
  else { QF_DISPATCH_B(B, rms_lm_head_kernel) }
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
