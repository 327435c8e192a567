// Split-K flash-decoding GQA attention for gfx950 (MI355X).
//
// Replaces _flash_decode_split_kernel (student_engine.py:32-115),
// _flash_decode_combine_kernel (:117-162) and their launcher
// _flash_decode_attention (:834-874).
//
// Work split: one workgroup of NW wave64s per (split, batch row b, kv head h);
// the waves interleave over 32-key tiles of the split's slot range, with the
// next tile's loads issued before the current tile is computed.  Per tile a
// wave
//   1. streams K straight from HBM into MFMA A-operand registers (16-byte
//      loads, rows permuted so the score tile comes out in P^T order),
//   2. streams V with coalesced 16-byte loads (8 lanes per 128-byte row) and
//      transposes it through a private LDS tile with 8-byte writes (the PV
//      product needs keys in-lane),
//   3. computes S^T = K Q^T (2 x 2 MFMA 16x16x32), adds scale and bias in the
//      log2 domain and runs the online softmax on the lane's query column,
//   4. accumulates O^T += V^T P^T (4 MFMAs, one per 16-wide d slice).
// The G query heads of a kv group ride the 16 MFMA columns (columns >= G are
// zero queries whose results are dropped), so K and V are read once per
// (b, h).  The waves merge through LDS.  Then, by mode:
//   kDirect   (one split)  the workgroup writes the fp16 output itself;
//   kPartial  it writes one partial (acc, m, l) in the reference's scratch
//             layout, with write-through (sc1) stores, and a second kernel
//             merges them (the reference's two-launch shape);
//   kFused    it writes the partial likewise, waits for the stores to
//             complete (s_waitcnt vmcnt(0) in every wave, then a barrier)
//             and takes the (b, h) ticket; the last workgroup of the
//             (b, h) merges all S partials (one wave per query) with sc1
//             loads, writes the output and re-arms the ticket.  Every
//             partial store is an agent-scope atomic store, so the completion
//             wait is all an agent-scope release has to add here; the full
//             release fence would also write back the whole L2 per workgroup.
// Every merge folds its partials in batches of independent loads (four or
// eight partials per lane, all in flight) followed by register / permlane /
// LDS reductions: one dependent memory round trip per batch, and one batch
// covers the single-launch merge's at most 32 splits and the combine's up to
// 128.
#include <mutex>

#include "qf_common.h"
#include "../../include/qf_attn.h"
#include "../../include/qf_paged.h"

namespace qf {

constexpr int kD = 64;
constexpr int kTile = 32;       // keys per wave iteration
constexpr int kVtStride = 36;   // LDS row stride (halves) of a transposed V tile
constexpr int kMaxG = 16;

// kPartialCap: kPartial over the capacity split (split_range<true>).
enum Mode { kDirect = 0, kPartial = 1, kFused = 2, kPartialCap = 3 };

// Merge mode of a call with `splits` partials; `ticket`: the caller passed
// merge counters (single launch).
constexpr int merge_mode(int splits, bool ticket) {
  return splits == 1 ? kDirect : (ticket ? kFused : kPartial);
}

struct DecodeArgs {
  const f16* q;
  int64_t q_sb, q_sh, q_sg;
  const f16* k;
  int64_t k_sb, k_sh, k_sn;
  const f16* v;
  int64_t v_sb, v_sh, v_sn;
  const f16* bias;
  int64_t bias_sb;
  const int64_t* kv_last;
  int64_t kv_last_sb;
  float* acc;
  float* m;
  float* l;
  int32_t* ticket;
  f16* out;
  int64_t o_sb, o_sh, o_sg;
  int B, KVH, G, cap, splits;
  int bias_vec;      // bias rows 16-byte aligned and cap % 8 == 0: 8 keys per load
  float scale_log2;  // scale * log2(e)
  // Paged caches: k/v are page pools (n_pages, KVH, P, D) with page strides
  // k_sp/v_sp (k_sb/v_sb unused); logical slot s of row b lives in page
  // table[b * t_sb + (s >> log2p)] at row s & (P - 1).  cap = pages per row * P.
  const int32_t* table;
  int64_t t_sb, k_sp, v_sp;
  int log2p, n_pages;
};
static_assert(covers_lines(sizeof(DecodeArgs),
                           {offsetof(DecodeArgs, q), offsetof(DecodeArgs, v),
                            offsetof(DecodeArgs, acc), offsetof(DecodeArgs, KVH),
                            offsetof(DecodeArgs, log2p)}),
              "the split kernel's touch_arg_lines fields cover every line");
// Partial-scratch store: a relaxed agent-scope atomic store, which the
// compiler emits as a write-through (sc1) store, so a workgroup on another
// XCD sees it without an L2 writeback.
__device__ __forceinline__ void st_wt(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Slot range [lo, hi) that split `s` of batch row `b` reads.  By default the
// row's valid slots end at upper = kv_last[b] + 1 (clamped to [0, cap]; cap
// without a bound) and split_len = ceil(upper / S), rounded up to whole
// 32-key tiles: every split stays busy and nothing past the newest slot is
// read, but the first tile's addresses wait for the kv_last load.  kCap
// splits the capacity as the reference does (split_len = ceil(cap / S) at
// SE:851), so the ranges need no device load; kv_last then only masks (see
// the kernel).  A compile-time choice: with a run-time one the ranges would
// still wait for the load through a select.
template <bool kCap>
__device__ __forceinline__ void split_range(const DecodeArgs& a, int b, int s, int& lo, int& hi) {
  int span = a.cap;
  if (!kCap && a.kv_last != nullptr) {
    const int64_t last = a.kv_last[(int64_t)b * a.kv_last_sb];
    span = (int)(last + 1 < 0 ? 0 : (last + 1 > a.cap ? a.cap : last + 1));
  }
  int split_len = (span + a.splits - 1) / a.splits;
  split_len = (split_len + kTile - 1) / kTile * kTile;
  lo = s * split_len;
  hi = lo + split_len < span ? lo + split_len : span;
}

// (M, L, A) <- log-sum-exp merge of two partial states (m in natural-log
// units, -inf for an empty state).
__device__ __forceinline__ void lse_merge(float& M, float& L, f32x4& A, float M2, float L2,
                                          f32x4 A2) {
  const float mn = fmaxf(M, M2);
  const float safe = (mn == kNegInf) ? 0.f : mn;
  const float w1 = (M == kNegInf) ? 0.f : fast_exp2((M - safe) * kLog2e);
  const float w2 = (M2 == kNegInf) ? 0.f : fast_exp2((M2 - safe) * kLog2e);
  L = L * w1 + L2 * w2;
  A = A * w1 + A2 * w2;
  M = mn;
}

// Merges the states of lanes l and l ^ 16 (kXor32: l ^ 32).  The permlane
// swaps hand both lanes the pair in the same (lower row, upper row) order, so
// the two lanes end with bit-identical states.
template <bool kXor32>
__device__ __forceinline__ void lse_merge_lanes(float& M, float& L, f32x4& A) {
  float m0, m1, l0, l1;
  f32x4 a0, a1;
  const auto pair = [](float x, float& lo, float& hi) {
    if (kXor32) xor32_pair(x, lo, hi);
    else xor16_pair(x, lo, hi);
  };
  pair(M, m0, m1);
  pair(L, l0, l1);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float lo, hi;
    pair(A[c], lo, hi);
    a0[c] = lo;
    a1[c] = hi;
  }
  lse_merge(m0, l0, a0, m1, l1, a1);
  M = m0;
  L = l0;
  A = a0;
}

// Folds partials of query q of (b, h) = bh into the running state (M, L, A)
// of dims 4*d4 .. +3, d4 = lane % 16.  The wave's four 16-lane rows hold the
// consecutive subs sub0 + lane / 16 out of nsub; sub folds partials
// j = sub + nsub * u, batch after batch of kB (j < S).  In a batch the wave
// loads each of its 4 kB partials' (m, l) once -- lane i loads partial
// sub0 + i % 4 + nsub * (i / 4) -- and hands them to the 16 lanes that fold
// the partial with ds_bpermute; the acc slices are one 16-byte load per lane
// and partial.  So a batch is 2 + kB vector memory instructions per wave, all
// in flight before the first wait: one round trip.  (Sixteen lanes loading
// each (m, l) would make it 2 kB more, and the merge is bound by those
// instructions.)  Every partial index goes into the vector offset: the buffer
// range check covers the vector and immediate offsets but not the scalar
// offset, and only the checked offset turns a partial past S (the last
// batch of a split count that is not a multiple of nsub * kB) into zeros
// instead of a read of whatever follows the scratch.
// kCoherent: sc1 loads, for partials that other workgroups of the same
// launch stored with sc1 stores.
template <int kB, bool kCoherent>
__device__ __forceinline__ void fold_wave(const DecodeArgs& a, int bh, int q, int lane, int sub0,
                                          int nsub, float& M, float& L, f32x4& A) {
  static_assert(4 * kB <= 64, "a batch's (m, l) must fit one load per lane");
  const int G = a.G, S = a.splits;
  const int s4 = lane >> 4, d4 = lane & 15, sub = sub0 + s4;
  constexpr int aux = kCoherent ? kSc1 : 0;
  const int64_t pbase = (int64_t)bh * S;
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(a.acc + pbase * G * kD, (int64_t)S * G * kD * 4);
  const __amdgpu_buffer_rsrc_t rm = buffer_rsrc(a.m + pbase * G, (int64_t)S * G * 4);
  const __amdgpu_buffer_rsrc_t rl = buffer_rsrc(a.l + pbase * G, (int64_t)S * G * 4);
  const int ml_lane = lane < 4 * kB ? lane : 0;
  const int j_ml = sub0 + (ml_lane & 3) + nsub * (ml_lane >> 2);
  const int acc_step = nsub * G * kD * 4;
  for (int j0 = 0; j0 < S; j0 += nsub * kB) {
    // Partials past S read 0 (the buffers end there; the offsets are all
    // vector offsets, which the range check covers) and are masked below.
    const float m_mine = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(rm, ((j0 + j_ml) * G + q) * 4, 0, aux));
    const float l_mine = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(rl, ((j0 + j_ml) * G + q) * 4, 0, aux));
    const int acc_off = (((j0 + sub) * G + q) * kD + 4 * d4) * 4;
    f32x4 av[kB];
#pragma unroll
    for (int u = 0; u < kB; ++u)
      av[u] = __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, acc_off + u * acc_step, 0, aux));
    // Keep every load of the batch above this point: left alone, the
    // scheduler sinks loads next to their uses, and the batch becomes a chain
    // of dependent round trips.
    __builtin_amdgcn_sched_barrier(0);
    float mv[kB], lv[kB];
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      mv[u] = __shfl(m_mine, s4 + 4 * u);
      lv[u] = __shfl(l_mine, s4 + 4 * u);
      if (j0 + sub + nsub * u >= S) mv[u] = kNegInf;
    }
    float mc = mv[0];
#pragma unroll
    for (int u = 1; u < kB; ++u) mc = fmaxf(mc, mv[u]);
    const float mn = fmaxf(M, mc);
    const float safe = (mn == kNegInf) ? 0.f : mn;
    const float r = (M == kNegInf) ? 0.f : fast_exp2((M - safe) * kLog2e);
    L *= r;
    A *= r;
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const float wu = (mv[u] == kNegInf) ? 0.f : fast_exp2((mv[u] - safe) * kLog2e);
      L += wu * lv[u];
      A += wu * av[u];
    }
    M = mn;
  }
}

// fp16 out[b, h, q, 4*d4 .. +3] = A / L.
__device__ __forceinline__ void store_out(const DecodeArgs& a, int bh, int q, int d4, float L,
                                          f32x4 A) {
  const float inv = 1.f / L;
  const int b = bh / a.KVH, h = bh % a.KVH;
  const f16x4 o = {(f16)(A[0] * inv), (f16)(A[1] * inv), (f16)(A[2] * inv), (f16)(A[3] * inv)};
  *reinterpret_cast<f16x4*>(a.out + b * a.o_sb + h * a.o_sh + q * a.o_sg + 4 * d4) = o;
}

enum Bias { kNoBias = 0, kBiasVec = 1, kBiasScalar = 2 };

// The V rows are kept as raw 32-bit words (two dims each): as f16 vectors
// the compiler splits them into 16-bit pieces across the tile loop's back
// edge, which puts unpacking (and a wait) right behind every load.
struct Tile {
  f16x8 k[2][2];  // [score block j][k step kk]
  u32x4 v[4];     // 4 keys x 8 dims
  f16x8 bias;     // bias of the lane's keys t0 + 8*grp .. +7
};

// Issues every load of one 32-key tile -- K operands, V rows and the bias of
// the lane's 8 keys -- with no wait in between.  K and V, read once per call,
// use non-temporal loads: against plain loads, graph-replayed calls over
// caches rotated past the MALL, config 2 7.01 vs 7.32 us, B=1 L=32768 split +
// combine 9.3 vs 10.1, B=16 L=32768 49.2 vs 53.6 (same outputs).  Keys past `last` re-read
// slot `last` (their scores are masked).  kBiasVec reads the 8 bias values
// as one 16-byte load from min(kbase, cap - 8): in bounds, aligned (the
// caller checks cap % 8 == 0 and 16-byte rows), and correct for every key
// below cap because kbase is a multiple of 8.
template <int kBias>
__device__ __forceinline__ void load_tile(Tile& t, const f16* kb, const f16* vb, const f16* biasb,
                                          int64_t k_sn, int64_t v_sn, int t0, int last, int cap,
                                          int lane) {
  const int col = lane & 15, grp = lane >> 4;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    // Score-block row r reads key t0 + 8*(r/4) + 4*j + r%4, so C block j holds
    // keys t0 + 8*grp + 4*j + i in register i: exactly the P^T operand order.
    int key = t0 + 8 * (col >> 2) + 4 * j + (col & 3);
    key = key < last ? key : last;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) t.k[j][kk] = load16_nt(kb + (int64_t)key * k_sn + 32 * kk + 8 * grp);
  }
  // V: lane (m = lane & 7, c = lane >> 3) reads dims 8c..8c+7 of keys
  // t0 + 4m + r; the 8 lanes sharing m cover whole 128-byte rows.
  const int m4 = 4 * (lane & 7), c8 = 8 * (lane >> 3);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    int key = t0 + m4 + r;
    key = key < last ? key : last;
    t.v[r] = __builtin_bit_cast(u32x4, load16_nt(vb + (int64_t)key * v_sn + c8));
  }
  const int kbase = t0 + 8 * grp;
  if (kBias == kBiasVec) {
    t.bias = load16(biasb + (kbase < cap - 8 ? kbase : cap - 8));
  } else if (kBias == kBiasScalar) {
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) t.bias[jj] = biasb[kbase + jj < last ? kbase + jj : last];
  }
}

// Physical page of slot `slot` of row b, clamped into the pool (a page id
// outside [0, n_pages) is a caller error; clamping keeps the reads in bounds).
__device__ __forceinline__ int page_of(const DecodeArgs& a, int b, int slot) {
  const int p = a.table[(int64_t)b * a.t_sb + (slot >> a.log2p)];
  return min(max(p, 0), a.n_pages - 1);
}

template <int NW, int kBias, int kMode, bool kPaged>
__global__ __launch_bounds__(NW * 64) void decode_split_kernel(DecodeArgs a) {
  constexpr bool kHasBias = kBias != kNoBias;
  constexpr int NT = NW * 64;
  // LDS: per-wave transposed V tiles during the sweep; each wave's region
  // then holds that wave's accumulator for the cross-wave merge.
  constexpr int kVtBytes = NW * kD * kVtStride * 2;
  __shared__ __attribute__((aligned(16))) unsigned char lds_raw[kVtBytes];
  __shared__ float sm_ml[2][NW][kMaxG];
  __shared__ int sh_last;

  const int s = blockIdx.x;
  const int bh = blockIdx.y;
  // The fields the first loads depend on (q, the kv_last bound, K/V and the
  // bias rows), one from each further line (acc, log2p).
  const int KVH = touch_arg_lines(a.KVH, a.q, a.v, a.bias, a.kv_last, a.kv_last_sb, a.acc, a.log2p);
  const int b = bh / KVH, h = bh % KVH;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: tile math stays scalar
  const int col = lane & 15;  // query column / A-operand row
  const int grp = lane >> 4;  // 8-wide k chunk of the operands

  // Q^T operand: lane holds Q[col][32*kk + 8*grp .. +7].  Issued before the
  // split range is known (it may depend on kv_last, a device load).
  // Columns >= G load query G-1 (in bounds) and are zeroed by a select, so
  // the loads carry no branch and fly together with the first tile's.
  f16x8 qf[2];
  {
    const int qc = col < a.G ? col : a.G - 1;
    const f16* qp = a.q + b * a.q_sb + h * a.q_sh + qc * a.q_sg + 8 * grp;
    f16x8 zero;
#pragma unroll
    for (int e = 0; e < 8; ++e) zero[e] = (f16)0.f;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const f16x8 ld = load16(qp + 32 * kk);
      qf[kk] = col < a.G ? ld : zero;
    }
  }

  constexpr bool kCap = kMode == kPartialCap;
  int lo, hi;
  split_range<kCap>(a, b, s, lo, hi);
  // kCap: kv_last only masks.  It is read with a vector load (a VGPR
  // address), issued with the q loads ahead of the first tile's, and first
  // used in the first tile's compute: the wait for it is then an in-order
  // vmcnt wait the tile loads behind it have not been held up by.  (A
  // scalar load is waited for with lgkmcnt(0), which the next scalar load of
  // a kernel argument forces before the tile loads are issued.)
  int64_t kvl = (int64_t)a.cap - 1;
  if (kCap && a.kv_last != nullptr) {
    int zero = 0;
    asm("" : "+v"(zero));
    kvl = a.kv_last[(int64_t)b * a.kv_last_sb + zero];
  }

  float m_run = kNegInf, l_run = 0.f;
  f32x4 o[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const f16* kb = a.k + b * a.k_sb + h * a.k_sh;
  const f16* vb = a.v + b * a.v_sb + h * a.v_sh;
  const f16* biasb = kHasBias ? a.bias + b * a.bias_sb : nullptr;
  f16(*vt)[kVtStride] = reinterpret_cast<f16(*)[kVtStride]>(lds_raw + w * kD * kVtStride * 2);

  // Paged caches: lane j holds the physical page of this wave's tile
  // win + j (tile i of the wave starts at lo + (w + i*NW) * kTile and lies in
  // one page, since pages hold a multiple of kTile slots and tiles start on
  // kTile boundaries); one load per 64 tiles of the wave.  The tile's base
  // pointers are then shifted so that logical slot numbers index them.
  int pid = 0;
  const auto load_pids = [&](int win, int clamp) {
    int t = lo + (w + (win + lane) * NW) * kTile;
    t = t < clamp ? t : clamp;
    pid = page_of(a, b, t > 0 ? t : 0);
  };
  const auto tile_base = [&](int i, int t0, const f16*& kt, const f16*& vtb) {
    if (!kPaged) {
      kt = kb;
      vtb = vb;
      return;
    }
    const int page = __builtin_amdgcn_readlane(pid, i & 63);
    const int64_t first = (int64_t)(t0 & ~((1 << a.log2p) - 1));  // first slot of the page
    kt = a.k + (int64_t)page * a.k_sp + h * a.k_sh - first * a.k_sn;
    vtb = a.v + (int64_t)page * a.v_sp + h * a.v_sh - first * a.v_sn;
  };

  const int last = hi - 1;
  constexpr int kStep = NW * kTile;
  const f16 *kt_, *vt_;
  // Issues the loads of the wave's tile i (first key tn) into t.
  const auto prefetch = [&](Tile& t, int i, int tn) __attribute__((always_inline)) {
    if (kPaged && (i & 63) == 0) load_pids(i, last);
    tile_base(i, tn, kt_, vt_);
    load_tile<kBias>(t, kt_, vt_, biasb, a.k_sn, a.v_sn, tn, last, a.cap, lane);
  };
  // Scores, online softmax and PV product of one tile (keys t0 .. t0 + 31).
  const auto consume = [&](const Tile& cur, int t0) __attribute__((always_inline)) {
    // Scores of keys at or past hv are dropped: hi, or under kCap also the
    // slots past kv_last.  The empty asm keeps the use of kvl (and so the
    // wait for its load) here instead of letting it be hoisted above the
    // tile loads.
    int hv = hi;
    if (kCap) {
      int64_t x = kvl;
      asm volatile("" : "+v"(x));
      const int upper = (int)(x + 1 < 0 ? 0 : (x + 1 > a.cap ? a.cap : x + 1));
      hv = __builtin_amdgcn_readfirstlane(hi < upper ? hi : upper);
    }
    // Bias of the lane's 8 keys t0 + 8*grp + jj, in log2 units.
    float bv[8];
    const int kbase = t0 + 8 * grp;
    if (kHasBias) {
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) bv[jj] = (float)cur.bias[jj] * kLog2e;
    }

    f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
    c0 = mfma16x16x32(cur.k[0][0], qf[0], c0);
    c0 = mfma16x16x32(cur.k[0][1], qf[1], c0);
    c1 = mfma16x16x32(cur.k[1][0], qf[0], c1);
    c1 = mfma16x16x32(cur.k[1][1], qf[1], c1);

    // Transpose V into LDS: vt[d][key - t0], four keys per 8-byte write.
    // Dim e of the four keys: the low (e even) or high half of word e / 2 of
    // each row, paired by byte selects.  Over the capacity split, rows at or
    // past hv are whatever the cache holds there: they are zeroed, since
    // their zero weights would not cancel a NaN or an infinity (0 * NaN).
    {
      const int m4 = 4 * (lane & 7), c8 = 8 * (lane >> 3);
      u32x4 vr[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        vr[r] = cur.v[r];
        if (kCap && t0 + m4 + r >= hv) vr[r] = u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const unsigned sel = (e & 1) ? 0x07060302u : 0x05040100u;
        const u32x2 w = {__builtin_amdgcn_perm(vr[1][e >> 1], vr[0][e >> 1], sel),
                         __builtin_amdgcn_perm(vr[3][e >> 1], vr[2][e >> 1], sel)};
        *reinterpret_cast<f16x4*>(&vt[c8 + e][m4]) = __builtin_bit_cast(f16x4, w);
      }
    }

    float sc[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      float x = (jj < 4 ? c0[jj] : c1[jj - 4]) * a.scale_log2;
      if (kHasBias) x += bv[jj];
      sc[jj] = kbase + jj < hv ? x : kNegInf;
    }
    float mt = sc[0];
#pragma unroll
    for (int jj = 1; jj < 8; ++jj) mt = fmaxf(mt, sc[jj]);
    mt = col_max(mt);
    const float m_new = fmaxf(m_run, mt);
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

    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const f16x4 va0 = *reinterpret_cast<const f16x4*>(&vt[16 * t + col][8 * grp]);
      const f16x4 va1 = *reinterpret_cast<const f16x4*>(&vt[16 * t + col][8 * grp + 4]);
      const f16x8 va = {va0[0], va0[1], va0[2], va0[3], va1[0], va1[1], va1[2], va1[3]};
      o[t] = mfma16x16x32(va, pb, o[t] * resc);
    }
    __builtin_amdgcn_wave_barrier();
  };
  // Two tile buffers in turn.  The wave's tile count n is known up front, so
  // the loop runs whole pairs whose prefetches are unconditional and the one
  // or two remaining tiles are peeled: no load batch sits behind a branch and
  // no two paths with different loads in flight meet, so the compiler's wait
  // before each use counts exactly the newer tile's loads as still in flight
  // and two tiles are in flight while the older one lands.  (With a
  // conditional prefetch the waits had to cover every load, the prefetch
  // included, so a tile's compute could not overlap the next tile's loads.)
  // The scheduling barriers keep each tile's first use below the next tile's
  // loads.
  int t0 = lo + w * kTile;
  const int n = t0 < hi ? (hi - t0 + kStep - 1) / kStep : 0;
  if (n > 0) {
    Tile ta, tb;
    prefetch(ta, 0, t0);
    int i = 0;
    for (; i + 2 < n; i += 2, t0 += 2 * kStep) {
      prefetch(tb, i + 1, t0 + kStep);
      __builtin_amdgcn_sched_barrier(0);
      consume(ta, t0);
      prefetch(ta, i + 2, t0 + 2 * kStep);
      __builtin_amdgcn_sched_barrier(0);
      consume(tb, t0 + kStep);
    }
    if (i + 2 == n) {
      prefetch(tb, i + 1, t0 + kStep);
      __builtin_amdgcn_sched_barrier(0);
      consume(ta, t0);
      consume(tb, t0 + kStep);
    } else {
      consume(ta, t0);
    }
  }

  l_run = col_sum(l_run);

  // Cross-wave merge, one barrier.  A wave's softmax state is replicated over
  // the four lanes of each query column.  Every wave publishes its (m, l) per
  // column and its unscaled accumulator as 16-byte rows [t][lane] in its own
  // V-tile region of LDS (no other wave touches that region, so no barrier
  // is needed before the overwrite); a wave that saw no tile publishes the
  // empty state (m = -inf, l = 0, zero accumulator), which drops out of the
  // merge.  After the barrier wave w' < min(NW, 4) merges (M, L) and sums the
  // NW accumulators of its 16-dim slices t = w', w' + NW, ..., each scaled by
  // exp2(m_w - M), and stores them from the MFMA layout (lane (q, grp) holds
  // dims 16t + 4grp .. +3 of query q).  Every LDS read of the pass is
  // independent of the others.
  constexpr int kWaveLds = kD * kVtStride * 2;  // bytes of a wave's V tile
  static_assert(4 * 64 * 16 <= kWaveLds, "a wave's accumulator fits its V-tile region");
  const auto sm_o = [&](int ww) { return reinterpret_cast<f32x4*>(lds_raw + ww * kWaveLds); };
  if (grp == 0) {
    sm_ml[0][w][col] = m_run;
    sm_ml[1][w][col] = l_run;
  }
  // The V-tile reads above and the f32 writes below alias the same bytes
  // through different types: keep the compiler from reordering them (the
  // wave's LDS accesses then execute in program order).
  asm volatile("" ::: "memory");
#pragma unroll
  for (int t = 0; t < 4; ++t) sm_o(w)[t * 64 + lane] = o[t];
  __syncthreads();

  const int S = a.splits, G = a.G;
  const int64_t part = (int64_t)bh * S + s;
  if (w < 4) {
    float mw[NW], wt[NW];
    float M = kNegInf;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      mw[ww] = sm_ml[0][ww][col];
      M = fmaxf(M, mw[ww]);
    }
    const float safe = (M == kNegInf) ? 0.f : M;
    float L = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      wt[ww] = (mw[ww] == kNegInf) ? 0.f : fast_exp2(mw[ww] - safe);
      L += wt[ww] * sm_ml[1][ww][col];
    }
    for (int t = w; t < 4; t += NW) {
      f32x4 acc = sm_o(0)[t * 64 + lane] * wt[0];
#pragma unroll
      for (int ww = 1; ww < NW; ++ww) acc += sm_o(ww)[t * 64 + lane] * wt[ww];
      if (col < G) {
        const int d = 16 * t + 4 * grp;
        if (kMode == kDirect) {
          const float inv = 1.f / L;
          const f16x4 ov = {(f16)(acc[0] * inv), (f16)(acc[1] * inv), (f16)(acc[2] * inv),
                            (f16)(acc[3] * inv)};
          *reinterpret_cast<f16x4*>(a.out + b * a.o_sb + h * a.o_sh + col * a.o_sg + d) = ov;
        } else {
          // Partials are written through (sc1) in both merge modes: the
          // single launch reads them from other XCDs, and before a combine
          // launch they leave no dirty L2 lines for the end-of-kernel
          // writeback (split + combine, B=1 L=32768: 10.16 vs 10.24 us;
          // B=1 L=8192 8.03 vs 8.19).  The resource must be wave-uniform (it
          // lives in SGPRs): one per split, the lane's query row and dims go
          // in the offset.
          const __amdgpu_buffer_rsrc_t ra =
              buffer_rsrc(a.acc + part * G * kD, (int64_t)G * kD * 4);
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc), ra,
                                                 (col * kD + d) * 4, 0, kSc1);
        }
      }
    }
    if (kMode != kDirect && w == 0 && grp == 0 && col < G) {
      st_wt(a.m + part * G + col, (M == kNegInf) ? kNegInf : M * kLn2);
      st_wt(a.l + part * G + col, L);
    }
  }

  if (kMode == kFused) {
    // Publication.  The partial stores above are write-through (sc1) stores,
    // i.e. relaxed agent-scope atomic stores.  Each wave waits until its own
    // have been acknowledged (vmcnt counts stores on gfx9); after the barrier
    // every store of the workgroup has completed, so they precede the ticket
    // increment in memory order.  The workgroup that completes the count
    // (one int32 counter per (b, h)) issues its partial loads only after the
    // increment has returned, and loads with sc1 (relaxed agent-scope atomic
    // loads), so it reads the stored values.  It merges all S partials --
    // wave w takes queries w, w + NW, ...; within a wave lane
    // (sub = lane / 16, d4 = lane % 16) folds partials j = sub (mod 4)
    // (fold_wave) and the four subs merge through permlane swaps -- then
    // re-arms the ticket.
    int32_t* tk = a.ticket + bh;
    s_waitcnt_vm(0);
    __syncthreads();
    if (tid == 0) sh_last = (atomicAdd(tk, 1) == S - 1);
    __syncthreads();
    if (!sh_last) return;
    for (int q = w; q < G; q += NW) {
      float Mq = kNegInf, Lq = 0.f;
      f32x4 Aq = {0.f, 0.f, 0.f, 0.f};
      if (S <= 16) fold_wave<4, true>(a, bh, q, lane, 0, 4, Mq, Lq, Aq);
      else fold_wave<8, true>(a, bh, q, lane, 0, 4, Mq, Lq, Aq);
      lse_merge_lanes<false>(Mq, Lq, Aq);
      lse_merge_lanes<true>(Mq, Lq, Aq);
      if (lane < 16) store_out(a, bh, q, lane, Lq, Aq);
    }
    if (tid == 0) atomicExch(tk, 0);
  }
}

#ifndef QF_DECODE_FUSED_VEC_UNIT
// Second launch of the two-kernel shape: one workgroup of four waves per
// (b, h, query).  Thread (sub = tid / 16, d4 = tid % 16) folds partials
// j = sub, sub + 16, ... of dims 4*d4 .. +3 (fold_wave, eight per batch);
// the 4 subs of a wave merge through permlane swaps (lanes d4 + 16r), the 4
// waves through LDS, and wave 0 writes fp16 acc / l.
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeArgs a) {
  __shared__ float red[3][16][6];
  const int G = touch_arg_lines(a.G, a.acc);  // the lines it reads
  const int bh = blockIdx.x / G, q = blockIdx.x % G;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int d4 = lane & 15;
  float M = kNegInf, L = 0.f;
  f32x4 A = {0.f, 0.f, 0.f, 0.f};
  fold_wave<8, false>(a, bh, q, lane, 4 * w, 16, M, L, A);
  lse_merge_lanes<false>(M, L, A);
  lse_merge_lanes<true>(M, L, A);
  if (w > 0 && lane < 16) {
    float* e = red[w - 1][lane];
    e[0] = M; e[1] = L; e[2] = A[0]; e[3] = A[1]; e[4] = A[2]; e[5] = A[3];
  }
  __syncthreads();
  if (w == 0 && lane < 16) {
#pragma unroll
    for (int ww = 0; ww < 3; ++ww) {
      const float* e = red[ww][lane];
      lse_merge(M, L, A, e[0], e[1], f32x4{e[2], e[3], e[4], e[5]});
    }
    store_out(a, bh, q, d4, L, A);
  }
}

// The single-launch-merge instances with a 16-byte bias over a contiguous
// cache (the ragged serving batch of the headline shape) are compiled in
// their own unit, decode_attn_fused_vec.hip, with LLVM's max-ILP machine
// scheduler; everything else here keeps the default one.  Measured on MI355X
// (outputs bit-identical): config 2 6.85 vs 6.97 us per launch, while the
// same flag on the whole file made config 3 (9.95 vs 9.71) and the
// single-launch merge without bias at B=12 L=5760 (12.05 vs 11.76) slower.
void launch_fused_vec(const DecodeArgs& a, int nw, dim3 grid, hipStream_t st);

template <int NW, int kBias, bool kPaged>
static void launch_split(const DecodeArgs& a, int mode, dim3 grid, hipStream_t st) {
  const dim3 block(NW * 64);
  if (mode == kDirect) {
    hipLaunchKernelGGL((decode_split_kernel<NW, kBias, kDirect, kPaged>), grid, block, 0, st, a);
  } else if (mode == kPartial) {
    hipLaunchKernelGGL((decode_split_kernel<NW, kBias, kPartial, kPaged>), grid, block, 0, st, a);
  } else if (mode == kPartialCap) {
    if constexpr (!kPaged)
      hipLaunchKernelGGL((decode_split_kernel<NW, kBias, kPartialCap, false>), grid, block, 0, st, a);
  } else if constexpr (kBias == kBiasVec && !kPaged) {
    launch_fused_vec(a, NW, grid, st);
  } else {
    hipLaunchKernelGGL((decode_split_kernel<NW, kBias, kFused, kPaged>), grid, block, 0, st, a);
  }
}

template <int NW, bool kPaged>
static void launch_nw(const DecodeArgs& a, int mode, dim3 grid, hipStream_t st) {
  if (!a.bias) launch_split<NW, kNoBias, kPaged>(a, mode, grid, st);
  else if (a.bias_vec) launch_split<NW, kBiasVec, kPaged>(a, mode, grid, st);
  else launch_split<NW, kBiasScalar, kPaged>(a, mode, grid, st);
}

#endif  // QF_DECODE_FUSED_VEC_UNIT

#ifdef QF_DECODE_FUSED_VEC_UNIT
void launch_fused_vec(const DecodeArgs& a, int nw, dim3 grid, hipStream_t st) {
  const dim3 block(nw * 64);
  if (nw == 16)
    hipLaunchKernelGGL((decode_split_kernel<16, kBiasVec, kFused, false>), grid, block, 0, st, a);
  else if (nw == 8)
    hipLaunchKernelGGL((decode_split_kernel<8, kBiasVec, kFused, false>), grid, block, 0, st, a);
  else if (nw == 4)
    hipLaunchKernelGGL((decode_split_kernel<4, kBiasVec, kFused, false>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((decode_split_kernel<2, kBiasVec, kFused, false>), grid, block, 0, st, a);
}
#endif

}  // namespace qf

#ifndef QF_DECODE_FUSED_VEC_UNIT
using namespace qf;

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Waves per workgroup (measured on MI355X): sixteen when one workgroup per
// kv head streams everything, eight up to two workgroups per CU (also for
// small grids: at B=1 with 8 splits, 8 waves beat 16 by 0.7 us per call), four
// for large grids -- and never more waves than the split has 32-key tiles
// (idle waves only lengthen the cross-wave merge).  The single-launch merge
// gives each query a wave: NW >= G.  Otherwise (below 16 waves), down to
// four waves, each wave gets at least two tiles, so its second tile's loads fly under the
// first's compute (config 3, 8 tiles per split: 4 waves 10.57 us, 8 waves
// 10.80).
static int pick_waves(const DecodeArgs& a, int mode) {
  const int64_t wgs = (int64_t)a.splits * a.B * a.KVH;
  int nw = wgs <= 2 ? 16 : (wgs <= 512 ? 8 : 4);
  const int split_len = (a.cap + a.splits - 1) / a.splits;
  const int tiles = (split_len + kTile - 1) / kTile;
  const int min_nw = mode == kFused ? a.G : 1;
  while (nw > 2 && nw / 2 >= tiles && nw / 2 >= min_nw) nw /= 2;
  if (mode != kFused && wgs > 2)
    while (nw > 4 && 2 * nw > tiles) nw /= 2;
  return nw;
}

// Validates the decode arguments and fills DecodeArgs; 0 or a QF_ERR_* code.
static int make_args(DecodeArgs& a, const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sg,
                     const void* k, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                     const void* v, int64_t v_sb, int64_t v_sh, int64_t v_sn,
                     const void* bias, int64_t bias_sb, const int64_t* kv_last,
                     int64_t kv_last_sb, float* acc, float* m, float* l, int splits,
                     int32_t* ticket, void* out, int64_t o_sb, int64_t o_sh, int64_t o_sg,
                     int B, int KVH, int G, int D, int cap, float scale, bool need_qkv,
                     bool need_out) {
  if (D != kD || G < 1 || G > kMaxG) return QF_ERR_UNSUPPORTED;
  if (!acc || !m || !l) return QF_ERR_INVALID_ARG;
  if (B < 1 || KVH < 1 || splits < 1 || splits > 65535 || B * (int64_t)KVH > 65535)
    return QF_ERR_INVALID_ARG;
  if ((int64_t)B * KVH * G > 0x7fffffff) return QF_ERR_INVALID_ARG;
  if (!aligned16(acc)) return QF_ERR_INVALID_ARG;
  if (need_qkv) {
    if (!q || !k || !v || cap < 1) return QF_ERR_INVALID_ARG;
    // 16-byte vector loads of q/k/v rows.
    if (!aligned16(q) || !aligned16(k) || !aligned16(v)) return QF_ERR_INVALID_ARG;
    if ((q_sb | q_sh | q_sg | k_sb | k_sh | k_sn | v_sb | v_sh | v_sn) & 7) return QF_ERR_INVALID_ARG;
  }
  if (need_out) {
    // 8-byte stores of out.
    if (!out || (reinterpret_cast<uintptr_t>(out) & 7u) != 0 || ((o_sb | o_sh | o_sg) & 3))
      return QF_ERR_INVALID_ARG;
  }
  a.q = static_cast<const f16*>(q);
  a.q_sb = q_sb; a.q_sh = q_sh; a.q_sg = q_sg;
  a.k = static_cast<const f16*>(k);
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_sn = k_sn;
  a.v = static_cast<const f16*>(v);
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_sn = v_sn;
  a.bias = static_cast<const f16*>(bias);
  a.bias_sb = bias_sb;
  a.bias_vec = bias != nullptr && aligned16(bias) && (bias_sb & 7) == 0 && cap % 8 == 0 && cap >= 8;
  a.kv_last = kv_last;
  a.kv_last_sb = kv_last_sb;
  a.acc = acc; a.m = m; a.l = l;
  a.ticket = ticket;
  a.out = static_cast<f16*>(out);
  a.o_sb = o_sb; a.o_sh = o_sh; a.o_sg = o_sg;
  a.B = B; a.KVH = KVH; a.G = G; a.cap = cap; a.splits = splits;
  a.scale_log2 = scale * kLog2e;
  a.table = nullptr;
  a.t_sb = a.k_sp = a.v_sp = 0;
  a.log2p = 0;
  a.n_pages = 0;
  return QF_OK;
}


template <bool kPaged>
static void launch_split_paging(const DecodeArgs& a, int mode, hipStream_t st) {
  const dim3 grid(a.splits, a.B * a.KVH);
  const int nw = pick_waves(a, mode);
  if (nw == 16) launch_nw<16, kPaged>(a, mode, grid, st);
  else if (nw == 8) launch_nw<8, kPaged>(a, mode, grid, st);
  else if (nw == 4) launch_nw<4, kPaged>(a, mode, grid, st);
  else launch_nw<2, kPaged>(a, mode, grid, st);
}

static void launch_split_mode(const DecodeArgs& a, int mode, hipStream_t st) {
  if (a.table != nullptr) launch_split_paging<true>(a, mode, st);
  else launch_split_paging<false>(a, mode, st);
}

static void launch_combine(const DecodeArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(decode_combine_kernel, dim3(a.B * a.KVH * a.G), dim3(256), 0, st, a);
}

extern "C" int qf_decode_attn(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sg,
                              const void* k, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                              const void* v, int64_t v_sb, int64_t v_sh, int64_t v_sn,
                              const void* bias, int64_t bias_sb,
                              const int64_t* kv_last, int64_t kv_last_sb,
                              float* acc, float* m, float* l, int splits,
                              int32_t* ticket,
                              void* out, int64_t o_sb, int64_t o_sh, int64_t o_sg,
                              int B, int KVH, int G, int D, int cap, float scale,
                              void* stream) {
  DecodeArgs a;
  const int rc = make_args(a, q, q_sb, q_sh, q_sg, k, k_sb, k_sh, k_sn, v, v_sb, v_sh, v_sn,
                           bias, bias_sb, kv_last, kv_last_sb, acc, m, l, splits, ticket, out,
                           o_sb, o_sh, o_sg, B, KVH, G, D, cap, scale, true, true);
  if (rc != QF_OK) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int mode = merge_mode(splits, ticket != nullptr);
  launch_split_mode(a, mode, st);
  if (mode == kPartial) launch_combine(a, st);
  return (int)hipGetLastError();
}

extern "C" int qf_decode_waves(int B, int KVH, int G, int cap, int splits, int fused) {
  if (G < 1 || G > kMaxG || B < 1 || KVH < 1 || cap < 1 || splits < 1 || splits > 65535)
    return QF_ERR_INVALID_ARG;
  DecodeArgs a{};
  a.B = B;
  a.KVH = KVH;
  a.G = G;
  a.cap = cap;
  a.splits = splits;
  return pick_waves(a, merge_mode(splits, fused != 0));
}

extern "C" int qf_decode_split(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sg,
                               const void* k, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                               const void* v, int64_t v_sb, int64_t v_sh, int64_t v_sn,
                               const void* bias, int64_t bias_sb,
                               const int64_t* kv_last, int64_t kv_last_sb,
                               float* acc, float* m, float* l, int splits,
                               int B, int KVH, int G, int D, int cap, float scale,
                               void* stream) {
  DecodeArgs a;
  const int rc = make_args(a, q, q_sb, q_sh, q_sg, k, k_sb, k_sh, k_sn, v, v_sb, v_sh, v_sn,
                           bias, bias_sb, kv_last, kv_last_sb, acc, m, l, splits, nullptr,
                           nullptr, 0, 0, 0, B, KVH, G, D, cap, scale, true, false);
  if (rc != QF_OK) return rc;
  launch_split_mode(a, kPartial, static_cast<hipStream_t>(stream));
  return (int)hipGetLastError();
}

extern "C" int qf_decode_split_capacity(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sg,
                                        const void* k, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                                        const void* v, int64_t v_sb, int64_t v_sh, int64_t v_sn,
                                        const void* bias, int64_t bias_sb,
                                        const int64_t* kv_last, int64_t kv_last_sb,
                                        float* acc, float* m, float* l, int splits,
                                        int B, int KVH, int G, int D, int cap, float scale,
                                        void* stream) {
  DecodeArgs a;
  const int rc = make_args(a, q, q_sb, q_sh, q_sg, k, k_sb, k_sh, k_sn, v, v_sb, v_sh, v_sn,
                           bias, bias_sb, kv_last, kv_last_sb, acc, m, l, splits, nullptr,
                           nullptr, 0, 0, 0, B, KVH, G, D, cap, scale, true, false);
  if (rc != QF_OK) return rc;
  launch_split_paging<false>(a, kPartialCap, static_cast<hipStream_t>(stream));
  return (int)hipGetLastError();
}

extern "C" int qf_decode_combine(const float* acc, const float* m, const float* l, int splits,
                                 void* out, int64_t o_sb, int64_t o_sh, int64_t o_sg,
                                 int B, int KVH, int G, int D, void* stream) {
  DecodeArgs a;
  const int rc = make_args(a, nullptr, 0, 0, 0, nullptr, 0, 0, 0, nullptr, 0, 0, 0, nullptr, 0,
                           nullptr, 0, const_cast<float*>(acc), const_cast<float*>(m),
                           const_cast<float*>(l), splits, nullptr, out, o_sb, o_sh, o_sg, B, KVH,
                           G, D, 1, 1.f, false, true);
  if (rc != QF_OK) return rc;
  launch_combine(a, static_cast<hipStream_t>(stream));
  return (int)hipGetLastError();
}

// Paged variants: the contiguous (B, KVH, cap, D) cache is replaced by page
// pools and a block table; everything else is the contiguous entry points'.
static int make_paged(DecodeArgs& a, int64_t kp_sp, int64_t vp_sp, const int32_t* block_table,
                      int64_t bt_sb, int pages_per_row, int n_pages, int page_size) {
  const int l2 = page_log2(page_size, pages_per_row, n_pages);
  if (l2 < 0) return QF_ERR_UNSUPPORTED;
  if (!block_table || bt_sb < pages_per_row) return QF_ERR_INVALID_ARG;
  if ((kp_sp | vp_sp) & 7) return QF_ERR_INVALID_ARG;
  a.table = block_table;
  a.t_sb = bt_sb;
  a.k_sp = kp_sp;
  a.v_sp = vp_sp;
  a.log2p = l2;
  a.n_pages = n_pages;
  return QF_OK;
}

extern "C" int qf_decode_attn_paged(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sg,
                                    const void* k_pool, int64_t kp_sp, int64_t kp_sh, int64_t kp_sn,
                                    const void* v_pool, int64_t vp_sp, int64_t vp_sh, int64_t vp_sn,
                                    const int32_t* block_table, int64_t bt_sb, int pages_per_row,
                                    int n_pages, int page_size,
                                    const void* bias, int64_t bias_sb,
                                    const int64_t* kv_last, int64_t kv_last_sb,
                                    float* acc, float* m, float* l, int splits,
                                    int32_t* ticket,
                                    void* out, int64_t o_sb, int64_t o_sh, int64_t o_sg,
                                    int B, int KVH, int G, int D, float scale, void* stream) {
  if (page_log2(page_size, pages_per_row, n_pages) < 0) return QF_ERR_UNSUPPORTED;
  DecodeArgs a;
  int rc = make_args(a, q, q_sb, q_sh, q_sg, k_pool, 0, kp_sh, kp_sn, v_pool, 0, vp_sh, vp_sn,
                     bias, bias_sb, kv_last, kv_last_sb, acc, m, l, splits, ticket, out, o_sb,
                     o_sh, o_sg, B, KVH, G, D, pages_per_row * page_size, scale, true, true);
  if (rc == QF_OK)
    rc = make_paged(a, kp_sp, vp_sp, block_table, bt_sb, pages_per_row, n_pages, page_size);
  if (rc != QF_OK) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int mode = merge_mode(splits, ticket != nullptr);
  launch_split_mode(a, mode, st);
  if (mode == kPartial) launch_combine(a, st);
  return (int)hipGetLastError();
}

extern "C" int qf_decode_split_paged(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sg,
                                     const void* k_pool, int64_t kp_sp, int64_t kp_sh, int64_t kp_sn,
                                     const void* v_pool, int64_t vp_sp, int64_t vp_sh, int64_t vp_sn,
                                     const int32_t* block_table, int64_t bt_sb, int pages_per_row,
                                     int n_pages, int page_size,
                                     const void* bias, int64_t bias_sb,
                                     const int64_t* kv_last, int64_t kv_last_sb,
                                     float* acc, float* m, float* l, int splits,
                                     int B, int KVH, int G, int D, float scale, void* stream) {
  if (page_log2(page_size, pages_per_row, n_pages) < 0) return QF_ERR_UNSUPPORTED;
  DecodeArgs a;
  int rc = make_args(a, q, q_sb, q_sh, q_sg, k_pool, 0, kp_sh, kp_sn, v_pool, 0, vp_sh, vp_sn,
                     bias, bias_sb, kv_last, kv_last_sb, acc, m, l, splits, nullptr, nullptr, 0,
                     0, 0, B, KVH, G, D, pages_per_row * page_size, scale, true, false);
  if (rc == QF_OK)
    rc = make_paged(a, kp_sp, vp_sp, block_table, bt_sb, pages_per_row, n_pages, page_size);
  if (rc != QF_OK) return rc;
  launch_split_mode(a, kPartial, static_cast<hipStream_t>(stream));
  return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// No-allocation decode: the partials and merge counters of qf_decode_attn in
// a static device array (one copy per GPU), for callers that cannot allocate.
// ---------------------------------------------------------------------------

namespace {

constexpr int kNoAllocCounters = 65536;  // one per (b, h); make_args caps B*KVH at 65535
constexpr int64_t kNoAllocCounterBytes = (int64_t)kNoAllocCounters * 4;
constexpr int64_t kNoAllocBytes = kNoAllocCounterBytes + QF_NOALLOC_PARTIAL_BYTES;
constexpr int kMaxDevices = 64;

// Counters first (256 KiB), then acc / m / l of one call.  In host code
// `scratch` names a host-side stand-in: only the address from
// hipGetSymbolAddress (noalloc_base) may reach a kernel.
static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

std::mutex g_noalloc_mu;
unsigned char* g_noalloc_base[kMaxDevices] = {};

__global__ __launch_bounds__(256) void zero_counters_kernel(int32_t* p, int n) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0;
}

// Device address of `scratch` on the GPU that owns `st` (the null stream
// belongs to the current device).  The first call on a device looks the
// address up with that device current and zeroes the counters on `st` with a
// fill kernel, not a memset node: when that first call happens under stream
// capture the fill is recorded into the caller's graph and runs again at
// every replay, which is harmless because every merge leaves its counter at
// zero (and the array is zero when the library loads).
int noalloc_base(hipStream_t st, unsigned char** base) {
  int dev = -1;
  hipError_t e;
  if (st == nullptr) {
    e = hipGetDevice(&dev);
  } else {
    hipDevice_t d = -1;
    e = hipStreamGetDevice(st, &d);
    dev = (int)d;
  }
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return QF_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  if (g_noalloc_base[dev] == nullptr) {
    int cur = -1;
    e = hipGetDevice(&cur);
    if (e != hipSuccess) return (int)e;
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return (int)e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess && p == nullptr) e = hipErrorInvalidSymbol;
    if (e == hipSuccess) {
      hipLaunchKernelGGL(zero_counters_kernel, dim3(64), dim3(256), 0, st,
                         reinterpret_cast<int32_t*>(p), kNoAllocCounters);
      e = hipGetLastError();
    }
    if (cur != dev) {
      const hipError_t r = hipSetDevice(cur);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess) return (int)e;
    g_noalloc_base[dev] = static_cast<unsigned char*>(p);
  }
  *base = g_noalloc_base[dev];
  return QF_OK;
}

}  // namespace

extern "C" int qf_decode_attn_noalloc(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sg,
                                      const void* k, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                                      const void* v, int64_t v_sb, int64_t v_sh, int64_t v_sn,
                                      const void* bias, int64_t bias_sb,
                                      const int64_t* kv_last, int64_t kv_last_sb,
                                      int splits,
                                      void* out, int64_t o_sb, int64_t o_sh, int64_t o_sg,
                                      int B, int KVH, int G, int D, int cap, float scale,
                                      void* stream) {
  // Shape checks before any HIP call (make_args repeats them on the real pointers).
  if (D != kD || G < 1 || G > kMaxG) return QF_ERR_UNSUPPORTED;
  if (B < 1 || KVH < 1 || splits < 1 || splits > 65535 || B * (int64_t)KVH > 65535)
    return QF_ERR_INVALID_ARG;
  const int64_t rows = (int64_t)B * KVH * splits * G;
  const int64_t n_acc = rows * kD;
  if ((n_acc + 2 * rows) * 4 > (int64_t)QF_NOALLOC_PARTIAL_BYTES) return QF_ERR_SCRATCH_LIMIT;
  if (!q || !k || !v || !out || cap < 1) return QF_ERR_INVALID_ARG;
  hipStream_t st = static_cast<hipStream_t>(stream);
  unsigned char* base = nullptr;
  int rc = noalloc_base(st, &base);
  if (rc != QF_OK) return rc;
  float* acc = reinterpret_cast<float*>(base + kNoAllocCounterBytes);
  float* m = acc + n_acc;
  float* l = m + rows;
  // The merge qf_decode_attn uses for this split count with a caller ticket
  // (single launch) up to 32 splits, and without one (split + combine) above.
  const int mode = merge_mode(splits, splits <= 32);
  int32_t* ticket = mode == kFused ? reinterpret_cast<int32_t*>(base) : nullptr;
  DecodeArgs a;
  rc = make_args(a, q, q_sb, q_sh, q_sg, k, k_sb, k_sh, k_sn, v, v_sb, v_sh, v_sn, bias, bias_sb,
                 kv_last, kv_last_sb, acc, m, l, splits, ticket, out, o_sb, o_sh, o_sg, B, KVH,
                 G, D, cap, scale, true, true);
  if (rc != QF_OK) return rc;
  launch_split_mode(a, mode, st);
  if (mode == kPartial) launch_combine(a, st);
  return (int)hipGetLastError();
}

#endif  // QF_DECODE_FUSED_VEC_UNIT
