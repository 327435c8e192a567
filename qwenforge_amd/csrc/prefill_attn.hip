// Causal GQA flash-prefill for gfx950 (MI355X), with rotate-half RoPE and the
// KV-cache append optionally fused in.
//
// Replaces _gqa_flash_prefill_kernel (student_engine.py:164-251) as launched by
// the student_qwen::gqa_flash_prefill custom op (:254-280), plus the eager
// RoPE in front of it (:767, :542-554) and the slice append of the cached
// prefill (:715-716).
//
// Two kernels, both over query tiles of 64 rows launched heaviest-first (the
// last rows see the most keys), 16 query rows per wave:
//   prefill_lds2_kernel (every call with a cache to append to, and every call
//     without RoPE): a pre-pass writes rotated K and raw V to the cache, then
//     one workgroup of eight waves per query tile streams the key tiles back
//     from the cache into LDS with direct-to-LDS loads, the even tiles to
//     waves 0-3 and the odd ones to waves 4-7, which merge at the end;
//   prefill_kernel (RoPE without a cache): four waves per query tile, K
//     rotated in registers on its way to LDS.
// prefill_kernel: K/V tiles of 64 keys are double-buffered in LDS: while the
// waves compute on tile t, the registers already hold tile t+1's global
// loads, which are rotated (K) and written to the other LDS buffer
// afterwards, so one barrier per tile separates the phases and HBM latency
// overlaps the MFMA work.  Per 64-key tile the workgroup
//   - loads K with 16-byte loads, applies RoPE in registers (both halves of a
//     rotate-half pair are loaded by the same thread), stores the rotated rows
//     to LDS in natural [key][d] layout,
//   - loads V four keys per thread and stores it transposed ([d][key]) with
//     8-byte LDS writes,
//   - on the diagonal tile of the group's first query head, also writes the
//     rotated K and raw V into the cache (each key tile is written exactly
//     once per (b, kv head)).
// Each wave computes S^T = K Q^T and O^T += V^T P^T with
// v_mfma_f32_16x16x32_f16 and an online softmax in the log2 domain, one
// max/rescale decision per 64-key tile (the output accumulators are only
// rescaled when the running max grows by more than kRescaleSlack); Q is
// rotated in registers once at the start.  The causal mask is applied only on
// the diagonal and tail tiles.
#include <atomic>

#include "qf_common.h"
#include "../../include/qf_attn.h"
#include "../../include/qf_paged.h"

namespace qf {

namespace prefill {

constexpr int kD = 64;
constexpr int kBM = 64;        // query rows per workgroup
constexpr int kBN = 64;        // keys per tile
constexpr int kWaves = 4;
constexpr int kKStride = 72;   // LDS row stride (halves) of the K tile
constexpr int kVtStride = 68;  // LDS row stride (halves) of the V^T tile

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
  // Work order of the streaming kernel's one-dimensional grid when it needs
  // one to two workgroups per CU: the CU count (the first round), else 0
  // (heaviest query tiles first throughout).
  int snake;
  // Packed variable-length rows (ragged prefill): row b's tokens are
  // [cu[b], cu[b+1]) of q/k/v/out/cos/sin, whose batch strides are then 0;
  // S holds the longest row.  kv_packed: k/v are those packed inputs (1) or
  // the per-row cache (0).  cu == nullptr: every row has S tokens.
  const int* cu;
  int total;  // packed token count (bounds every row)
  int kv_packed;
  // Paged caches: kc/vc are page pools (page strides kc_sb/vc_sb); slot s of
  // row b lives in page table[b * t_sb + (s >> log2p)] at row s & (P - 1).
  // ppr = pages per row.
  const int32_t* table;
  int64_t t_sb;
  int log2p, n_pages, ppr;
};
// The fields the attention kernels (q, v, kc, B or QH, snake) and the
// pre-pass (k, v, kc, KVH, cu) pass to touch_arg_lines.
static_assert(covers_lines(sizeof(Args), {offsetof(Args, q), offsetof(Args, v), offsetof(Args, kc),
                                          offsetof(Args, B), offsetof(Args, snake)}),
              "touch_arg_lines fields cover every line");
static_assert(covers_lines(sizeof(Args), {offsetof(Args, k), offsetof(Args, v), offsetof(Args, kc),
                                          offsetof(Args, KVH), offsetof(Args, cu)}),
              "touch_arg_lines fields cover every line");

// Element offset of slot `slot` of row b (kv head 0) in a cache: contiguous,
// or through the block table (ok = false for a page outside the pool).
__device__ __forceinline__ int64_t cache_row(const Args& a, int b, int64_t slot, int64_t sb,
                                             int64_t sn, bool& ok) {
  if (a.table == nullptr) {
    ok = true;
    return b * sb + slot * sn;
  }
  const int page = a.table[b * a.t_sb + (slot >> a.log2p)];
  ok = page >= 0 && page < a.n_pages;
  return (int64_t)page * sb + (slot & ((1 << a.log2p) - 1)) * sn;
}

// Token count and first packed token of row b, clamped to [0, total) and to
// the longest row S, so any cu contents keep every access in bounds.
__device__ __forceinline__ void row_span(const Args& a, int b, int& S, int64_t& tok0) {
  if (a.cu != nullptr) {
    const int lo = min(max(a.cu[b], 0), a.total);
    const int hi = min(max(a.cu[b + 1], lo), a.total);
    tok0 = lo;
    S = min(hi - lo, a.S);
  } else {
    tok0 = 0;
    S = a.S;
  }
}

// Registers holding one K/V tile between its global load and its LDS store.
// The K rotation happens at store time, so the loads stay in flight while the
// previous tile is computed.
struct Stage {
  f16x8 klo, khi;   // K row (tid >> 2), dims 8c..8c+7 and 32+8c..
  f16x8 cs[4];      // cos/sin of that row for both halves (RoPE only)
  f16x8 v[4];       // threads < 128: V rows 4m..4m+3, dims 8c'..8c'+7
};

// Loader mapping, fixed for the kernel: thread -> K row (tid >> 2) with the
// 8-wide chunk pair 8*(tid & 3) / +32; threads < 128 -> V rows 4*(tid & 15)
// .. +3 with dims 8*(tid >> 4) .. +7.  The per-thread pointers are computed
// once; a tile only adds its uniform (scalar) row offset.
struct Loader {
  const f16* kp;     // K row pointer of tile 0 (+ chunk)
  const f16* vp;     // first V row pointer of tile 0 (+ chunk)
  int64_t cso;       // cos/sin element offset of tile 0's K row (+ chunk)
  int krow, kc8, vrow, vc8;
};

template <bool kRope>
__device__ __forceinline__ void stage_load(Stage& st, const Args& a, const f16* kb, const f16* vb,
                                           int64_t cs_off, const Loader& ld, int key0, bool tail,
                                           int tid) {
  const int S = a.S;
  if (!tail) {
    const f16* kp = ld.kp + key0 * a.k_sn;
    st.klo = load16(kp);
    st.khi = load16(kp + 32);
    if (kRope) {
      const int64_t co = ld.cso + key0 * a.cs_sn;
      st.cs[0] = load16(a.cos + co);
      st.cs[1] = load16(a.sin + co);
      st.cs[2] = load16(a.cos + co + 32);
      st.cs[3] = load16(a.sin + co + 32);
    }
    if (tid < 128) {
      const f16* vp = ld.vp + key0 * a.v_sn;
#pragma unroll
      for (int r = 0; r < 4; ++r) st.v[r] = load16(vp + r * a.v_sn);
    }
    return;
  }
  // Last tile: rows past the sequence repeat row S-1 (their scores are masked).
  {
    int key = key0 + ld.krow;
    key = key < S ? key : S - 1;
    const f16* kp = kb + (int64_t)key * a.k_sn + ld.kc8;
    st.klo = load16(kp);
    st.khi = load16(kp + 32);
    if (kRope) {
      const int64_t co = cs_off + (int64_t)key * a.cs_sn + ld.kc8;
      st.cs[0] = load16(a.cos + co);
      st.cs[1] = load16(a.sin + co);
      st.cs[2] = load16(a.cos + co + 32);
      st.cs[3] = load16(a.sin + co + 32);
    }
  }
  if (tid < 128) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int key = key0 + ld.vrow + r;
      key = key < S ? key : S - 1;
      st.v[r] = load16(vb + (int64_t)key * a.v_sn + ld.vc8);
    }
  }
}

template <bool kRope>
__device__ __forceinline__ void stage_rope(Stage& st) {
  if (kRope) rope_pair(st.klo, st.khi, st.cs[0], st.cs[1], st.cs[2], st.cs[3]);
}

__device__ __forceinline__ void stage_store(const Stage& st, f16 (*ks)[kKStride],
                                            f16 (*vts)[kVtStride], const Loader& ld, int tid) {
  *reinterpret_cast<f16x8*>(&ks[ld.krow][ld.kc8]) = st.klo;
  *reinterpret_cast<f16x8*>(&ks[ld.krow][32 + ld.kc8]) = st.khi;
  if (tid < 128) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const f16x4 col4 = {st.v[0][e], st.v[1][e], st.v[2][e], st.v[3][e]};
      *reinterpret_cast<f16x4*>(&vts[ld.vc8 + e][ld.vrow]) = col4;
    }
  }
}

// Rotated K and raw V of a tile into the cache at slots start_pos + key.
__device__ __forceinline__ void stage_append(const Stage& st, const Args& a, int b, int hk,
                                             const Loader& ld, int key0, int tid) {
  const int S = a.S;
  {
    const int key = key0 + ld.krow;
    if (key < S) {
      f16* kd = a.kc + b * a.kc_sb + hk * a.kc_sh + (a.start_pos + key) * a.kc_sn;
      store16(kd + ld.kc8, st.klo);
      store16(kd + 32 + ld.kc8, st.khi);
    }
  }
  if (tid < 128) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = key0 + ld.vrow + r;
      if (key < S)
        store16(a.vc + b * a.vc_sb + hk * a.vc_sh + (a.start_pos + key) * a.vc_sn + ld.vc8, st.v[r]);
    }
  }
}

// Running max is only moved when a tile's max exceeds it by more than this
// many log2 units: until then p = exp2(s - m) <= 2^8 stays exact enough in
// fp16 and the output accumulators need no rescaling (the final division by
// the running sum makes the result independent of the reference point).
constexpr float kRescaleSlack = 8.f;

template <bool kRope, bool kAppend>
__global__ __launch_bounds__(kWaves * 64) void prefill_kernel(Args a) {
  __shared__ __attribute__((aligned(16))) f16 ks[2][kBN][kKStride];
  __shared__ __attribute__((aligned(16))) f16 vts[2][kD][kVtStride];

  const int n_mtiles = gridDim.x;
  const int mt = n_mtiles - 1 - blockIdx.x;  // heaviest tiles first
  const int bq = blockIdx.y;
  const int QH = touch_arg_lines(a.QH, a.q, a.v, a.kc, a.snake);
  const int b = bq / QH, hq = bq % QH;
  const int hk = hq / a.G;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int S = a.S;

  const f16* kb = a.k + b * a.k_sb + hk * a.k_sh;
  const f16* vb = a.v + b * a.v_sb + hk * a.v_sh;
  const int64_t cs_off = b * a.cs_sb;  // this batch row's cos/sin tables
  const bool writer = kAppend && (hq % a.G == 0);
  const int key_end = (mt + 1) * kBM < S ? (mt + 1) * kBM : S;
  const int n_ktiles = (key_end + kBN - 1) / kBN;
  Loader ld;
  ld.krow = tid >> 2;
  ld.kc8 = 8 * (tid & 3);
  ld.vrow = 4 * (tid & 15);
  ld.vc8 = 8 * (tid >> 4);
  ld.kp = kb + ld.krow * a.k_sn + ld.kc8;
  ld.vp = vb + ld.vrow * a.v_sn + ld.vc8;
  ld.cso = cs_off + ld.krow * a.cs_sn + ld.kc8;

  // Tile 0 goes out first; Q is loaded and rotated while it is in flight.
  Stage st;
  stage_load<kRope>(st, a, kb, vb, cs_off, ld, 0, kBN > S, tid);

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

  float m_use = kNegInf, l_run = 0.f;
  f32x4 o[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  stage_rope<kRope>(st);
  if (writer && mt == 0) stage_append(st, a, b, hk, ld, 0, tid);
  stage_store(st, ks[0], vts[0], ld, tid);
  __syncthreads();

  const float ks2 = a.scale_log2;
  for (int kt = 0; kt < n_ktiles; ++kt) {
    const int buf = kt & 1;
    const int key0 = kt * kBN;
    const bool more = kt + 1 < n_ktiles;
    if (more) stage_load<kRope>(st, a, kb, vb, cs_off, ld, key0 + kBN, key0 + 2 * kBN > S, tid);

    // S^T for the whole 64-key tile: block 2*ch + j holds keys
    // key0 + 32*ch + 8*grp + 4*j + i in register i (column = query).
    f32x4 c[4];
#pragma unroll
    for (int ch = 0; ch < 2; ++ch)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int krow = 32 * ch + 8 * (col >> 2) + 4 * j + (col & 3);
        const f16x8 a0 = *reinterpret_cast<const f16x8*>(&ks[buf][krow][8 * grp]);
        const f16x8 a1 = *reinterpret_cast<const f16x8*>(&ks[buf][krow][32 + 8 * grp]);
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        acc = mfma16x16x32(a0, qf[0], acc);
        c[2 * ch + j] = mfma16x16x32(a1, qf[1], acc);
      }
    if (key0 + kBN > mt * kBM || key0 + kBN > S) {  // diagonal or tail tile: mask
#pragma unroll
      for (int blk = 0; blk < 4; ++blk)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = key0 + 32 * (blk >> 1) + 8 * grp + 4 * (blk & 1) + i;
          if (!(key <= qrow && key < S)) c[blk][i] = kNegInf;
        }
    }
    float mx = fmaxf(fmaxf(c[0][0], c[0][1]), fmaxf(c[0][2], c[0][3]));
#pragma unroll
    for (int blk = 1; blk < 4; ++blk)
      mx = fmaxf(mx, fmaxf(fmaxf(c[blk][0], c[blk][1]), fmaxf(c[blk][2], c[blk][3])));
    mx *= ks2;
    // The lane-local max decides (one ballot); the column max over the four
    // lanes sharing a query is only formed on the rare rescale path, so every
    // lane of a column keeps the same reference point.
    if (__any(mx > m_use + kRescaleSlack)) {
      const float m_new = fmaxf(m_use, col_max(mx));
      const float resc = (m_new == kNegInf) ? 1.f : fast_exp2(m_use - m_new);
      l_run *= resc;
#pragma unroll
      for (int t = 0; t < 4; ++t) o[t] *= resc;
      m_use = m_new;
    }
    const float neg_m = (m_use == kNegInf) ? 0.f : -m_use;
    float psum = 0.f;
    f16x8 pb[2];
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = fast_exp2(__builtin_fmaf(c[blk][i], ks2, neg_m));  // 0 for masked keys
        psum += p;
        pb[blk >> 1][4 * (blk & 1) + i] = (f16)p;
      }
    l_run += psum;
#pragma unroll
    for (int ch = 0; ch < 2; ++ch)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const f16x4 va0 = *reinterpret_cast<const f16x4*>(&vts[buf][16 * t + col][32 * ch + 8 * grp]);
        const f16x4 va1 = *reinterpret_cast<const f16x4*>(&vts[buf][16 * t + col][32 * ch + 8 * grp + 4]);
        const f16x8 va = {va0[0], va0[1], va0[2], va0[3], va1[0], va1[1], va1[2], va1[3]};
        o[t] = mfma16x16x32(va, pb[ch], o[t]);
      }
    if (more) {
      stage_rope<kRope>(st);
      if (writer && kt + 1 == mt) stage_append(st, a, b, hk, ld, key0 + kBN, tid);
      stage_store(st, ks[buf ^ 1], vts[buf ^ 1], ld, tid);
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


// ---------------------------------------------------------------------------
// Streaming variant for K/V that are already rotated (and, in the fused op,
// already in the cache): tiles go HBM -> LDS with asynchronous 16-byte
// direct-to-LDS loads (buffer_load ... lds), so no registers stage the data
// and the next tiles are in flight while the current ones are computed.
// LDS rows are
// 128 bytes, XOR-swizzled in 16-byte chunks (chunk c of row r lives at
// c ^ swz(r)).  gfx950's LDS serves 256 bytes per cycle (64 banks of 4
// bytes: a 16-byte read takes 16 lanes at a time).  With
// swz(r) = r1 | r3 << 1 | (r1 ^ r4) << 2 (ri = bit i of r) the 16 lanes of a
// K operand read (rows 8*(c/4) + 4j + c%4, one logical chunk) hit 16
// distinct 16-byte bank groups, i.e. the reads are conflict-free; a swizzle
// that breaks this doubles SQ_LDS_BANK_CONFLICT (measured).  V^T operands come
// from ds_read_b64_tr_b16: within each 16-lane group, lane i receives element
// i % 4 of the 8-byte words addressed by lanes 4t + i/4 (t = 0..3), so lanes
// that address 4 keys x 16 dims of V receive V^T[d][4 keys] directly.
constexpr int kRowBytes = kD * 2;  // 128

__device__ __forceinline__ int swz(int row) {
  const int r1 = (row >> 1) & 1, r3 = (row >> 3) & 1, r4 = (row >> 4) & 1;
  return r1 | (r3 << 1) | ((r1 ^ r4) << 2);
}

typedef __attribute__((address_space(3))) void lds_void;
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// 32-bit LDS address of a pointer into a __shared__ array.
__device__ __forceinline__ unsigned lds_addr(const unsigned char* p) {
  return (unsigned)(uintptr_t)(const lds_void*)p;
}

// LDS operand reads of a tile, written as inline asm.  The tiles arrive by
// LDS DMA (buffer_load ... lds), which the compiler tracks with the vector
// memory counter; it cannot tell that a read of one stage does not alias the
// DMA into another, and before every compiler-visible LDS read it would wait
// for the DMA just issued for the next tiles (vmcnt(0)), which serialises the
// prefetch.  These reads carry no such wait: the barrier of the step orders
// them after their own tile's DMA, and the caller waits for the reads
// themselves (lgkmcnt) before the first use.
template <int kOff>
__device__ __forceinline__ u32x4 lds_read_b128(unsigned addr) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(kOff));
  return r;
}

// ds_read_b64_tr_b16: lane i receives the 16-bit elements that the
// transposed 8-byte reads of its lane group place there (the V^T operand).
template <int kOff>
__device__ __forceinline__ u32x2 lds_read_tr_b64(unsigned addr) {
  u32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(kOff));
  return r;
}

// Per-lane state of the streaming prefill, shared by its tile steps.
struct LdsCtx {
  const f16* kb;
  const f16* vb;
  int kvo[2];         // byte offset, within a tile, of this lane's two K rows' chunk
  int vvo[2];         // same for V
  // Next tile to issue (tiles are issued in increasing order): its first K/V
  // byte and the valid bytes from there to the end of the sequence.
  const unsigned char* knext;
  const unsigned char* vnext;
  int64_t krem, vrem;
  int64_t k_sn, v_sn;
  // Paged caches: tile kt_issue's rows start in the page of slot
  // start + 64 * kt_issue; lane j of `pid` holds the physical page of
  // logical page pwin + j of this row (`trow`), reloaded every 64 pages.
  const unsigned char* kpool;  // pool + kv head offset (bytes)
  const unsigned char* vpool;
  const int32_t* trow;
  int64_t k_sp, v_sp, start;   // page strides (bytes), first slot of the sequence
  int pid, pwin, kt_issue, log2p, ppr, n_pages;
  int S, mt, qrow, grp, lrow0, pch, w;
  // LDS byte offsets of the operand reads for ch = 0, j = 0 (K) and
  // ch = 0, h = 0 (V^T); the other (ch, j / h) add the row offsets
  // (32 ch + 4 j) * 128 (resp. 4 h), which leave the swizzle unchanged, as
  // immediates.
  int koff[2];  // [kk]
  int voff[4];  // [d tile]
  f16x8 qf[2];
  float m_use, ks2;
  f32x4 l4;   // running sum of p per query column, kept by an MFMA against ones
  f32x4 o[4];
};

// Buffer resource over `rem` valid bytes from `base` (a tile's first row):
// the tile's address and valid byte count live in SGPRs, so a lane's load
// offset within the tile never changes, and rows past the sequence (the last
// tile's tail) read as zero (their scores are masked).  Needs row strides
// >= 64 elements so a row's 128 bytes lie below the record count.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const unsigned char* base, int64_t rem) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(base), (short)0,
                                           (int)(rem < 0x7fffffff ? rem : 0x7fffffff), 0x00020000);
}

// Physical pages of logical pages [win, win + 64) of the row into lane j,
// clamped to the row's table and to the pool.
__device__ __forceinline__ void load_pids(LdsCtx& c, int win) {
  int j = win + (threadIdx.x & 63);
  j = j < c.ppr ? j : c.ppr - 1;
  const int p = c.trow[j];
  c.pid = min(max(p, 0), c.n_pages - 1);
  c.pwin = win;
}

// Async loads of the next tile (this wave's 16 rows of K and of V) into
// (Kd, Vd); advances the issue cursor by kAdv tiles (scalar adds only).  Paged
// caches: the tile's rows lie in one page (start and the page size are
// multiples of 64), whose base comes from the page ids held in `pid`.
template <bool kPaged, int kAdv = 1>
__device__ __forceinline__ void lds_issue(LdsCtx& c, unsigned char* Kd, unsigned char* Vd) {
  if (kPaged) {
    const int64_t slot0 = c.start + (int64_t)c.kt_issue * kBN;
    const int lp = (int)(slot0 >> c.log2p);
    if (lp - c.pwin >= 64) load_pids(c, lp);
    const int page = __builtin_amdgcn_readlane(c.pid, lp - c.pwin);
    const int64_t row = slot0 & ((1 << c.log2p) - 1);
    c.knext = c.kpool + (int64_t)page * c.k_sp + row * c.k_sn * 2;
    c.vnext = c.vpool + (int64_t)page * c.v_sp + row * c.v_sn * 2;
    c.kt_issue += kAdv;
  }
  const __amdgpu_buffer_rsrc_t rk = tile_rsrc(c.knext, c.krem);
  const __amdgpu_buffer_rsrc_t rv = tile_rsrc(c.vnext, c.vrem);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(Kd + (16 * c.w + 8 * i) * kRowBytes),
                                             16, c.kvo[i], 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(Vd + (16 * c.w + 8 * i) * kRowBytes),
                                             16, c.vvo[i], 0, 0, 0);
  }
  const int64_t kstep = kAdv * kBN * c.k_sn * 2, vstep = kAdv * kBN * c.v_sn * 2;
  c.knext += kstep;
  c.vnext += vstep;
  c.krem -= kstep;
  c.vrem -= vstep;
}

// v_max3_f32 on raw registers.  fmaxf would first canonicalise the MFMA
// results (v_max_f32 x, x per operand: IEEE mode quiets signalling NaNs); the
// scores here are finite or -inf, so the plain three-input max is exact.
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Max of a lane's 16 scores: a depth-3 tree of seven max3.  The hazard
// recognizer does not look into inline asm, so it would insert no wait
// states between the score MFMAs and an asm read of their results: the
// s_nops, tied to all sixteen score registers (every max3 depends on them,
// and they on the MFMAs), give a matrix-core result the 16 wait states it
// may need before a VALU read, however close the scheduler puts the max.
__device__ __forceinline__ float max16(f32x4 (&sc)[4]) {
  asm volatile("s_nop 7\n\ts_nop 7" : "+v"(sc[0]), "+v"(sc[1]), "+v"(sc[2]), "+v"(sc[3]));
  const float a = max3_raw(sc[0][0], sc[0][1], sc[0][2]);
  const float b = max3_raw(sc[0][3], sc[1][0], sc[1][1]);
  const float d = max3_raw(sc[1][2], sc[1][3], sc[2][0]);
  const float e = max3_raw(sc[2][1], sc[2][2], sc[2][3]);
  const float f = max3_raw(sc[3][0], sc[3][1], sc[3][2]);
  return max3_raw(max3_raw(a, b, d), max3_raw(e, f, sc[3][3]), kNegInf);
}

// Scores, online softmax and PV of key tile kt from the LDS stage (Ks, Vs),
// whose loads have landed; `refill` runs once the K operands are in
// registers (the V^T reads come later).
template <typename Refill>
__device__ __forceinline__ void tile_compute(LdsCtx& c, int kt, const unsigned char* Ks,
                                             const unsigned char* Vs, Refill&& refill) {
  const int key0 = kt * kBN;
  // K operands of tile kt, then (in flight under the score MFMAs and the
  // softmax) its V^T operands.
  const unsigned ks = lds_addr(Ks), vs = lds_addr(Vs);
  u32x4 kr[2][2][2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const unsigned ka0 = ks + c.koff[kk];
    kr[0][0][kk] = lds_read_b128<0>(ka0);
    kr[0][1][kk] = lds_read_b128<4 * kRowBytes>(ka0);
    kr[1][0][kk] = lds_read_b128<32 * kRowBytes>(ka0);
    kr[1][1][kk] = lds_read_b128<36 * kRowBytes>(ka0);
  }
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(kr[0][0][0]), "+v"(kr[0][0][1]), "+v"(kr[0][1][0]), "+v"(kr[0][1][1]),
                 "+v"(kr[1][0][0]), "+v"(kr[1][0][1]), "+v"(kr[1][1][0]), "+v"(kr[1][1][1]));
  u32x2 vr[2][4][2];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const unsigned va0 = vs + c.voff[t];
    vr[0][t][0] = lds_read_tr_b64<0>(va0);
    vr[0][t][1] = lds_read_tr_b64<4 * kRowBytes>(va0);
    vr[1][t][0] = lds_read_tr_b64<32 * kRowBytes>(va0);
    vr[1][t][1] = lds_read_tr_b64<36 * kRowBytes>(va0);
  }
  f16x8 ka[2][2][2];
#pragma unroll
  for (int ch = 0; ch < 2; ++ch)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) ka[ch][j][kk] = __builtin_bit_cast(f16x8, kr[ch][j][kk]);
  // Refill after the K operands are in registers (the V^T reads come later).
  refill();
  f32x4 sc[4];
#pragma unroll
  for (int ch = 0; ch < 2; ++ch)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      acc = mfma16x16x32(ka[ch][j][0], c.qf[0], acc);
      sc[2 * ch + j] = mfma16x16x32(ka[ch][j][1], c.qf[1], acc);
    }
  if (key0 + kBN > c.mt * kBM || key0 + kBN > c.S) {  // diagonal or tail tile: mask
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = key0 + 32 * (blk >> 1) + 8 * c.grp + 4 * (blk & 1) + i;
        if (!(key <= c.qrow && key < c.S)) sc[blk][i] = kNegInf;
      }
  }
  float mx = max16(sc);
  mx *= c.ks2;
  if (__any(mx > c.m_use + kRescaleSlack)) {
    const float m_new = fmaxf(c.m_use, col_max(mx));
    const float resc = (m_new == kNegInf) ? 1.f : fast_exp2(c.m_use - m_new);
    c.l4 *= resc;
#pragma unroll
    for (int t = 0; t < 4; ++t) c.o[t] *= resc;
    c.m_use = m_new;
  }
  const float neg_m = (c.m_use == kNegInf) ? 0.f : -c.m_use;
  f16x8 pb[2];
#pragma unroll
  for (int blk = 0; blk < 4; ++blk)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = fast_exp2(__builtin_fmaf(sc[blk][i], c.ks2, neg_m));  // 0 for masked keys
      pb[blk >> 1][4 * (blk & 1) + i] = (f16)p;
    }
  // Row sums of P^T on the matrix core: ones x P^T puts sum_k p[k][q] in every
  // row of column q, already reduced over the four lanes of the column, and
  // over the same fp16 p the PV product uses.
  const f16x8 ones = {(f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f};
  c.l4 = mfma16x16x32(ones, pb[0], c.l4);
  c.l4 = mfma16x16x32(ones, pb[1], c.l4);
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(vr[0][0][0]), "+v"(vr[0][0][1]), "+v"(vr[0][1][0]), "+v"(vr[0][1][1]),
                 "+v"(vr[0][2][0]), "+v"(vr[0][2][1]), "+v"(vr[0][3][0]), "+v"(vr[0][3][1]),
                 "+v"(vr[1][0][0]), "+v"(vr[1][0][1]), "+v"(vr[1][1][0]), "+v"(vr[1][1][1]),
                 "+v"(vr[1][2][0]), "+v"(vr[1][2][1]), "+v"(vr[1][3][0]), "+v"(vr[1][3][1]));
#pragma unroll
  for (int ch = 0; ch < 2; ++ch)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const f16x4 lo = __builtin_bit_cast(f16x4, vr[ch][t][0]);
      const f16x4 hi = __builtin_bit_cast(f16x4, vr[ch][t][1]);
      const f16x8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      c.o[t] = mfma16x16x32(va, pb[ch], c.o[t]);
    }
}

// Grouped form: one workgroup of 4 kG waves per query tile.  Wave group g
// (waves 4g .. 4g + 3) takes key tiles g, g + kG, ..., each group a copy of
// the four-wave pipeline (16 query rows per wave, the same tile_compute), on
// a two-stage LDS ring that holds every group's tile of a step: the loads of
// step i + 1 are issued after step i's barrier, when every wave is done with
// step i - 1's stage.  At the end groups 1 .. kG-1 hand their softmax states
// to group 0 through LDS, which merges them.  The heaviest query tile takes
// 1/kG of the steps, with no partial or merge through memory.  kG = 2: two
// workgroups per CU; kG = 4: one (both four waves per SIMD).
constexpr int kTileBytes = kBN * kRowBytes;

template <int kG, bool kRopeQ, bool kPaged>
__global__ __launch_bounds__(kG * 4 * 64, 4) void prefill_lds2_kernel(Args a) {
  __shared__ __attribute__((aligned(16))) unsigned char ring[2][kG][2][kTileBytes];  // [stage][group][K, V]
  // Rotated Q fragments, formed once per workgroup by group 0 and read by the
  // other groups (same 16 rows per wave index, same lane layout).  Every wave
  // group loading Q and its cos/sin rows itself doubles the requests of the
  // start-up burst, when all workgroups load at once and the 14 heads'
  // workgroups of a query tile read the same table rows: measured 1.1 µs of a
  // 24 µs call at S=2048, outputs bit-identical.
  constexpr bool kShareQ = kRopeQ && kG > 1;
  __shared__ __attribute__((aligned(16))) f16x8 qsh[kShareQ ? 4 : 1][2][64];  // [w][half][lane]

  // One-dimensional grid, (query tile, b * QH + q head) with the head
  // fastest and the heaviest query tiles first.
  const int n_bq = touch_arg_lines(a.B, a.q, a.v, a.kc, a.snake) * a.QH;
  const int n_mtiles = (a.S + kBM - 1) / kBM;
  // Item (query tile, head) of this workgroup; items are numbered heaviest
  // first.  With a second round (a.snake = CUs, P = grid - CUs workgroups past
  // one per CU): the first round's last CUs - P workgroups, whose CUs get no
  // second one, take the heaviest items; its first P take the next ones; the
  // second round takes the rest lightest first, so workgroup CUs + j meets
  // the item of workgroup j on its CU.
  int item = (int)blockIdx.x;
  if (a.snake > 0) {
    const int T = (int)gridDim.x, P = T - a.snake, H = a.snake - P;
    if (item >= a.snake) item = T - 1 - (item - a.snake);
    else item = item < P ? H + item : item - P;
  }
  const int mt = n_mtiles - 1 - item / n_bq;
  const int bq = item % n_bq;
  const int b = bq / a.QH, hq = bq % a.QH;
  const int hk = hq / a.G;
  const int tid = threadIdx.x;
  // Wave-uniform (scalar) group and row block: the group picks the tiles'
  // addresses, which buffer resources need in scalar registers.
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = wave >> 2;  // key tiles g, g + kG, ...
  const int w = wave & 3;   // 16-row block of the query tile
  const int col = lane & 15, grp = lane >> 4;
  int S;
  int64_t tok0;
  row_span(a, b, S, tok0);
  if (mt * kBM >= S) return;  // a shorter packed row: this query tile is empty
  const int key_end = (mt + 1) * kBM < S ? (mt + 1) * kBM : S;
  const int n_all = (key_end + kBN - 1) / kBN;
  const int n_steps = (n_all + kG - 1) / kG;
  const int n_mine = (n_all - g + kG - 1) / kG;

  LdsCtx c;
  const int64_t kvt = a.kv_packed ? tok0 : 0;
  c.kb = a.k + b * a.k_sb + kvt * a.k_sn + hk * a.k_sh;
  c.vb = a.v + b * a.v_sb + kvt * a.v_sn + hk * a.v_sh;
  c.k_sn = a.k_sn;
  c.v_sn = a.v_sn;
  c.S = S;
  c.mt = mt;
  c.grp = grp;
  c.w = w;
  c.qrow = mt * kBM + w * 16 + col;
  c.lrow0 = 16 * w + (lane >> 3);
  c.pch = lane & 7;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = c.lrow0 + 8 * i;
    const int ch = c.pch ^ swz(r);
    c.kvo[i] = (int)(r * c.k_sn * 2) + 16 * ch;
    c.vvo[i] = (int)(r * c.v_sn * 2) + 16 * ch;
  }

  // ---- Q^T operand (16 rows per wave), rotated in registers; loads go first.
  const bool qload = !kShareQ || g == 0;
  f16x8 qcs[4];
  if (qload) {
    const int qr = c.qrow < S ? c.qrow : S - 1;
    const f16* qp = a.q + b * a.q_sb + hq * a.q_sh + (tok0 + qr) * a.q_sn + 8 * grp;
    c.qf[0] = load16(qp);
    c.qf[1] = load16(qp + 32);
    if (kRopeQ) {
      const int64_t co = b * a.cs_sb + (tok0 + qr) * a.cs_sn + 8 * grp;
      qcs[0] = load16(a.cos + co);
      qcs[1] = load16(a.sin + co);
      qcs[2] = load16(a.cos + co + 32);
      qcs[3] = load16(a.sin + co + 32);
    }
  }
  c.knext = reinterpret_cast<const unsigned char*>(c.kb + (int64_t)g * kBN * c.k_sn);
  c.vnext = reinterpret_cast<const unsigned char*>(c.vb + (int64_t)g * kBN * c.v_sn);
  c.krem = (int64_t)(S - g * kBN) * c.k_sn * 2;
  c.vrem = (int64_t)(S - g * kBN) * c.v_sn * 2;
  if (kPaged) {
    c.kpool = reinterpret_cast<const unsigned char*>(a.k + hk * a.k_sh);
    c.vpool = reinterpret_cast<const unsigned char*>(a.v + hk * a.v_sh);
    c.trow = a.table + b * a.t_sb;
    c.k_sp = a.k_sb * 2;
    c.v_sp = a.v_sb * 2;
    c.start = a.start_pos;
    c.log2p = a.log2p;
    c.ppr = a.ppr;
    c.n_pages = a.n_pages;
    c.kt_issue = g;
    load_pids(c, (int)((a.start_pos + (int64_t)g * kBN) >> a.log2p));
  }
  if (n_mine > 0) lds_issue<kPaged, kG>(c, ring[0][g][0], ring[0][g][1]);  // tile g
  if (kRopeQ && qload) rope_pair(c.qf[0], c.qf[1], qcs[0], qcs[1], qcs[2], qcs[3]);
  if (kShareQ) {
    // Before the loop's first barrier; the tile loads are already in flight.
    if (g == 0) {
      qsh[w][0][lane] = c.qf[0];
      qsh[w][1][lane] = c.qf[1];
    }
    __syncthreads();
    if (g > 0) {
      c.qf[0] = qsh[w][0][lane];
      c.qf[1] = qsh[w][1][lane];
    }
  }
  {
    const int rk = 8 * (col >> 2) + (col & 3);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) c.koff[kk] = rk * kRowBytes + 16 * ((grp + 4 * kk) ^ swz(rk));
    const int rv = 8 * grp + (col >> 2);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int d = 16 * t + 4 * (col & 3);
      c.voff[t] = rv * kRowBytes + 16 * ((d >> 3) ^ swz(rv)) + 2 * (d & 7);
    }
  }
  c.m_use = kNegInf;
  c.l4 = f32x4{0.f, 0.f, 0.f, 0.f};
  c.ks2 = a.scale_log2;
#pragma unroll
  for (int t = 0; t < 4; ++t) c.o[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int i = 0; i < n_steps; ++i) {
    // This wave's loads of step i have landed; after the barrier every
    // wave's have, and every wave is done with step i - 1's stage, which
    // takes step i + 1's tiles.  (A group without a tile in the last step
    // still takes part in the barrier.)
    s_waitcnt_vm(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (i < n_mine) {
      const int st = i & 1;
      tile_compute(c, kG * i + g, ring[st][g][0], ring[st][g][1], [&] {
        if (i + 1 < n_mine) lds_issue<kPaged, kG>(c, ring[st ^ 1][g][0], ring[st ^ 1][g][1]);
      });
    }
  }

  // Merge the groups: groups 1 .. kG-1 write (o, m, l) to LDS (the ring is
  // free once every wave is past its last step), group 0 merges them.
  float l_run = c.l4[0];
  f32x4* sm_o = reinterpret_cast<f32x4*>(&ring[0][0][0][0]);  // [g-1][w][t][lane]
  float* sm_ml = reinterpret_cast<float*>(&ring[0][0][0][0] + (kG - 1) * 4 * 4 * 64 * 16);  // [g-1][w][lane][m, l]
  __syncthreads();
  if (g > 0) {
    const int slot = (g - 1) * 4 + w;
#pragma unroll
    for (int t = 0; t < 4; ++t) sm_o[(slot * 4 + t) * 64 + lane] = c.o[t];
    sm_ml[(slot * 64 + lane) * 2] = c.m_use;
    sm_ml[(slot * 64 + lane) * 2 + 1] = l_run;
  }
  __syncthreads();
  if (g > 0 || c.qrow >= S) return;
  float mg[kG], lg[kG];
  mg[0] = c.m_use;
  lg[0] = l_run;
  float mn = c.m_use;
#pragma unroll
  for (int gg = 1; gg < kG; ++gg) {
    const int slot = (gg - 1) * 4 + w;
    mg[gg] = sm_ml[(slot * 64 + lane) * 2];
    lg[gg] = sm_ml[(slot * 64 + lane) * 2 + 1];
    mn = fmaxf(mn, mg[gg]);
  }
  float sg[kG], l_tot = 0.f;
#pragma unroll
  for (int gg = 0; gg < kG; ++gg) {
    sg[gg] = (mg[gg] == kNegInf) ? 0.f : fast_exp2(mg[gg] - mn);
    l_tot += lg[gg] * sg[gg];
  }
  const float inv = 1.f / l_tot;
  f16* op = a.out + b * a.o_sb + hq * a.o_sh + (tok0 + c.qrow) * a.o_sn;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    f32x4 o = c.o[t] * sg[0];
#pragma unroll
    for (int gg = 1; gg < kG; ++gg) o += sm_o[((((gg - 1) * 4 + w) * 4) + t) * 64 + lane] * sg[gg];
    f16x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = (f16)(o[i] * inv);
    *reinterpret_cast<f16x4*>(op + 16 * t + 4 * grp) = r;
  }
}

// Pre-pass of the cached prefill: rotated K (or K as is) and raw V of every
// token into the cache at slot start_pos + token, once per (b, kv head);
// 16 tokens per workgroup, 16 threads per token (4 for K's rotate-half chunk
// pairs, 8 for V's chunks).
__global__ __launch_bounds__(256) void rope_kv_prefill_kernel(Args a) {
  const int tok = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  const int bh = blockIdx.y;
  const int KVH = touch_arg_lines(a.KVH, a.k, a.v, a.kc, a.cu);
  const int b = bh / KVH, h = bh % KVH;
  int S;
  int64_t tok0;
  row_span(a, b, S, tok0);
  if (tok >= S || sub >= 12) return;
  const int64_t slot = a.start_pos + tok;
  const int64_t t = tok0 + tok;  // packed token index (== tok for equal-length rows)
  bool ok;
  if (sub < 4) {
    const f16* src = a.k + b * a.k_sb + h * a.k_sh + t * a.k_sn + 8 * sub;
    f16x8 lo = load16(src), hi = load16(src + 32);
    if (a.cos != nullptr) {
      const int64_t co = b * a.cs_sb + t * a.cs_sn + 8 * sub;
      rope_pair(lo, hi, load16(a.cos + co), load16(a.sin + co), load16(a.cos + co + 32),
                load16(a.sin + co + 32));
    }
    f16* dst = a.kc + cache_row(a, b, slot, a.kc_sb, a.kc_sn, ok) + h * a.kc_sh + 8 * sub;
    if (ok) {
      store16(dst, lo);
      store16(dst + 32, hi);
    }
  } else {
    const int c = sub - 4;
    const f16x8 val = load16(a.v + b * a.v_sb + h * a.v_sh + t * a.v_sn + 8 * c);
    f16* dst = a.vc + cache_row(a, b, slot, a.vc_sb, a.vc_sn, ok) + h * a.vc_sh + 8 * c;
    if (ok) store16(dst, val);
  }
}

}  // namespace prefill
}  // namespace qf

using namespace qf;

static bool aligned16p(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

using qf::prefill::Args;

// Shared launch sequence of the dense and the packed (varlen) entry points;
// `a` is filled and validated.  Returns 0 or a QF_ERR_* / hipError_t code.
// CUs of the device that owns `st` (cached per device); 0 if it cannot be read.
static int stream_cus(hipStream_t st) {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];
  int dev = -1;
  if (st == nullptr) {
    if (hipGetDevice(&dev) != hipSuccess) return 0;
  } else {
    hipDevice_t d = -1;
    if (hipStreamGetDevice(st, &d) != hipSuccess) return 0;
    dev = (int)d;
  }
  if (dev < 0 || dev >= kMaxDevices) return 0;
  int cus = cached[dev].load(std::memory_order_relaxed);
  if (cus == 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus < 0)
      return 0;
    cached[dev].store(cus, std::memory_order_relaxed);
  }
  return cus;
}

static int prefill_launch(Args a, bool rope, bool append, hipStream_t st) {
  using namespace qf::prefill;
  const int B = a.B, QH = a.QH, KVH = a.KVH, S = a.S;
  // The streaming kernel addresses a tile's rows with 32-bit byte offsets and
  // bounds them by the record count of a buffer resource; check its source
  // (the cache when appending) before anything is launched.
  const int64_t ksn = append ? a.kc_sn : a.k_sn, vsn = append ? a.vc_sn : a.v_sn;
  if (!(rope && !append) &&
      (ksn < kD || vsn < kD || ksn * 2 * kBN > 0x7fffffff || vsn * 2 * kBN > 0x7fffffff))
    return QF_ERR_UNSUPPORTED;
  dim3 grid((S + kBM - 1) / kBM, B * QH), block(kWaves * 64);
  if (rope && !append) {
    // No cache to hold the rotated keys: rotate K in registers tile by tile.
    if (a.cu != nullptr) return QF_ERR_UNSUPPORTED;
    hipLaunchKernelGGL((prefill_kernel<true, false>), grid, block, 0, st, a);
    return (int)hipGetLastError();
  }
  const bool paged = a.table != nullptr;
  if (append) {
    // Pre-pass: rotated K (or K as is) and V into the cache; then stream the
    // finished rows back from the cache (paged: the kernel finds each tile's
    // page from start_pos and the block table).
    hipLaunchKernelGGL(rope_kv_prefill_kernel, dim3((S + 15) / 16, B * KVH), dim3(256), 0, st, a);
    a.k = a.kc + (paged ? 0 : a.start_pos * a.kc_sn);
    a.k_sb = a.kc_sb; a.k_sh = a.kc_sh; a.k_sn = a.kc_sn;
    a.v = a.vc + (paged ? 0 : a.start_pos * a.vc_sn);
    a.v_sb = a.vc_sb; a.v_sh = a.vc_sh; a.v_sn = a.vc_sn;
    a.kv_packed = 0;
  } else if (paged) {
    return QF_ERR_INVALID_ARG;  // paged prefill always appends
  }
  // One eight-wave workgroup per (query tile, b * QH + q head).
  if ((int64_t)grid.x * B * QH > 0x7fffffff) return QF_ERR_UNSUPPORTED;
  const dim3 lgrid((unsigned)(grid.x * B * QH));
  // Two groups (measured on MI355X: four, one 16-wave workgroup per CU,
  // were slower at every size, 28.8 vs 26.0 us at S=2048).
  constexpr int G = 2;
  const dim3 lblock(G * 4 * 64);
  // Two workgroups fit a CU.  When the grid needs more than one per CU but
  // no more than two, the first round (one per CU) shares most CUs with a
  // second-round workgroup.  The heaviest query tiles go to the CUs that get
  // none, the next ones are paired with the lightest (the second round runs
  // lightest first), whose short lives slow the long ones least.  Measured on
  // MI355X, same outputs, against heaviest-first throughout: S=2048 call 23.4
  // -> 22.9 us, S=1536 18.8 -> 18.6, S=2304 26.1 -> 25.45 with the pairing;
  // the unpaired heaviest tiles take about 0.1 us more off the attention.
  a.snake = 0;
  {
    const int cus = stream_cus(st);
    if (cus > 0 && lgrid.x > (unsigned)cus && lgrid.x <= 2u * (unsigned)cus) a.snake = cus;
  }
  if (paged) {
    if (rope) hipLaunchKernelGGL((prefill_lds2_kernel<G, true, true>), lgrid, lblock, 0, st, a);
    else hipLaunchKernelGGL((prefill_lds2_kernel<G, false, true>), lgrid, lblock, 0, st, a);
  } else {
    if (rope) hipLaunchKernelGGL((prefill_lds2_kernel<G, true, false>), lgrid, lblock, 0, st, a);
    else hipLaunchKernelGGL((prefill_lds2_kernel<G, false, false>), lgrid, lblock, 0, st, a);
  }
  return (int)hipGetLastError();
}

static int fill_common(Args& a, const void* q, const void* k, const void* v, const void* cos,
                       const void* sin, void* k_cache, int64_t kc_sb, int64_t kc_sh, int64_t kc_sn,
                       void* v_cache, int64_t vc_sb, int64_t vc_sh, int64_t vc_sn,
                       int64_t start_pos, int cap, void* out, int B, int QH, int KVH, int S,
                       int D, float scale, bool& rope, bool& append) {
  using namespace qf::prefill;
  if (D != kD) return QF_ERR_UNSUPPORTED;
  if (!q || !k || !v || !out) return QF_ERR_INVALID_ARG;
  if (B < 1 || KVH < 1 || QH < KVH || QH % KVH != 0 || S < 1) return QF_ERR_INVALID_ARG;
  if ((int64_t)B * QH > 65535) return QF_ERR_INVALID_ARG;
  rope = cos != nullptr || sin != nullptr;
  if (rope && (!cos || !sin)) return QF_ERR_INVALID_ARG;
  append = k_cache != nullptr || v_cache != nullptr;
  if (append && (!k_cache || !v_cache)) return QF_ERR_INVALID_ARG;
  if (append && (start_pos < 0 || start_pos + S > cap)) return QF_ERR_INVALID_ARG;
  if (!aligned16p(q) || !aligned16p(k) || !aligned16p(v)) return QF_ERR_INVALID_ARG;
  if ((reinterpret_cast<uintptr_t>(out) & 7u)) return QF_ERR_INVALID_ARG;
  if (rope && (!aligned16p(cos) || !aligned16p(sin))) return QF_ERR_INVALID_ARG;
  if (append && (!aligned16p(k_cache) || !aligned16p(v_cache) ||
                 ((kc_sb | kc_sh | kc_sn | vc_sb | vc_sh | vc_sn) & 7)))
    return QF_ERR_INVALID_ARG;
  a.q = static_cast<const f16*>(q);
  a.k = static_cast<const f16*>(k);
  a.v = static_cast<const f16*>(v);
  a.cos = static_cast<const f16*>(cos);
  a.sin = static_cast<const f16*>(sin);
  a.kc = static_cast<f16*>(k_cache);
  a.kc_sb = kc_sb; a.kc_sh = kc_sh; a.kc_sn = kc_sn;
  a.vc = static_cast<f16*>(v_cache);
  a.vc_sb = vc_sb; a.vc_sh = vc_sh; a.vc_sn = vc_sn;
  a.start_pos = start_pos;
  a.out = static_cast<f16*>(out);
  a.B = B; a.QH = QH; a.KVH = KVH; a.G = QH / KVH; a.S = S;
  a.scale_log2 = scale * kLog2e;
  a.cu = nullptr;
  a.total = 0;
  a.kv_packed = 1;
  a.table = nullptr;
  a.t_sb = 0;
  a.log2p = 0;
  a.n_pages = 0;
  a.ppr = 0;
  return QF_OK;
}

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
  Args a;
  bool rope, append;
  const int rc = fill_common(a, q, k, v, cos, sin, k_cache, kc_sb, kc_sh, kc_sn, v_cache, vc_sb,
                             vc_sh, vc_sn, start_pos, cap, out, B, QH, KVH, S, D, scale, rope,
                             append);
  if (rc != QF_OK) return rc;
  if ((q_sb | q_sh | q_sn | k_sb | k_sh | k_sn | v_sb | v_sh | v_sn) & 7) return QF_ERR_INVALID_ARG;
  if ((o_sb | o_sh | o_sn) & 3) return QF_ERR_INVALID_ARG;
  if (rope && ((cs_sb | cs_sn) & 7)) return QF_ERR_INVALID_ARG;
  a.q_sb = q_sb; a.q_sh = q_sh; a.q_sn = q_sn;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_sn = k_sn;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_sn = v_sn;
  a.cs_sb = cs_sb; a.cs_sn = cs_sn;
  a.o_sb = o_sb; a.o_sh = o_sh; a.o_sn = o_sn;
  return prefill_launch(a, rope, append, static_cast<hipStream_t>(stream));
}

extern "C" int qf_prefill_varlen(const void* q, int64_t q_sh, int64_t q_sn,
                                 const void* k, int64_t k_sh, int64_t k_sn,
                                 const void* v, int64_t v_sh, int64_t v_sn,
                                 const int32_t* cu_seqlens, int total, int max_seqlen,
                                 const void* cos, const void* sin, int64_t cs_sn,
                                 void* k_cache, int64_t kc_sb, int64_t kc_sh, int64_t kc_sn,
                                 void* v_cache, int64_t vc_sb, int64_t vc_sh, int64_t vc_sn,
                                 int64_t start_pos, int cap,
                                 void* out, int64_t o_sh, int64_t o_sn,
                                 int B, int QH, int KVH, int D, float scale, void* stream) {
  using namespace qf::prefill;
  if (!cu_seqlens || total < 1) return QF_ERR_INVALID_ARG;
  Args a;
  bool rope, append;
  const int rc = fill_common(a, q, k, v, cos, sin, k_cache, kc_sb, kc_sh, kc_sn, v_cache, vc_sb,
                             vc_sh, vc_sn, start_pos, cap, out, B, QH, KVH, max_seqlen, D, scale,
                             rope, append);
  if (rc != QF_OK) return rc;
  if (rope && !append) return QF_ERR_UNSUPPORTED;  // rotated keys need the cache
  if ((q_sh | q_sn | k_sh | k_sn | v_sh | v_sn) & 7) return QF_ERR_INVALID_ARG;
  if ((o_sh | o_sn) & 3) return QF_ERR_INVALID_ARG;
  if (rope && (cs_sn & 7)) return QF_ERR_INVALID_ARG;
  a.q_sb = 0; a.q_sh = q_sh; a.q_sn = q_sn;
  a.k_sb = 0; a.k_sh = k_sh; a.k_sn = k_sn;
  a.v_sb = 0; a.v_sh = v_sh; a.v_sn = v_sn;
  a.cs_sb = 0; a.cs_sn = cs_sn;
  a.o_sb = 0; a.o_sh = o_sh; a.o_sn = o_sn;
  a.cu = cu_seqlens;
  a.total = total;
  return prefill_launch(a, rope, append, static_cast<hipStream_t>(stream));
}

extern "C" int qf_prefill_varlen_paged(const void* q, int64_t q_sh, int64_t q_sn,
                                       const void* k, int64_t k_sh, int64_t k_sn,
                                       const void* v, int64_t v_sh, int64_t v_sn,
                                       const int32_t* cu_seqlens, int total, int max_seqlen,
                                       const void* cos, const void* sin, int64_t cs_sn,
                                       void* k_pool, int64_t kp_sp, int64_t kp_sh, int64_t kp_sn,
                                       void* v_pool, int64_t vp_sp, int64_t vp_sh, int64_t vp_sn,
                                       const int32_t* block_table, int64_t bt_sb,
                                       int pages_per_row, int n_pages, int page_size,
                                       int64_t start_pos,
                                       void* out, int64_t o_sh, int64_t o_sn,
                                       int B, int QH, int KVH, int D, float scale, void* stream) {
  using namespace qf::prefill;
  const int l2 = page_log2(page_size, pages_per_row, n_pages);
  if (l2 < 0) return QF_ERR_UNSUPPORTED;
  if (!cu_seqlens || total < 1 || !block_table || !k_pool || !v_pool) return QF_ERR_INVALID_ARG;
  if (bt_sb < pages_per_row || start_pos % kBN != 0) return QF_ERR_INVALID_ARG;
  Args a;
  bool rope, append;
  const int rc = fill_common(a, q, k, v, cos, sin, k_pool, kp_sp, kp_sh, kp_sn, v_pool, vp_sp,
                             vp_sh, vp_sn, start_pos, pages_per_row * page_size, out, B, QH, KVH,
                             max_seqlen, D, scale, rope, append);
  if (rc != QF_OK) return rc;
  if ((q_sh | q_sn | k_sh | k_sn | v_sh | v_sn) & 7) return QF_ERR_INVALID_ARG;
  if ((o_sh | o_sn) & 3) return QF_ERR_INVALID_ARG;
  if (rope && (cs_sn & 7)) return QF_ERR_INVALID_ARG;
  a.q_sb = 0; a.q_sh = q_sh; a.q_sn = q_sn;
  a.k_sb = 0; a.k_sh = k_sh; a.k_sn = k_sn;
  a.v_sb = 0; a.v_sh = v_sh; a.v_sn = v_sn;
  a.cs_sb = 0; a.cs_sn = cs_sn;
  a.o_sb = 0; a.o_sh = o_sh; a.o_sn = o_sn;
  a.cu = cu_seqlens;
  a.total = total;
  a.table = block_table;
  a.t_sb = bt_sb;
  a.log2p = l2;
  a.n_pages = n_pages;
  a.ppr = pages_per_row;
  return prefill_launch(a, rope, append, static_cast<hipStream_t>(stream));
}
