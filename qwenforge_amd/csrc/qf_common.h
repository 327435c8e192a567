// Shared device helpers for the gfx950 attention kernels.
//
// Matrix-core convention used by every kernel in this library: scores are
// computed transposed, S^T = K * Q^T, and the output as O^T = V^T * P^T, with
// v_mfma_f32_16x16x32_f16.  Its operand layouts (wave64) are
//   A (16 x 32):  lane l holds A[l % 16][8*(l/16) .. 8*(l/16)+7]
//   B (32 x 16):  lane l holds B[8*(l/16) .. 8*(l/16)+7][l % 16]
//   C (16 x 16):  lane l holds C[4*(l/16) + i][l % 16], i = 0..3
// so the query index is always the lane's column (l % 16): the softmax
// statistics of a query live in the four lanes {c, c+16, c+32, c+48}, and the
// probabilities produced as a C tile feed the P^T operand of the next MFMA
// without any data movement (see the key permutation in the kernels).
#pragma once

#include <cstddef>
#include <initializer_list>

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qf {

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ f16x8 load16(const f16* p) {
  return *reinterpret_cast<const f16x8*>(p);
}

// 16-byte non-temporal load (the nt cache policy), for data a launch reads
// exactly once: KV-cache tiles in decode, streamed weights.
__device__ __forceinline__ f16x8 load16_nt(const f16* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(p));
}

__device__ __forceinline__ void store16(f16* p, f16x8 v) {
  *reinterpret_cast<f16x8*>(p) = v;
}

// Cache policy bits of a buffer access that match a relaxed agent-scope
// atomic load / store on gfx950 (sc1: write-through, L2-bypassing), for data
// exchanged between workgroups of one launch (possibly on different XCDs).
constexpr int kSc1 = 16;

// Buffer resource over `bytes` bytes at `base`: accesses past the end read 0
// and write nothing.  The resource lives in SGPRs, so `base` must be
// wave-uniform; lane-dependent parts go in the access offset.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                           (int)(bytes < 0x7fffffff ? bytes : 0x7fffffff),
                                           0x00020000);
}

// Returns x after taking the fields f... as SGPR inputs of one empty asm:
// their scalar loads are issued together and waited for once, before x's
// first use.  A kernel passes a value it needs at once as x and, from every
// other 64-byte line of its argument block that it reads, a field it uses
// early (covers_lines checks the choice), plus any further field its first
// data loads depend on (each later field load waits for a scalar-cache hit).
// Left to the compiler, a field is loaded where it is first used -- behind a
// branch, or after an earlier wait -- and the first load from each line
// misses the scalar cache: one more dependent memory round trip before the
// kernel's first data load.  After the batch the touched fields sit in SGPRs
// and the rest of their lines in the scalar cache.  The asm is not volatile
// and has an output, so it has no side effects: a volatile one counts as a
// possible memory write, after which the compiler reads uniform global data
// (a bound such as kv_last) with vector instead of scalar loads.  One asm for
// all fields: chained ones let the scheduler interleave the loads with waits.
template <typename T, typename A>
__device__ __forceinline__ T touch_arg_lines(T x, A f1) {
  asm("" : "+s"(x) : "s"(f1));
  return x;
}
template <typename T, typename A, typename B, typename C>
__device__ __forceinline__ T touch_arg_lines(T x, A f1, B f2, C f3) {
  asm("" : "+s"(x) : "s"(f1), "s"(f2), "s"(f3));
  return x;
}
template <typename T, typename A, typename B, typename C, typename D>
__device__ __forceinline__ T touch_arg_lines(T x, A f1, B f2, C f3, D f4) {
  asm("" : "+s"(x) : "s"(f1), "s"(f2), "s"(f3), "s"(f4));
  return x;
}
template <typename T, typename A, typename B, typename C, typename D, typename E, typename F,
          typename G>
__device__ __forceinline__ T touch_arg_lines(T x, A f1, B f2, C f3, D f4, E f5, F f6, G f7) {
  asm("" : "+s"(x) : "s"(f1), "s"(f2), "s"(f3), "s"(f4), "s"(f5), "s"(f6), "s"(f7));
  return x;
}

// True if every 64-byte line of a `bytes`-byte argument block holds one of
// the field offsets (a touch_arg_lines choice that leaves no line out).
constexpr bool covers_lines(size_t bytes, std::initializer_list<size_t> offsets) {
  for (size_t line = 0; 64 * line < bytes; ++line) {
    bool hit = false;
    for (size_t o : offsets) hit = hit || o / 64 == line;
    if (!hit) return false;
  }
  return true;
}

// s_waitcnt vmcnt(n) for n in {0, 4}, leaving the other counters alone.
// gfx9 encoding: vmcnt[3:0] | expcnt=7 | lgkmcnt=15 | vmcnt[5:4] << 14.
// On gfx9 vmcnt also counts stores, so vmcnt(0) returns only once every
// earlier vector store of the wave has been acknowledged.
__device__ __forceinline__ void s_waitcnt_vm(int n) {
  if (n == 0) __builtin_amdgcn_s_waitcnt(0x0F70);
  else __builtin_amdgcn_s_waitcnt(0x0F74);  // vmcnt(4)
}

// fp16(x) for an fp32 value, round-to-nearest-even.
__device__ __forceinline__ float round16(float x) { return (float)(f16)x; }

// Rotate-half RoPE of one 8-element chunk pair with the eager fp16 rounding
// sequence out = fp16(fp16(x*cos) + fp16(rotate_half(x)*sin)): `lo` holds
// dims [c, c+8) of the first half, `hi` the matching dims [c+32, c+40) of the
// second half; rotate_half(x) is -hi on the first half and lo on the second.
// Contraction is off here: hipcc narrows each rounded product to an fp16
// multiply and would otherwise fuse product and sum into one fma, skipping the
// rounding of the second product that the eager sequence performs.
__device__ __forceinline__ void rope_pair(f16x8& lo, f16x8& hi, f16x8 cos_lo, f16x8 sin_lo,
                                          f16x8 cos_hi, f16x8 sin_hi) {
#pragma clang fp contract(off)
  f16x8 out_lo, out_hi;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float xl = (float)lo[e], xh = (float)hi[e];
    // fp16(-y) == -fp16(y), so a + fp16(-xh*sin) is written as a - fp16(xh*sin).
    const float a = round16(xl * (float)cos_lo[e]);
    const float b = round16(xh * (float)sin_lo[e]);
    const float c = round16(xh * (float)cos_hi[e]);
    const float d = round16(xl * (float)sin_hi[e]);
    out_lo[e] = (f16)(a - b);
    out_hi[e] = (f16)(c + d);
  }
  lo = out_lo;
  hi = out_hi;
}

// Reductions over the four lanes that share a query column (l ^ 16, l ^ 32).
// gfx950's v_permlane16_swap / v_permlane32_swap exchange rows between two
// VGPRs in the VALU: with both operands = x, the two results hold, in every
// lane l, x[l] and x[l ^ 16] (resp. x[l ^ 32]).  No LDS round trip (a
// ds_bpermute costs ~100+ cycles of latency on the softmax's serial chain).
__device__ __forceinline__ void xor16_pair(float x, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

__device__ __forceinline__ void xor32_pair(float x, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

// Both orders of each pair give the same fp32 result (max and + commute), so
// every lane of a column ends with bit-identical values.
__device__ __forceinline__ float col_max(float x) {
  float a, b;
  xor16_pair(x, a, b);
  xor32_pair(fmaxf(a, b), a, b);
  return fmaxf(a, b);
}

__device__ __forceinline__ float col_sum(float x) {
  float a, b;
  xor16_pair(x, a, b);
  xor32_pair(a + b, a, b);
  return a + b;
}

// Paged KV caches (host side): page_size must be a power of two in
// [64, 4096] (a 32-key decode tile and a 64-key prefill tile then never
// straddle a page), with at least one page per row and a non-empty pool.
// Returns log2(page_size), or -1 when the geometry is unsupported.
inline int page_log2(int page_size, int pages_per_row, int n_pages) {
  if (page_size < 64 || page_size > 4096 || (page_size & (page_size - 1)) != 0) return -1;
  if (pages_per_row < 1 || n_pages < 1) return -1;
  if ((int64_t)pages_per_row * page_size > 0x7fffffff) return -1;
  int l = 0;
  while ((1 << l) < page_size) ++l;
  return l;
}

}  // namespace qf
