// Streaming-read calibration kernel: the HBM read rate the box reaches for a
// given size, measured beside the decode kernels (see include/qf_probe.h).
#include "qf_common.h"
#include "../../include/qf_attn.h"
#include "../../include/qf_probe.h"

namespace qf {

// Four 16-byte loads per thread and iteration, all issued before any use;
// the XOR of everything a wave read goes to sink[4 * block + wave].  The
// loads are non-temporal, the flavor the decode kernels stream K/V and
// weights with, so this is the rate those reads can reach.
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ src,
                                                          int64_t n16, uint32_t* sink) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  uint32_t acc = 0;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 a = __builtin_nontemporal_load(src + i);
    const u32x4 b = __builtin_nontemporal_load(src + i + stride);
    const u32x4 c = __builtin_nontemporal_load(src + i + 2 * stride);
    const u32x4 d = __builtin_nontemporal_load(src + i + 3 * stride);
    const u32x4 x = a ^ b ^ c ^ d;
    acc ^= x[0] ^ x[1] ^ x[2] ^ x[3];
  }
  for (; i < n16; i += stride) {
    const u32x4 a = __builtin_nontemporal_load(src + i);
    acc ^= a[0] ^ a[1] ^ a[2] ^ a[3];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, off);
  if ((threadIdx.x & 63) == 0) sink[4 * blockIdx.x + (threadIdx.x >> 6)] = acc;
}

}  // namespace qf

extern "C" int qf_stream_read(const void* src, int64_t bytes, uint32_t* sink, int workgroups,
                              void* stream) {
  if (!src || !sink || bytes < 16 || (bytes & 15) || workgroups < 1 || workgroups > 65535)
    return QF_ERR_INVALID_ARG;
  if ((reinterpret_cast<uintptr_t>(src) & 15u) != 0) return QF_ERR_INVALID_ARG;
  hipLaunchKernelGGL(qf::stream_read_kernel, dim3(workgroups), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const qf::u32x4*>(src),
                     bytes / 16, sink);
  return (int)hipGetLastError();
}
