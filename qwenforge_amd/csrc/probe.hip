// Calibration kernels: the HBM read rate the box reaches for a given size,
// and the launch floor of a graph node (empty, one and two dependent memory
// round trips), measured beside the decode kernels (see include/qf_probe.h).
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

// Launch-floor probe: a kernel shaped like a decode launch (workgroups x
// threads) whose critical path is `kTrips` dependent memory round trips and
// nothing else.  kTrips 0 returns at once; 1: each thread issues one 16-byte
// non-temporal load of its own slice of `src` and each wave writes the XOR to
// sink; 2: the load offset first depends on a device int64 read (as a decode
// split range depends on kv_last), then the same tile load.
template <int kTrips>
__global__ void launch_probe_kernel(const u32x4* __restrict__ src, int64_t n16,
                                    const int64_t* __restrict__ index, uint32_t* sink) {
  if (kTrips == 0) return;
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (kTrips == 2) i += (uint64_t)index[0];
  i = i < (uint64_t)n16 ? i : i % (uint64_t)n16;  // any index value stays in bounds
  const u32x4 a = __builtin_nontemporal_load(src + i);
  uint32_t acc = a[0] ^ a[1] ^ a[2] ^ a[3];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, off);
  if ((threadIdx.x & 63) == 0) sink[(blockIdx.x * blockDim.x + threadIdx.x) >> 6] = acc;
}

}  // namespace qf

extern "C" int qf_launch_probe(const void* src, int64_t bytes, const int64_t* index,
                               uint32_t* sink, int workgroups, int threads, int round_trips,
                               void* stream) {
  if (workgroups < 1 || workgroups > 65535 || threads < 64 || threads > 1024 || (threads & 63))
    return QF_ERR_INVALID_ARG;
  if (round_trips < 0 || round_trips > 2) return QF_ERR_INVALID_ARG;
  if (round_trips > 0) {
    if (!src || !sink || bytes < 16 || (bytes & 15)) return QF_ERR_INVALID_ARG;
    if ((reinterpret_cast<uintptr_t>(src) & 15u) != 0) return QF_ERR_INVALID_ARG;
    if (round_trips == 2 && !index) return QF_ERR_INVALID_ARG;
  }
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const auto* s16 = static_cast<const qf::u32x4*>(src);
  const dim3 grid(workgroups), block(threads);
  if (round_trips == 0)
    hipLaunchKernelGGL(qf::launch_probe_kernel<0>, grid, block, 0, st, s16, bytes / 16, index, sink);
  else if (round_trips == 1)
    hipLaunchKernelGGL(qf::launch_probe_kernel<1>, grid, block, 0, st, s16, bytes / 16, index, sink);
  else
    hipLaunchKernelGGL(qf::launch_probe_kernel<2>, grid, block, 0, st, s16, bytes / 16, index, sink);
  return (int)hipGetLastError();
}

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
