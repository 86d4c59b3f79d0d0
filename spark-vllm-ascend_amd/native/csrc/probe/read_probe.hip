// Streaming-read probe: the HBM ceiling the decode kernels are measured
// against.  It reads a buffer once -- 16-byte loads, every load of a lane
// issued before any of them is used -- and writes one word per wave (the XOR
// of what the wave read, so the loads cannot be dropped).  A GEMV or attention
// launch that moves B bytes cannot beat this kernel on the same B bytes: it
// has the same launch and first-load latency and no arithmetic.  No
// counterpart in the reference: a measurement instrument, built into its own
// library (libsmx_probe.so) that only the benchmark loads, declared in
// read_probe.h beside this file, never part of libsmx.so.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "read_probe.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int LOADS>
__global__ __launch_bounds__(256) void read_probe_kernel(const u32x4* __restrict__ src,
                                                         int64_t n16, uint32_t* __restrict__ sink) {
  const int64_t base = (int64_t)blockIdx.x * (256 * LOADS) + threadIdx.x;
  u32x4 v[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int64_t j = base + (int64_t)i * 256;
    v[i] = src[j < n16 ? j : n16 - 1];  // clamped, unconditional: all loads in flight
  }
  uint32_t x = 0;
#pragma unroll
  for (int i = 0; i < LOADS; ++i) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x ^= (uint32_t)__shfl_xor((int)x, o, 64);
  // lane 0 of each wave.  A plain store: only the host reads the sink (no
  // later kernel does), and an agent-scope store would make every wave wait
  // for its write-through before ending, which the instrument must not time.
  if ((threadIdx.x & 63) == 0) sink[blockIdx.x * 4 + (threadIdx.x >> 6)] = x;
}

}  // namespace

extern "C" int32_t smx_probe_abi_version(void) { return SMX_PROBE_ABI_VERSION; }

extern "C" int64_t smx_read_probe_sink_size(int64_t bytes, int32_t loads_per_lane) {
  if (bytes < 16 || bytes % 16 || !(loads_per_lane == 1 || loads_per_lane == 2 ||
                                    loads_per_lane == 4 || loads_per_lane == 8 ||
                                    loads_per_lane == 16))
    return -1;
  const int64_t per_wg = 256ll * 16 * loads_per_lane;
  return 4 * ((bytes + per_wg - 1) / per_wg);  // one word per wave, 4 waves per workgroup
}

extern "C" int smx_read_probe(void* stream, const void* src, int64_t bytes, uint32_t* sink,
                              int64_t sink_size, int32_t loads_per_lane) {
  if (!src || !sink || (uintptr_t)src % 16 != 0 || (uintptr_t)sink % 4 != 0)
    return SMX_PROBE_EINVAL;
  const int64_t words = smx_read_probe_sink_size(bytes, loads_per_lane);
  if (words <= 0 || words / 4 >= (1ll << 31) || sink_size != words) return SMX_PROBE_EINVAL;
  const unsigned grid = (unsigned)(words / 4);
  const int64_t n16 = bytes / 16;
  const hipStream_t s = (hipStream_t)stream;
  const auto* p = reinterpret_cast<const u32x4*>(src);
  switch (loads_per_lane) {
    case 1: hipLaunchKernelGGL(read_probe_kernel<1>, dim3(grid), dim3(256), 0, s, p, n16, sink); break;
    case 2: hipLaunchKernelGGL(read_probe_kernel<2>, dim3(grid), dim3(256), 0, s, p, n16, sink); break;
    case 4: hipLaunchKernelGGL(read_probe_kernel<4>, dim3(grid), dim3(256), 0, s, p, n16, sink); break;
    case 8: hipLaunchKernelGGL(read_probe_kernel<8>, dim3(grid), dim3(256), 0, s, p, n16, sink); break;
    default: hipLaunchKernelGGL(read_probe_kernel<16>, dim3(grid), dim3(256), 0, s, p, n16, sink); break;
  }
  return (int)hipGetLastError();
}
