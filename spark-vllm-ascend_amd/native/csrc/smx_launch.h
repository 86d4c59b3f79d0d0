// Kernel launches of the C-ABI entry points: launched on the caller's HIP
// stream, or, while a step runner records on the calling thread, handed to it
// as (kernel, grid, workgroup, dynamic LDS, kernel-argument bytes) for replay
// as hand-written AQL dispatch packets (step_runner.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

namespace smx {

// Receives the launches made on one thread while a runner records.
class LaunchSink {
 public:
  virtual void record(const void* host_fn, dim3 grid, dim3 block, uint32_t dynamic_lds,
                      const void* kernarg, size_t kernarg_size) = 0;

 protected:
  ~LaunchSink() = default;
};

// The calling thread's sink (null when nothing records).
LaunchSink*& launch_sink();

// Explicit kernel arguments laid out as the AMDGPU kernel ABI lays them out in
// the kernarg segment: in declaration order, each at the next offset aligned
// to its type's alignment.  The kernels of this library take no implicit
// (hidden) arguments, which the runner checks against the code object's
// kernarg segment size.
constexpr size_t kMaxKernarg = 256;

template <typename T>
inline size_t pack_kernarg(unsigned char* buf, size_t off, const T& v) {
  off = (off + alignof(T) - 1) & ~(alignof(T) - 1);
  if (off + sizeof(T) <= kMaxKernarg) memcpy(buf + off, &v, sizeof(T));
  return off + sizeof(T);
}

template <typename... P, typename... A>
inline void record_launch(LaunchSink* sink, void (*fn)(P...), dim3 grid, dim3 block,
                          uint32_t dynamic_lds, A&&... args) {
  static_assert(sizeof...(P) == sizeof...(A), "argument count differs from the kernel's");
  alignas(16) unsigned char buf[kMaxKernarg] = {};
  size_t off = 0;
  ((off = pack_kernarg<P>(buf, off, static_cast<P>(args))), ...);
  // a size beyond kMaxKernarg is reported to the sink, which rejects it
  sink->record(reinterpret_cast<const void*>(fn), grid, block, dynamic_lds, buf, off);
}

}  // namespace smx

// Drop-in for hipLaunchKernelGGL at every launch site of the library.
#define SMX_LAUNCH(kernel, grid, block, lds, stream, ...)                                     \
  do {                                                                                        \
    if (::smx::LaunchSink* smx_sink_ = ::smx::launch_sink())                                  \
      ::smx::record_launch(smx_sink_, kernel, dim3(grid), dim3(block), (uint32_t)(lds),       \
                           __VA_ARGS__);                                                      \
    else                                                                                      \
      hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);                      \
  } while (0)
