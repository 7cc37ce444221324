// Kernel launches that can carry the completion event of an execution: given an event, the launch records it as
// part of the kernel dispatch itself (hipExtLaunchKernel's stop event) instead of a separate marker packet after
// it, which would cost the queue one more packet round trip between consecutive executions.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

namespace ryft {

template <typename F, typename... Args>
inline void launch_k(hipEvent_t done, F kernel, dim3 grid, dim3 block, uint32_t shmem, hipStream_t s, Args... args) {
  if (done) hipExtLaunchKernelGGL(kernel, grid, block, shmem, s, nullptr, done, 0, args...);
  else hipLaunchKernelGGL(kernel, grid, block, shmem, s, args...);
}

// A launcher that ends up launching nothing still owes the event its place in the stream.
inline void record_done(hipEvent_t done, hipStream_t s) {
  if (done) (void)hipEventRecord(done, s);
}

}  // namespace ryft
