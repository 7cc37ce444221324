// Kernel launches that can carry the completion event of an execution: given an event, the launch records it as
// part of the kernel dispatch itself (hipExtLaunchKernel's stop event) instead of a separate marker packet after
// it, which would cost the queue one more packet round trip between consecutive executions. In the same way the
// next launch of the calling thread can carry a start event (`pending_start`, set by the runtime's per-step kernel
// timing): the step's duration is then its kernels' own, not that plus a marker packet's dispatch latency.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "kernels.h"

namespace ryft {

// The pending start event (pending_start() is declared in kernels.h), handed to exactly one launch.
inline hipEvent_t take_start() {
  hipEvent_t e = pending_start();
  pending_start() = nullptr;
  return e;
}

template <typename F, typename... Args>
inline void launch_k(hipEvent_t done, F kernel, dim3 grid, dim3 block, uint32_t shmem, hipStream_t s, Args... args) {
  hipEvent_t start = take_start();
  if (done || start) hipExtLaunchKernelGGL(kernel, grid, block, shmem, s, start, done, 0, args...);
  else hipLaunchKernelGGL(kernel, grid, block, shmem, s, args...);
}

// A launcher that ends up launching nothing still owes the events their place in the stream.
inline void record_done(hipEvent_t done, hipStream_t s) {
  if (hipEvent_t start = take_start()) (void)hipEventRecord(start, s);
  if (done) (void)hipEventRecord(done, s);
}

}  // namespace ryft
