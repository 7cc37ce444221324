// Kernel launches that can carry the completion event of an execution: given an event, the launch records it as
// part of the kernel dispatch itself (hipExtLaunchKernel's stop event) instead of a separate marker packet after
// it, which would cost the queue one more packet round trip between consecutive executions.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <utility>

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

// Compute units of the current device (looked up once per device).
inline int device_cus() {
  static std::mutex mu;
  static std::map<int, int> cache;
  int dev = 0;
  (void)hipGetDevice(&dev);
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
  cache[dev] = cus;
  return cus;
}

// Workgroups of `threads` threads of a kernel that one compute unit holds at once (its register and LDS needs
// decide), looked up once per kernel.
template <typename F>
inline int resident_blocks(F kernel, int threads) {
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, int> cache;
  const std::pair<const void*, int> key{(const void*)kernel, threads};
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0) != hipSuccess || n < 1) n = 1;
  cache[key] = n;
  return n;
}

}  // namespace ryft
