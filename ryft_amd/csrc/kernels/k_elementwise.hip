// Elementwise programs and reductions (HBM-bound). The elementwise kernel is a grid-stride loop over the iteration
// space; the reduction assigns one wavefront (64 lanes) per output element and combines lanes with cross-lane
// shuffles, which suits row reductions (softmax / RMSNorm rows of 10^3–10^4 elements).
#include <hip/hip_runtime.h>

#include <string>

#include "../common.h"
#include "ew_device.h"
#include "kernels.h"

namespace ryft {

template <bool COORDS>
__global__ void __launch_bounds__(256) ew_kernel(const EwProgram P) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t lin = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; lin < P.total; lin += stride) {
    int32_t coord[EW_MAX_RANK];
    if (COORDS) decompose(lin, P, coord);
    uint32_t regs[EW_MAX_REGS];
    ew_run(P, lin, coord, nullptr, regs);
    for (int o = 0; o < P.n_out; ++o)
      store_bits(P.out_ptr[o], lin, P.out_dtype[o], regs[P.out_reg[o]], (P.out_float_mask >> o) & 1);
  }
}

static int grid_for(int64_t total, int threads) {
  int64_t blocks = (total + threads - 1) / threads;
  const int64_t cap = 256 * 32;  // 32 blocks per CU is plenty for a grid-stride loop
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  return (int)blocks;
}

void launch_elementwise(const EwProgram& p, hipStream_t stream) {
  if (p.total == 0) return;
  dim3 grid(grid_for(p.total, 256)), block(256);
  if (p.needs_coords) hipLaunchKernelGGL(ew_kernel<true>, grid, block, 0, stream, p);
  else hipLaunchKernelGGL(ew_kernel<false>, grid, block, 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail(PJRT_Error_Code_INTERNAL, std::string("elementwise launch failed: ") + hipGetErrorString(e));
}

// ------------------------------------------------------------------------------------------------ reductions
__device__ __forceinline__ uint32_t red_combine(uint32_t a, uint32_t b, int kind, bool fl) {
  if (fl) {
    float x = __uint_as_float(a), y = __uint_as_float(b);
    switch (kind) {
      case RED_ADD: return __float_as_uint(x + y);
      case RED_MAX: return __float_as_uint((x != x || y != y) ? __uint_as_float(0x7fc00000u) : fmaxf(x, y));
      case RED_MIN: return __float_as_uint((x != x || y != y) ? __uint_as_float(0x7fc00000u) : fminf(x, y));
      case RED_MUL: return __float_as_uint(x * y);
      default: return a;
    }
  }
  int32_t x = (int32_t)a, y = (int32_t)b;
  switch (kind) {
    case RED_ADD: return (uint32_t)(x + y);
    case RED_MAX: return (uint32_t)(x > y ? x : y);
    case RED_MIN: return (uint32_t)(x < y ? x : y);
    case RED_MUL: return (uint32_t)(x * y);
    case RED_AND: return a & b;
    case RED_OR: return a | b;
    default: return a;
  }
}

template <bool COORDS>
__global__ void __launch_bounds__(256) reduce_kernel(const ReduceArgs A) {
  const EwProgram& P = A.prologue;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const bool fl = A.is_float != 0;
  const uint32_t init = A.init_ptr ? load_bits(A.init_ptr, 0, A.init_dtype) : (uint32_t)A.init.i;
  // lanes start from the body's identity; the init value enters once, after the cross-lane combine
  uint32_t ident;
  switch (A.kind) {
    case RED_ADD: case RED_OR: ident = 0u; break;
    case RED_MUL: ident = fl ? __float_as_uint(1.0f) : 1u; break;
    case RED_MAX: ident = fl ? 0xff800000u : 0x80000000u; break;
    case RED_MIN: ident = fl ? 0x7f800000u : 0x7fffffffu; break;
    default: ident = 0xffffffffu; break;  // RED_AND
  }
  for (int64_t o = (int64_t)blockIdx.x * 4 + wave; o < A.outer; o += (int64_t)gridDim.x * 4) {
    uint32_t acc = ident;
    for (int64_t r = lane; r < A.inner; r += 64) {
      int64_t lin = o * A.inner + r;
      int32_t coord[EW_MAX_RANK];
      if (COORDS) decompose(lin, P, coord);
      uint32_t regs[EW_MAX_REGS];
      ew_run(P, lin, coord, nullptr, regs);
      acc = red_combine(acc, regs[P.out_reg[0]], A.kind, fl);
    }
    for (int off = 32; off > 0; off >>= 1) {
      uint32_t other = (uint32_t)__shfl_xor((int)acc, off, 64);
      acc = red_combine(acc, other, A.kind, fl);
    }
    if (lane == 0) store_bits(P.out_ptr[0], o, P.out_dtype[0], red_combine(acc, init, A.kind, fl), fl);
  }
}

void launch_reduce(const ReduceArgs& a, hipStream_t stream) {
  if (a.outer == 0) return;
  int64_t blocks = (a.outer + 3) / 4;
  if (blocks > 256 * 16) blocks = 256 * 16;
  dim3 grid((unsigned)blocks), block(256);
  if (a.prologue.needs_coords) hipLaunchKernelGGL(reduce_kernel<true>, grid, block, 0, stream, a);
  else hipLaunchKernelGGL(reduce_kernel<false>, grid, block, 0, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail(PJRT_Error_Code_INTERNAL, std::string("reduce launch failed: ") + hipGetErrorString(e));
}

}  // namespace ryft
