// Elementwise programs and reductions (HBM-bound). Each thread evaluates the program's instruction list on VEC = 8
// consecutive elements of the innermost dimension at once, so the (uniform) instruction dispatch is paid once per 8
// elements and contiguous leaves / outputs move as 8- to 32-byte vectors; the program's registers stay in VGPRs.
// Shapes whose innermost dimension is not a multiple of 8 run the same program one element per thread (registers in
// VGPRs). Reductions give each output row a workgroup (long rows, e.g. RMSNorm's 4096) or one wavefront (shorter
// rows), combine within the thread, across lanes with shuffles and across wavefronts through LDS; the init value
// enters once at the end.
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
    RegFile1 R;
    ew_run(P, lin, coord, nullptr, R);
    for (int o = 0; o < P.n_out; ++o)
      store_bits(P.out_ptr[o], lin, P.out_dtype[o], R.get(P.out_reg[o]), (P.out_float_mask >> o) & 1);
  }
}

constexpr int VEC = 8;    // elements per thread in the vectorised kernels
constexpr int VNT = 256;  // threads per workgroup there
using VRegs = SwitchRegFile<VEC>;

// Stores V consecutive register values (float bits if `is_float`, else int32) as `dtype` at out[lin..lin+V).
template <int V>
__device__ __forceinline__ void store_vec(void* out, int64_t lin, int dtype, const uint32_t* v, bool is_float) {
  static_assert(V == 4 || V == 8, "vector stores are written for 4 or 8 elements");
  char* p = (char*)out;
  switch (dtype) {
    case DT_F32: case DT_S32: case DT_U32: {
      uint32_t w[V];
#pragma unroll
      for (int e = 0; e < V; ++e) w[e] = (dtype != DT_F32 || is_float) ? v[e] : __float_as_uint((float)(int32_t)v[e]);
      *(u32x4v*)(p + lin * 4) = u32x4v{w[0], w[1], w[2], w[3]};
      if constexpr (V == 8) *(u32x4v*)(p + lin * 4 + 16) = u32x4v{w[4], w[5], w[6], w[7]};
      break;
    }
    case DT_BF16: case DT_F16: {
      uint32_t w[V / 2];
#pragma unroll
      for (int q = 0; q < V / 2; ++q) {
        const float a = is_float ? __uint_as_float(v[2 * q]) : (float)(int32_t)v[2 * q];
        const float b = is_float ? __uint_as_float(v[2 * q + 1]) : (float)(int32_t)v[2 * q + 1];
        if (dtype == DT_BF16) w[q] = f32x2_to_bf16x2_bits(a, b);
        else w[q] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) | ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
      }
      if constexpr (V == 8) *(u32x4v*)(p + lin * 2) = u32x4v{w[0], w[1], w[2], w[3]};
      else *(u32x2v*)(p + lin * 2) = u32x2v{w[0], w[1]};
      break;
    }
    case DT_F8E4M3FN: case DT_F8E5M2: case DT_S8: case DT_U8: case DT_PRED: {
      uint32_t w[V / 4];
#pragma unroll
      for (int q = 0; q < V / 4; ++q) w[q] = 0u;
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const float f = is_float ? __uint_as_float(v[e]) : (float)(int32_t)v[e];
        uint32_t byte;
        if (dtype == DT_F8E4M3FN) byte = f32_to_e4m3fn_bits(f);
        else if (dtype == DT_F8E5M2) byte = f32_to_e5m2_bits(f);
        else if (dtype == DT_PRED) byte = v[e] != 0;
        else byte = is_float ? (uint32_t)f2i_sat(f, dtype) & 0xffu : v[e] & 0xffu;
        w[e >> 2] |= byte << (8 * (e & 3));
      }
      if constexpr (V == 8) *(u32x2v*)(p + lin) = u32x2v{w[0], w[1]};
      else *(uint32_t*)(p + lin) = w[0];
      break;
    }
    default:
#pragma unroll
      for (int e = 0; e < V; ++e) store_bits(out, lin + e, dtype, v[e], is_float);
      break;
  }
}

// Coordinates of a linear index; 32-bit arithmetic when the iteration space allows it.
__device__ __forceinline__ void decompose_fast(int64_t lin, const EwProgram& P, int32_t* coord) {
  if (P.total <= 0x7fffffff) {
    uint32_t l = (uint32_t)lin;
    for (int d = P.rank - 1; d >= 0; --d) {
      const uint32_t sd = (uint32_t)P.shape[d];
      coord[d] = (int32_t)(l % sd);
      l /= sd;
    }
  } else {
    decompose(lin, P, coord);
  }
}

template <bool COORDS>
__global__ void __launch_bounds__(VNT) ew_kernel_vec(const EwProgram P) {
  VRegs R;
  const int64_t chunks = P.total / VEC;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < chunks; c += stride) {
    const int64_t lin = c * VEC;
    int32_t coord[EW_MAX_RANK];
    if (COORDS) decompose_fast(lin, P, coord);
    ew_run_v<VEC>(P, lin, coord, nullptr, R);
    for (int o = 0; o < P.n_out; ++o) {
      uint32_t v[VEC];
      R.load(P.out_reg[o], v);
      store_vec<VEC>(P.out_ptr[o], lin, P.out_dtype[o], v, (P.out_float_mask >> o) & 1);
    }
  }
}

static int grid_for(int64_t total, int threads) {
  int64_t blocks = (total + threads - 1) / threads;
  const int64_t cap = 256 * 32;  // 32 blocks per CU is plenty for a grid-stride loop
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  return (int)blocks;
}

// Element size in bytes of the types leaves and outputs use.
static int elem_size(int dt) {
  switch (dt) {
    case DT_F64: case DT_S64: case DT_U64: return 8;
    case DT_F32: case DT_S32: case DT_U32: return 4;
    case DT_BF16: case DT_F16: case DT_S16: case DT_U16: return 2;
    default: return 1;
  }
}

// Chooses how each leaf is read when VEC consecutive innermost elements are evaluated together; false when the
// program cannot run VEC-wide (innermost extent not a multiple of VEC, misaligned outputs, huge strides).
static bool prepare_vec(EwProgram& p, bool check_outputs) {
  if (p.rank < 1 || p.shape[p.rank - 1] % VEC != 0) return false;
  for (int i = 0; i < p.n_leaves; ++i) {
    EwLeaf& L = p.leaves[i];
    const int es = elem_size(L.dtype);
    const int64_t s = L.kind == EW_LEAF_SCALAR ? 0 : (L.kind == EW_LEAF_IDENTITY ? 1 : L.strides[p.rank - 1]);
    L.vstride = 0;
    if (s == 0) { L.vmode = EW_VEC_BCAST; continue; }
    bool contig = s == 1 && es <= 4 && ((uintptr_t)L.ptr % (uintptr_t)(VEC * es)) == 0 && L.offset % VEC == 0;
    if (contig && L.kind == EW_LEAF_GENERAL)
      for (int d = 0; d < p.rank - 1; ++d)
        if (L.strides[d] % VEC) contig = false;
    if (contig) { L.vmode = EW_VEC_CONTIG; continue; }
    if (s > INT32_MAX || s < INT32_MIN) return false;
    L.vmode = EW_VEC_GATHER;
    L.vstride = (int32_t)s;
  }
  if (check_outputs)
    for (int o = 0; o < p.n_out; ++o)
      if (((uintptr_t)p.out_ptr[o] % (uintptr_t)(VEC * elem_size(p.out_dtype[o]))) != 0) return false;
  return true;
}

void launch_elementwise(const EwProgram& p, hipStream_t stream) {
  if (p.total == 0) return;
  EwProgram v = p;
  if (prepare_vec(v, true)) {
    dim3 grid(grid_for(v.total / VEC, VNT)), block(VNT);
    if (v.needs_coords) hipLaunchKernelGGL(ew_kernel_vec<true>, grid, block, 0, stream, v);
    else hipLaunchKernelGGL(ew_kernel_vec<false>, grid, block, 0, stream, v);
  } else {
    dim3 grid(grid_for(p.total, 256)), block(256);
    if (p.needs_coords) hipLaunchKernelGGL(ew_kernel<true>, grid, block, 0, stream, p);
    else hipLaunchKernelGGL(ew_kernel<false>, grid, block, 0, stream, p);
  }
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
      RegFile1 R;
      ew_run(P, lin, coord, nullptr, R);
      acc = red_combine(acc, R.get(P.out_reg[0]), A.kind, fl);
    }
    for (int off = 32; off > 0; off >>= 1) {
      uint32_t other = (uint32_t)__shfl_xor((int)acc, off, 64);
      acc = red_combine(acc, other, A.kind, fl);
    }
    if (lane == 0) store_bits(P.out_ptr[0], o, P.out_dtype[0], red_combine(acc, init, A.kind, fl), fl);
  }
}

__device__ __forceinline__ uint32_t red_identity(int kind, bool fl) {
  switch (kind) {
    case RED_ADD: case RED_OR: return 0u;
    case RED_MUL: return fl ? __float_as_uint(1.0f) : 1u;
    case RED_MAX: return fl ? 0xff800000u : 0x80000000u;
    case RED_MIN: return fl ? 0x7f800000u : 0x7fffffffu;
    default: return 0xffffffffu;  // RED_AND
  }
}

// G threads per output row (VNT: one workgroup, 64: one wavefront); each thread folds VEC-element chunks.
template <int G, bool COORDS>
__global__ void __launch_bounds__(VNT) reduce_kernel_vec(const ReduceArgs A) {
  __shared__ uint32_t part[VNT / 64];
  VRegs R;
  const EwProgram& P = A.prologue;
  constexpr int RB = VNT / G;  // rows per workgroup
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = threadIdx.x / G, t = threadIdx.x % G;
  const bool fl = A.is_float != 0;
  const uint32_t init = A.init_ptr ? load_bits(A.init_ptr, 0, A.init_dtype) : (uint32_t)A.init.i;
  const uint32_t ident = red_identity(A.kind, fl);
  const int64_t chunks = A.inner / VEC;
  for (int64_t o = (int64_t)blockIdx.x * RB + g; o < A.outer; o += (int64_t)gridDim.x * RB) {
    uint32_t acc = ident;
    for (int64_t c = t; c < chunks; c += G) {
      const int64_t lin = o * A.inner + c * VEC;
      int32_t coord[EW_MAX_RANK];
      if (COORDS) decompose_fast(lin, P, coord);
      ew_run_v<VEC>(P, lin, coord, nullptr, R);
      uint32_t v[VEC];
      R.load(P.out_reg[0], v);
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc = red_combine(acc, v[e], A.kind, fl);
    }
    for (int off = 32; off > 0; off >>= 1) acc = red_combine(acc, (uint32_t)__shfl_xor((int)acc, off, 64), A.kind, fl);
    if constexpr (G == VNT) {
      if (lane == 0) part[wave] = acc;
      __syncthreads();
      if (threadIdx.x == 0) {
        uint32_t r = part[0];
        for (int w = 1; w < VNT / 64; ++w) r = red_combine(r, part[w], A.kind, fl);
        store_bits(P.out_ptr[0], o, P.out_dtype[0], red_combine(r, init, A.kind, fl), fl);
      }
      __syncthreads();  // part[] is reused by the next row
    } else {
      if (lane == 0) store_bits(P.out_ptr[0], o, P.out_dtype[0], red_combine(acc, init, A.kind, fl), fl);
    }
  }
}

void launch_reduce(const ReduceArgs& a, hipStream_t stream) {
  if (a.outer == 0) return;
  ReduceArgs v = a;
  if (a.inner % VEC == 0 && prepare_vec(v.prologue, false)) {
    const bool coords = v.prologue.needs_coords != 0;
    if (a.inner / VEC >= 2 * VNT) {  // long rows: a workgroup per row
      dim3 grid((unsigned)(a.outer < 256 * 16 ? a.outer : 256 * 16)), block(VNT);
      if (coords) hipLaunchKernelGGL((reduce_kernel_vec<VNT, true>), grid, block, 0, stream, v);
      else hipLaunchKernelGGL((reduce_kernel_vec<VNT, false>), grid, block, 0, stream, v);
    } else {  // a wavefront per row
      int64_t blocks = (a.outer + VNT / 64 - 1) / (VNT / 64);
      if (blocks > 256 * 16) blocks = 256 * 16;
      dim3 grid((unsigned)blocks), block(VNT);
      if (coords) hipLaunchKernelGGL((reduce_kernel_vec<64, true>), grid, block, 0, stream, v);
      else hipLaunchKernelGGL((reduce_kernel_vec<64, false>), grid, block, 0, stream, v);
    }
  } else {
    int64_t blocks = (a.outer + 3) / 4;
    if (blocks > 256 * 16) blocks = 256 * 16;
    dim3 grid((unsigned)blocks), block(256);
    if (a.prologue.needs_coords) hipLaunchKernelGGL(reduce_kernel<true>, grid, block, 0, stream, a);
    else hipLaunchKernelGGL(reduce_kernel<false>, grid, block, 0, stream, a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail(PJRT_Error_Code_INTERNAL, std::string("reduce launch failed: ") + hipGetErrorString(e));
}

}  // namespace ryft
