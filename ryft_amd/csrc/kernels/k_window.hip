// dynamic_slice / dynamic_update_slice windows and gather (crates/ryft-mlir/src/dialects/stable_hlo/operations/
// manipulation.rs:943-1307): the window origin comes from device scalars (the start indices, one 0-d integer tensor
// per dimension), clamped per dimension to [0, shape - window] as StableHLO specifies, so any index value — negative,
// or past the end — gives an in-bounds window. Every thread reads the same few scalars (cached), then moves
// elements of the window: a whole 16-byte vector per thread where the window's rows are contiguous runs of whole
// vectors in both tensors, one element per thread otherwise. Memory-bound byte moves; no arithmetic on the values.
#include <hip/hip_runtime.h>

#include <string>

#include "../common.h"
#include "ew_device.h"
#include "kernels.h"
#include "launch.h"

namespace ryft {
namespace {

typedef uint32_t u32x4w __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int elem_size_of(int dt) {
  return dt == DT_S8 || dt == DT_U8 ? 1 : dt == DT_S16 || dt == DT_U16 ? 2 : dt == DT_S32 || dt == DT_U32 ? 4 : 8;
}

// One start index as a signed 64-bit value; unsigned values past INT64_MAX saturate (they clamp to the last origin
// either way).
__device__ __forceinline__ int64_t start_index(const void* p, int dt) {
  switch (dt) {
    case DT_S8: return *(const int8_t*)p;
    case DT_S16: return *(const int16_t*)p;
    case DT_S32: return *(const int32_t*)p;
    case DT_S64: return *(const int64_t*)p;
    case DT_U8: return *(const uint8_t*)p;
    case DT_U16: return *(const uint16_t*)p;
    case DT_U32: return *(const uint32_t*)p;
    default: {
      const uint64_t v = *(const uint64_t*)p;
      return v > (uint64_t)INT64_MAX ? INT64_MAX : (int64_t)v;
    }
  }
}

// Element offset of the window origin in the large tensor, and its row-major strides.
__device__ __forceinline__ int64_t window_origin(const WindowArgs& A, int64_t (&stride)[WIN_MAX_RANK]) {
  int64_t s = 1, origin = 0;
  for (int d = A.rank - 1; d >= 0; --d) {
    stride[d] = s;
    s *= A.shape[d];
  }
  for (int d = 0; d < A.rank; ++d) {
    int64_t v = start_index(A.idx[d], A.idx_dtype);
    const int64_t hi = A.shape[d] - A.win[d];
    v = v < 0 ? 0 : (v > hi ? hi : v);
    origin += v * stride[d];
  }
  return origin;
}

// UNIT bytes per thread and step: the element size, or 16 when the window rows are runs of whole 16-byte vectors at
// 16-byte aligned positions of both tensors (the launcher checks the shapes and pointers; the origin is checked here,
// uniformly, and the element path taken when it is not aligned).
template <int ES, bool VEC>
__global__ void __launch_bounds__(256) window_kernel(const WindowArgs A) {
  int64_t stride[WIN_MAX_RANK];
  const int64_t origin = window_origin(A, stride);
  const int r = A.rank;
  constexpr int PER = VEC ? 16 / ES : 1;  // elements per thread and step
  const bool vec = VEC && (origin * ES) % 16 == 0;
  const int64_t units = vec ? A.total / PER : A.total;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < units; u += step) {
    const int64_t e = vec ? u * PER : u;  // window element (row-major over win)
    int64_t rem = e, off = origin;
    for (int d = r - 1; d >= 0; --d) {
      const int64_t c = rem % A.win[d];
      rem /= A.win[d];
      off += c * stride[d];
    }
    const int64_t s_at = A.mode == WIN_READ ? off : e, d_at = A.mode == WIN_READ ? e : off;
    if (vec) {
      *(u32x4w*)((char*)A.dst + d_at * ES) = *(const u32x4w*)((const char*)A.src + s_at * ES);
    } else if constexpr (ES == 1) {
      ((uint8_t*)A.dst)[d_at] = ((const uint8_t*)A.src)[s_at];
    } else if constexpr (ES == 2) {
      ((uint16_t*)A.dst)[d_at] = ((const uint16_t*)A.src)[s_at];
    } else if constexpr (ES == 4) {
      ((uint32_t*)A.dst)[d_at] = ((const uint32_t*)A.src)[s_at];
    } else {
      ((uint64_t*)A.dst)[d_at] = ((const uint64_t*)A.src)[s_at];
    }
  }
}

// gather: one result element per thread and step (PER = 16 / ES consecutive elements along the result's last
// dimension when that dimension is an offset dimension of the operand's last dimension and both rows hold whole
// 16-byte vectors; moved as one vector when the operand position is aligned, element by element otherwise).
template <int ES, bool VEC>
__global__ void __launch_bounds__(256) gather_kernel(const GatherArgs A) {
  int64_t ostride[WIN_MAX_RANK], istride[WIN_MAX_RANK];
  {
    int64_t s = 1;
    for (int d = A.op_rank - 1; d >= 0; --d) {
      ostride[d] = s;
      s *= A.op_shape[d];
    }
    s = 1;
    for (int d = A.idx_rank - 1; d >= 0; --d) {
      istride[d] = s;
      s *= A.idx_shape[d];
    }
  }
  constexpr int PER = VEC ? 16 / ES : 1;
  const int64_t units = A.total / PER;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < units; u += step) {
    const int64_t e = u * PER;
    int64_t icoord[WIN_MAX_RANK];
    for (int d = 0; d < A.idx_rank; ++d) icoord[d] = 0;
    int64_t op_off = 0, rem = e;
    for (int r = A.out_rank - 1; r >= 0; --r) {
      const int64_t c = rem % A.out_shape[r];
      rem /= A.out_shape[r];
      if (A.out_to_op[r] >= 0) op_off += c * ostride[A.out_to_op[r]];
      if (A.out_to_idx[r] >= 0) icoord[A.out_to_idx[r]] = c;
    }
    for (int d = 0; d < A.op_rank; ++d)
      if (A.op_batch[d] >= 0) op_off += icoord[A.op_batch[d]] * ostride[d];
    int64_t ioff = 0;
    for (int d = 0; d < A.idx_rank; ++d) ioff += icoord[d] * istride[d];
    const int64_t ivstep = A.ivd < A.idx_rank ? istride[A.ivd] : 0;  // icoord[ivd] is 0 here
    for (int k = 0; k < A.n_map; ++k) {
      const int dt = A.idx_dtype;
      const char* p = (const char*)A.indices + (ioff + k * ivstep) * (int64_t)elem_size_of(dt);
      int64_t v = start_index(p, dt);
      const int d = A.map[k];
      const int64_t hi = A.op_shape[d] - A.slice[d];
      v = v < 0 ? 0 : (v > hi ? hi : v);
      op_off += v * ostride[d];
    }
    if (VEC && (op_off * ES) % 16 == 0) {
      *(u32x4w*)((char*)A.out + e * ES) = *(const u32x4w*)((const char*)A.operand + op_off * ES);
    } else {
#pragma unroll
      for (int q = 0; q < PER; ++q) {
        if constexpr (ES == 1) ((uint8_t*)A.out)[e + q] = ((const uint8_t*)A.operand)[op_off + q];
        else if constexpr (ES == 2) ((uint16_t*)A.out)[e + q] = ((const uint16_t*)A.operand)[op_off + q];
        else if constexpr (ES == 4) ((uint32_t*)A.out)[e + q] = ((const uint32_t*)A.operand)[op_off + q];
        else ((uint64_t*)A.out)[e + q] = ((const uint64_t*)A.operand)[op_off + q];
      }
    }
  }
}

template <int ES>
void launch_gather_es(const GatherArgs& a, bool vec, hipStream_t stream, hipEvent_t done) {
  const int64_t units = vec ? a.total / (16 / ES) : a.total;
  const int64_t blocks = std::min<int64_t>((units + 255) / 256, 256 * 16);
  if (vec) launch_k(done, gather_kernel<ES, true>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  else launch_k(done, gather_kernel<ES, false>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
}

template <int ES>
void launch_es(const WindowArgs& a, bool vec, hipStream_t stream, hipEvent_t done) {
  const int64_t units = vec ? a.total / (16 / ES) : a.total;
  const int64_t blocks = std::min<int64_t>((units + 255) / 256, 256 * 16);
  if (vec) launch_k(done, window_kernel<ES, true>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  else launch_k(done, window_kernel<ES, false>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
}

}  // namespace

void launch_window(const WindowArgs& a, hipStream_t stream, hipEvent_t done) {
  if (a.rank < 0 || a.rank > WIN_MAX_RANK) fail(PJRT_Error_Code_INTERNAL, "window rank out of range");
  int64_t total = 1;
  for (int d = 0; d < a.rank; ++d) {
    if (a.win[d] < 0 || a.win[d] > a.shape[d]) fail(PJRT_Error_Code_INTERNAL, "window larger than its tensor");
    if (!a.idx[d]) fail(PJRT_Error_Code_INTERNAL, "window start index pointer is null");
    total *= a.win[d];
  }
  if (total != a.total) fail(PJRT_Error_Code_INTERNAL, "window element count mismatch");
  if (a.idx_dtype < DT_S8 || a.idx_dtype > DT_U64) fail(PJRT_Error_Code_INTERNAL, "window start indices must be integers");
  if (a.mode != WIN_READ && a.mode != WIN_WRITE) fail(PJRT_Error_Code_INTERNAL, "window mode");
  if (total == 0) return record_done(done, stream);
  // whole 16-byte vectors: the innermost window extent covers whole vectors, the tensors' innermost rows hold whole
  // vectors, and both base pointers are 16-byte aligned (so every row of the window starts on a vector when the
  // origin does; the kernel checks that)
  const int es = a.elem_bytes;
  const int64_t inner_w = a.rank ? a.win[a.rank - 1] : 1, inner_s = a.rank ? a.shape[a.rank - 1] : 1;
  const bool vec = es < 16 && (inner_w * es) % 16 == 0 && (inner_s * es) % 16 == 0 &&
                   (((uintptr_t)a.src | (uintptr_t)a.dst) & 15) == 0;
  switch (es) {
    case 1: return launch_es<1>(a, vec, stream, done);
    case 2: return launch_es<2>(a, vec, stream, done);
    case 4: return launch_es<4>(a, vec, stream, done);
    case 8: return launch_es<8>(a, vec, stream, done);
    default: fail(PJRT_Error_Code_INTERNAL, "window element size " + std::to_string(es));
  }
}

void launch_gather(const GatherArgs& a, hipStream_t stream, hipEvent_t done) {
  // the shapes the kernel's index arithmetic relies on, checked before the launch: every result coordinate mapped to
  // an operand dimension stays inside the slice there, every start-indices coordinate inside that tensor
  auto rank_ok = [](int r) { return r >= 0 && r <= WIN_MAX_RANK; };
  if (!rank_ok(a.out_rank) || !rank_ok(a.op_rank) || !rank_ok(a.idx_rank) || a.n_map < 0 || a.n_map > a.op_rank ||
      a.ivd < 0 || a.ivd > a.idx_rank)
    fail(PJRT_Error_Code_INTERNAL, "gather ranks out of range");
  if (a.idx_dtype < DT_S8 || a.idx_dtype > DT_U64) fail(PJRT_Error_Code_INTERNAL, "gather start indices must be integers");
  int64_t total = 1;
  int offset_of[WIN_MAX_RANK] = {0, 0, 0, 0, 0, 0};  // result dims offsetting each operand dim (at most one)
  for (int r = 0; r < a.out_rank; ++r) {
    total *= a.out_shape[r];
    const int d = a.out_to_op[r], i = a.out_to_idx[r];
    if (d >= 0 && d < a.op_rank && ++offset_of[d] > 1) fail(PJRT_Error_Code_INTERNAL, "gather offset dims repeat");
    if ((d >= 0) == (i >= 0)) fail(PJRT_Error_Code_INTERNAL, "gather result dimension must be an offset or a batch dim");
    if (d >= a.op_rank || (d >= 0 && a.out_shape[r] > a.slice[d])) fail(PJRT_Error_Code_INTERNAL, "gather offset dim");
    if (i >= a.idx_rank || i == a.ivd || (i >= 0 && a.out_shape[r] != a.idx_shape[i]))
      fail(PJRT_Error_Code_INTERNAL, "gather batch dim");
  }
  if (total != a.total) fail(PJRT_Error_Code_INTERNAL, "gather element count mismatch");
  for (int d = 0; d < a.op_rank; ++d) {
    if (a.slice[d] < 0 || a.slice[d] > a.op_shape[d]) fail(PJRT_Error_Code_INTERNAL, "gather slice size");
    const int b = a.op_batch[d];
    if (b >= a.idx_rank || b == a.ivd || (b >= 0 && a.idx_shape[b] != a.op_shape[d]) || (b >= 0 && a.slice[d] > 1))
      fail(PJRT_Error_Code_INTERNAL, "gather batching dim");
  }
  for (int k = 0; k < a.n_map; ++k)
    if (a.map[k] < 0 || a.map[k] >= a.op_rank || a.op_batch[a.map[k]] >= 0)
      fail(PJRT_Error_Code_INTERNAL, "gather start_index_map");
  if ((a.ivd < a.idx_rank ? a.idx_shape[a.ivd] : 1) != a.n_map) fail(PJRT_Error_Code_INTERNAL, "gather index vectors");
  if (total == 0) return record_done(done, stream);
  for (int d = 0; d < a.op_rank; ++d)  // a non-empty result of an empty operand has no element to read
    if (a.op_shape[d] == 0) fail(PJRT_Error_Code_INVALID_ARGUMENT, "gather from an empty operand into a non-empty result");
  const int es = a.elem_bytes;
  const int last = a.out_rank - 1;
  const bool vec = es < 16 && last >= 0 && a.out_to_op[last] == a.op_rank - 1 && (a.out_shape[last] * es) % 16 == 0 &&
                   (a.op_shape[a.op_rank - 1] * es) % 16 == 0 &&
                   (((uintptr_t)a.operand | (uintptr_t)a.out) & 15) == 0;
  switch (es) {
    case 1: return launch_gather_es<1>(a, vec, stream, done);
    case 2: return launch_gather_es<2>(a, vec, stream, done);
    case 4: return launch_gather_es<4>(a, vec, stream, done);
    case 8: return launch_gather_es<8>(a, vec, stream, done);
    default: fail(PJRT_Error_Code_INTERNAL, "gather element size " + std::to_string(es));
  }
}

}  // namespace ryft
