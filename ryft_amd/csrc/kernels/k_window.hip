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


// ------------------------------------------------------------------------------------------------ scatter
// scatter (manipulation.rs:1614-1690): update element u lands on result index full_start + full_batching +
// full_window, where full_start places the index vector of u's scatter coordinates on the operand dims named by
// scatter_dims_to_operand_dims, full_batching the scatter coordinate of each input batching dim's indices batching dim,
// and full_window u's window coordinates on the operand dims that are neither inserted nor batching. A window whose
// start lies outside the operand (some mapped dim with start < 0 or start + window > extent) is skipped whole, as
// XLA does. Combining runs on 32-bit register values (floats as f32, rounded back to the element type; integers
// wrapped), the same arithmetic as the elementwise kernels; 64-bit elements are only replaced.

// The value `cur` combined with `upd` (register forms of element type dt).
__device__ __forceinline__ uint32_t scatter_combine(uint32_t cur, uint32_t upd, int kind, int dt) {
  if (kind == SC_SET) return upd;
  if (dt_is_float(dt)) {
    const float a = __uint_as_float(cur), b = __uint_as_float(upd);
    float r;
    switch (kind) {
      case SC_ADD: r = a + b; break;
      case SC_MUL: r = a * b; break;
      case SC_MIN: r = (a != a || b != b) ? __uint_as_float(0x7fc00000u) : fminf(a, b); break;
      default: r = (a != a || b != b) ? __uint_as_float(0x7fc00000u) : fmaxf(a, b); break;
    }
    return __float_as_uint(r);
  }
  const bool uns = dt == DT_U8 || dt == DT_U16 || dt == DT_U32 || dt == DT_PRED;
  const int32_t a = (int32_t)cur, b = (int32_t)upd;
  int32_t r;
  switch (kind) {
    case SC_ADD: r = dt == DT_PRED ? (a | b) : (int32_t)((uint32_t)a + (uint32_t)b); break;
    case SC_MUL: r = dt == DT_PRED ? (a & b) : (int32_t)((uint32_t)a * (uint32_t)b); break;
    case SC_MIN: r = uns ? (int32_t)min((uint32_t)a, (uint32_t)b) : min(a, b); break;
    case SC_MAX: r = uns ? (int32_t)max((uint32_t)a, (uint32_t)b) : max(a, b); break;
    case SC_AND: r = a & b; break;
    default: r = a | b; break;
  }
  return (uint32_t)r;
}

// One update element combined into the result element at `o` (u: its offset in the updates).
template <int ES>
__device__ __forceinline__ void scatter_apply(const ScatterArgs& A, int64_t o, int64_t u) {
  if constexpr (ES == 8) {  // replaced only (the planner admits no other combination of 64-bit elements)
    ((uint64_t*)A.out)[o] = ((const uint64_t*)A.updates)[u];
  } else {
    if (A.kind == SC_SET) {
      if constexpr (ES == 1) ((uint8_t*)A.out)[o] = ((const uint8_t*)A.updates)[u];
      else if constexpr (ES == 2) ((uint16_t*)A.out)[o] = ((const uint16_t*)A.updates)[u];
      else ((uint32_t*)A.out)[o] = ((const uint32_t*)A.updates)[u];
      return;
    }
    const uint32_t r = scatter_combine(load_bits(A.out, o, A.dtype), load_bits(A.updates, u, A.dtype), A.kind, A.dtype);
    store_bits(A.out, o, A.dtype, r, dt_is_float(A.dtype));
  }
}

// Row-major strides of the operand and the updates, and the operand offset of the window of scatter position
// `icoord` (its coordinates along the indices' dims; the index vector dim's is 0). False when the window starts outside
// the operand.
__device__ __forceinline__ bool scatter_window(const ScatterArgs& A, const int64_t (&icoord)[WIN_MAX_RANK],
                                               const int64_t (&ostride)[WIN_MAX_RANK], int64_t* op_off) {
  int64_t istride[WIN_MAX_RANK];
  int64_t s = 1;
  for (int d = A.idx_rank - 1; d >= 0; --d) {
    istride[d] = s;
    s *= A.idx_shape[d];
  }
  int64_t ioff = 0;
  for (int d = 0; d < A.idx_rank; ++d) ioff += icoord[d] * istride[d];
  const int64_t ivstep = A.ivd < A.idx_rank ? istride[A.ivd] : 0;
  int64_t off = 0;
  bool ok = true;
  for (int k = 0; k < A.n_map; ++k) {
    const char* p = (const char*)A.indices + (ioff + k * ivstep) * (int64_t)elem_size_of(A.idx_dtype);
    const int64_t v = start_index(p, A.idx_dtype);
    const int d = A.map[k];
    ok = ok && v >= 0 && v <= A.op_shape[d] - A.win[d];
    off += v * ostride[d];
  }
  for (int d = 0; d < A.op_rank; ++d)
    if (A.op_batch[d] >= 0) off += icoord[A.op_batch[d]] * ostride[d];
  *op_off = off;
  return ok;
}

__device__ __forceinline__ void scatter_strides(const ScatterArgs& A, int64_t (&ostride)[WIN_MAX_RANK],
                                                int64_t (&ustride)[WIN_MAX_RANK]) {
  int64_t s = 1;
  for (int d = A.op_rank - 1; d >= 0; --d) {
    ostride[d] = s;
    s *= A.op_shape[d];
  }
  s = 1;
  for (int d = A.upd_rank - 1; d >= 0; --d) {
    ustride[d] = s;
    s *= A.upd_shape[d];
  }
}

// serial: one workgroup, the windows in row-major order of the update's scatter dims, a barrier after each (the
// elements of one window land on distinct result elements, so its threads never collide).
template <int ES>
__global__ void __launch_bounds__(1024) scatter_serial_kernel(const ScatterArgs A) {
  int64_t ostride[WIN_MAX_RANK], ustride[WIN_MAX_RANK];
  scatter_strides(A, ostride, ustride);
  for (int64_t w = 0; w < A.n_windows; ++w) {
    int64_t icoord[WIN_MAX_RANK] = {0, 0, 0, 0, 0, 0};
    int64_t ubase = 0, rem = w;
    for (int r = A.upd_rank - 1; r >= 0; --r)
      if (A.upd_to_idx[r] >= 0) {
        const int64_t c = rem % A.upd_shape[r];
        rem /= A.upd_shape[r];
        icoord[A.upd_to_idx[r]] = c;
        ubase += c * ustride[r];
      }
    int64_t obase;
    if (scatter_window(A, icoord, ostride, &obase)) {
      for (int64_t e = threadIdx.x; e < A.win_elems; e += blockDim.x) {
        int64_t o = obase, u = ubase, q = e;
        for (int r = A.upd_rank - 1; r >= 0; --r)
          if (A.upd_to_op[r] >= 0) {
            const int64_t c = q % A.upd_shape[r];
            q /= A.upd_shape[r];
            o += c * ostride[A.upd_to_op[r]];
            u += c * ustride[r];
          }
        scatter_apply<ES>(A, o, u);
      }
    }
    __syncthreads();
  }
}

// parallel: every update element at once (the windows are disjoint).
template <int ES>
__global__ void __launch_bounds__(256) scatter_parallel_kernel(const ScatterArgs A) {
  int64_t ostride[WIN_MAX_RANK], ustride[WIN_MAX_RANK];
  scatter_strides(A, ostride, ustride);
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < A.total; u += (int64_t)gridDim.x * blockDim.x) {
    int64_t icoord[WIN_MAX_RANK] = {0, 0, 0, 0, 0, 0};
    int64_t wo = 0, rem = u;
    for (int r = A.upd_rank - 1; r >= 0; --r) {
      const int64_t c = rem % A.upd_shape[r];
      rem /= A.upd_shape[r];
      if (A.upd_to_idx[r] >= 0) icoord[A.upd_to_idx[r]] = c;
      else wo += c * ostride[A.upd_to_op[r]];
    }
    int64_t obase;
    if (scatter_window(A, icoord, ostride, &obase)) scatter_apply<ES>(A, obase + wo, u);
  }
}

template <int ES>
void launch_scatter_es(const ScatterArgs& a, hipStream_t stream, hipEvent_t done) {
  if (a.serial) {
    const int threads = a.win_elems >= 1024 ? 1024 : (a.win_elems >= 256 ? 256 : 64);
    launch_k(done, scatter_serial_kernel<ES>, dim3(1), dim3(threads), 0, stream, a);
  } else {
    const int64_t blocks = std::min<int64_t>((a.total + 255) / 256, 256 * 16);
    launch_k(done, scatter_parallel_kernel<ES>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  }
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

void launch_scatter(const ScatterArgs& a, hipStream_t stream, hipEvent_t done) {
  // the shapes the kernels' index arithmetic relies on, checked before the launch: each update dim walks either an
  // operand dim (inside that dim's window) or an indices dim (of the same extent), each operand batching dim has a
  // same-sized indices batching dim, and the index vectors have one component per mapped operand dim
  auto rank_ok = [](int r) { return r >= 0 && r <= WIN_MAX_RANK; };
  if (!rank_ok(a.upd_rank) || !rank_ok(a.op_rank) || !rank_ok(a.idx_rank) || a.n_map < 0 || a.n_map > a.op_rank ||
      a.ivd < 0 || a.ivd > a.idx_rank)
    fail(PJRT_Error_Code_INTERNAL, "scatter ranks out of range");
  if (a.idx_dtype < DT_S8 || a.idx_dtype > DT_U64) fail(PJRT_Error_Code_INTERNAL, "scatter indices must be integers");
  if (a.kind < SC_SET || a.kind > SC_OR || (a.elem_bytes == 8 && a.kind != SC_SET))
    fail(PJRT_Error_Code_INTERNAL, "scatter combination");
  int64_t total = 1, windows = 1, welems = 1;
  int walks[WIN_MAX_RANK] = {0, 0, 0, 0, 0, 0};
  for (int r = 0; r < a.upd_rank; ++r) {
    total *= a.upd_shape[r];
    const int d = a.upd_to_op[r], i = a.upd_to_idx[r];
    if ((d >= 0) == (i >= 0)) fail(PJRT_Error_Code_INTERNAL, "scatter update dimension must be a window or a scatter dim");
    if (d >= a.op_rank || (d >= 0 && (++walks[d] > 1 || a.upd_shape[r] != a.win[d])))
      fail(PJRT_Error_Code_INTERNAL, "scatter window dim");
    if (i >= a.idx_rank || i == a.ivd || (i >= 0 && a.upd_shape[r] != a.idx_shape[i]))
      fail(PJRT_Error_Code_INTERNAL, "scatter scatter dim");
    if (d >= 0) welems *= a.upd_shape[r];
    else windows *= a.upd_shape[r];
  }
  if (total != a.total || windows != a.n_windows || welems != a.win_elems)
    fail(PJRT_Error_Code_INTERNAL, "scatter element counts");
  for (int d = 0; d < a.op_rank; ++d) {
    if (a.win[d] < 0 || a.win[d] > a.op_shape[d] || (!walks[d] && a.win[d] != 1))
      fail(PJRT_Error_Code_INTERNAL, "scatter window size");
    const int b = a.op_batch[d];
    if (b >= a.idx_rank || b == a.ivd || (b >= 0 && (a.idx_shape[b] != a.op_shape[d] || walks[d])))
      fail(PJRT_Error_Code_INTERNAL, "scatter batching dim");
  }
  for (int k = 0; k < a.n_map; ++k)
    if (a.map[k] < 0 || a.map[k] >= a.op_rank || a.op_batch[a.map[k]] >= 0)
      fail(PJRT_Error_Code_INTERNAL, "scatter_dims_to_operand_dims");
  if ((a.ivd < a.idx_rank ? a.idx_shape[a.ivd] : 1) != a.n_map) fail(PJRT_Error_Code_INTERNAL, "scatter index vectors");
  if (total == 0) return record_done(done, stream);
  switch (a.elem_bytes) {
    case 1: return launch_scatter_es<1>(a, stream, done);
    case 2: return launch_scatter_es<2>(a, stream, done);
    case 4: return launch_scatter_es<4>(a, stream, done);
    case 8: return launch_scatter_es<8>(a, stream, done);
    default: fail(PJRT_Error_Code_INTERNAL, "scatter element size " + std::to_string(a.elem_bytes));
  }
}

}  // namespace ryft
