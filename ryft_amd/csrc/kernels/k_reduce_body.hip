// reduce with several inputs or a general body (StableHLO reduce, crates/ryft-mlir/src/dialects/stable_hlo/operations/
// functional.rs:109-230): the body program folded over each output's elements, or the argmax / argmin rule, in one
// launch, or in segments folded by a second launch for long rows of few outputs.
#include <hip/hip_runtime.h>

#include <string>

#include "../common.h"
#include "ew_device.h"
#include "ew_vec.h"
#include "kernels.h"
#include "launch.h"

namespace ryft {

// ------------------------------------------------------------------------------------------------ general bodies
// x ← body(x, y) over the N values of a reduce (the body program, staged in LDS as T, reads x as EW_ACC 0..N-1 and
// y as EW_ACC N..2N-1).
__device__ __forceinline__ void body_fold(const EwProgram& B, const EwTables* T, int n, uint32_t* x,
                                          const uint32_t* y) {
  uint32_t in[2 * RED_MAX_N];
#pragma unroll
  for (int i = 0; i < RED_MAX_N; ++i) {
    in[i] = x[i];
    in[RED_MAX_N + i] = y[i];
  }
  if (n < RED_MAX_N) in[n] = y[0];  // (n = 1: the folded value is EW_ACC 1)
  RegFile1 R;
  ew_run_v<1>(B, 0, nullptr, in, R, 0, -1, T);
#pragma unroll
  for (int i = 0; i < RED_MAX_N; ++i)
    if (i < n) x[i] = R.get(B.out_reg[i]);
}

// argmax / argmin: does the pair (x, position xi) replace (y, yi)? A NaN beats every number; equal values (and two
// NaNs) go to the lower position.
template <int KIND>
__device__ __forceinline__ bool arg_better(uint32_t x, uint32_t xi, uint32_t y, uint32_t yi, int vc) {
  const bool lower = (int32_t)xi < (int32_t)yi;
  if (vc == VC_FLOAT) {
    const float a = __uint_as_float(x), b = __uint_as_float(y);
    const bool an = a != a, bn = b != b;
    if (an | bn) return an && (!bn || lower);
    if (a == b) return lower;
    return KIND == ARG_MAX ? a > b : a < b;
  }
  if (x == y) return lower;
  if (vc == VC_SIGNED) return KIND == ARG_MAX ? (int32_t)x > (int32_t)y : (int32_t)x < (int32_t)y;
  return KIND == ARG_MAX ? x > y : x < y;
}

// x ← x ⊕ y: the body program, or the argmax / argmin rule (x[val] / y[val] the values, the others the positions)
template <int KIND>
__device__ __forceinline__ void fold(const ReduceBodyArgs& A, const EwTables* TB, uint32_t* x, const uint32_t* y) {
  if constexpr (KIND == ARG_NONE) {
    body_fold(A.body, TB, A.n, x, y);
  } else {
    const bool v0 = A.val == 0;
    if (arg_better<KIND>(v0 ? y[0] : y[1], v0 ? y[1] : y[0], v0 ? x[0] : x[1], v0 ? x[1] : x[0], A.value_class)) {
      x[0] = y[0];
      x[1] = y[1];
    }
  }
}

// the init values folded with a result (init first), stored as output element o
template <int KIND>
__device__ __forceinline__ void finish_output(const ReduceBodyArgs& A, const EwTables* TB, int64_t o,
                                              const uint32_t* acc, bool have) {
  uint32_t res[RED_MAX_N];
#pragma unroll
  for (int i = 0; i < RED_MAX_N; ++i)
    res[i] = i >= A.n ? 0u : (A.init_ptr[i] ? load_bits(A.init_ptr[i], 0, A.init_dtype[i]) : A.init[i]);
  if (have) fold<KIND>(A, TB, res, acc);
#pragma unroll
  for (int i = 0; i < RED_MAX_N; ++i)
    if (i < A.n) store_bits(A.out[i], o, A.out_dtype[i], res[i], A.out_float[i] != 0);
}

// G threads per (output, segment) item (256: a workgroup, 64: a wavefront). Each thread folds every G-th element of
// the segment, starting from its first one (no identity is known for a general body); the threads' values are
// folded across lanes with shuffles and, for G = 256, across wavefronts through LDS. With one segment per output the
// init values are folded in last and the output stored; otherwise the segment's value goes to the workspace.
// argmax / argmin scan key: an int32 whose signed order is the rule's preference — the value's order (reversed for
// argmin), NaN above everything, -0 equal to +0 — so that a scan in position order keeps the first element of the
// largest key.
template <int KIND, int VC>
__device__ __forceinline__ int32_t arg_key(uint32_t b) {
  int32_t ord;
  if constexpr (VC == VC_FLOAT) {
    const uint32_t mag = b & 0x7fffffffu;
    if (mag > 0x7f800000u) return INT32_MAX;  // NaN
    if (mag == 0) b = 0;                      // -0 ties with +0
    ord = (int32_t)(b ^ ((uint32_t)((int32_t)b >> 31) & 0x7fffffffu));
  } else if constexpr (VC == VC_UNSIGNED) {
    ord = (int32_t)(b ^ 0x80000000u);
  } else {
    ord = (int32_t)b;
  }
  return KIND == ARG_MAX ? ord : ~ord;
}

// MODE: 0 the prologue run per element, 1 per VEC elements; argmax / argmin of contiguous rows whose prologue is a
// plain load, without running it: 2 f32, 3 bf16, 4 s32, 5 u32 values read straight from the row as 16-byte loads,
// four chunks of VEC elements in flight per thread, each thread scanning its elements in position order by key.
template <int G, bool COORDS, int KIND, int MODE>
__global__ void __launch_bounds__(256) reduce_body_kernel(const ReduceBodyArgs A) {
  __shared__ EwTables TP, TB;
  __shared__ uint32_t part[4][RED_MAX_N + 1];
  const EwProgram& P = A.prologue;
  if constexpr (MODE < 2) stage_tables(P, &TP);
  if constexpr (KIND == ARG_NONE) stage_tables(A.body, &TB);
  if constexpr (MODE < 2 || KIND == ARG_NONE) __syncthreads();
  constexpr int RB = 256 / G;  // items per workgroup
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = threadIdx.x / G, t = threadIdx.x % G;
  const int64_t items = A.outer * A.segs;
  for (int64_t it = (int64_t)blockIdx.x * RB + g; it < items; it += (int64_t)gridDim.x * RB) {
    const int64_t o = it / A.segs, seg = it % A.segs;
    const int64_t r0 = seg * A.seg_len, r1 = A.inner < r0 + A.seg_len ? A.inner : r0 + A.seg_len;
    uint32_t acc[RED_MAX_N] = {};
    bool have = false;
    // element r's values (v) folded into acc
    auto take = [&](uint32_t* v) {
      if (have) {
        fold<KIND>(A, &TB, acc, v);
      } else {
#pragma unroll
        for (int i = 0; i < RED_MAX_N; ++i) acc[i] = v[i];
        have = true;
      }
    };
    if constexpr (MODE >= 2) {
      // the row's values read directly: element r of output o at leaf offset + o·inner + r
      constexpr int ES = MODE == 3 ? 2 : 4;
      constexpr int VC = MODE <= 3 ? VC_FLOAT : (MODE == 4 ? VC_SIGNED : VC_UNSIGNED);
      const EwLeaf& L = P.leaves[0];
      const char* row = (const char*)L.ptr + (L.offset + o * A.inner) * ES;
      auto values = [&](int64_t c, uint32_t* x) {  // chunk c: elements c·VEC .. c·VEC + VEC - 1
        uint32_t w[VEC * ES / 4];
        load_words<VEC * ES>(row + c * VEC * ES, w);
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          x[e] = ES == 4 ? w[e] : ((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
      };
      int32_t bk = 0;
      uint32_t bv = 0, bp = 0;
      bool bh = false;
      auto take_chunk = [&](int64_t c, const uint32_t* x) {  // (chunks arrive in position order)
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const int32_t k = arg_key<KIND, VC>(x[e]);
          const bool rep = !bh || k > bk;
          bk = rep ? k : bk;
          bv = rep ? x[e] : bv;
          bp = rep ? (uint32_t)(c * VEC + e) : bp;
          bh = true;
        }
      };
      const int64_t c1 = r1 / VEC;
      for (int64_t c = r0 / VEC + t; c < c1; c += 4 * G) {  // (the loads of all four chunks issued before any use)
        uint32_t x[4][VEC];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (c + u * G < c1) values(c + u * G, x[u]);
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (c + u * G < c1) take_chunk(c + u * G, x[u]);
      }
      if (bh) {
        acc[0] = A.val == 0 ? bv : bp;
        acc[1] = A.val == 0 ? bp : bv;
        have = true;
      }
    } else if constexpr (MODE == 1) {
      // VEC consecutive elements per program run (segment bounds and the row are multiples of VEC)
      VRegs R;
      for (int64_t c = r0 / VEC + t; c < r1 / VEC; c += G) {
        const int64_t lin = o * A.inner + c * VEC;
        int32_t coord[EW_MAX_RANK];
        if (COORDS) decompose_fast(lin, P, coord);
        ew_run_v<VEC>(P, lin, coord, nullptr, R, 0, -1, &TP);
        uint32_t x0[VEC], x1[VEC];
        R.load(P.out_reg[0], x0);
        if (KIND == ARG_NONE && A.n > 1) R.load(P.out_reg[1], x1);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          uint32_t v[RED_MAX_N];
          const uint32_t pos = (uint32_t)(c * VEC + e);
          if constexpr (KIND == ARG_NONE) {
            v[0] = x0[e];
            v[1] = A.n > 1 ? x1[e] : 0u;
          } else {
            v[0] = A.val == 0 ? x0[e] : pos;
            v[1] = A.val == 0 ? pos : x0[e];
          }
          take(v);
        }
      }
    } else {
      for (int64_t r = r0 + t; r < r1; r += G) {
        const int64_t lin = o * A.inner + r;
        int32_t coord[EW_MAX_RANK];
        if (COORDS) decompose_fast(lin, P, coord);
        RegFile1 R;
        ew_run_v<1>(P, lin, coord, nullptr, R, 0, -1, &TP);
        uint32_t v[RED_MAX_N];
        if constexpr (KIND == ARG_NONE) {
#pragma unroll
          for (int i = 0; i < RED_MAX_N; ++i) v[i] = i < A.n ? R.get(P.out_reg[i]) : 0u;
        } else {  // the value from the prologue, the position from the element's index
          const uint32_t x = R.get(P.out_reg[0]);
          v[0] = A.val == 0 ? x : (uint32_t)r;
          v[1] = A.val == 0 ? (uint32_t)r : x;
        }
        take(v);
      }
    }
    // across the wavefront (every lane of it works on this item)
    for (int off = 32; off > 0; off >>= 1) {
      uint32_t y[RED_MAX_N];
#pragma unroll
      for (int i = 0; i < RED_MAX_N; ++i) y[i] = (uint32_t)__shfl_xor((int)acc[i], off, 64);
      const bool yh = __shfl_xor((int)have, off, 64) != 0;
      if (have && yh) {
        fold<KIND>(A, &TB, acc, y);
      } else if (yh) {
#pragma unroll
        for (int i = 0; i < RED_MAX_N; ++i) acc[i] = y[i];
        have = true;
      }
    }
    bool write = lane == 0;
    if constexpr (G == 256) {
      if (lane == 0) {
#pragma unroll
        for (int i = 0; i < RED_MAX_N; ++i) part[wave][i] = acc[i];
        part[wave][RED_MAX_N] = have;
      }
      __syncthreads();
      write = threadIdx.x == 0;
      if (write) {
        for (int w = 1; w < 4; ++w) {
          if (!part[w][RED_MAX_N]) continue;
          if (have) {
            fold<KIND>(A, &TB, acc, part[w]);
          } else {
#pragma unroll
            for (int i = 0; i < RED_MAX_N; ++i) acc[i] = part[w][i];
            have = true;
          }
        }
      }
    }
    if (write) {
      if (A.segs > 1) {
        uint32_t* w = (uint32_t*)A.ws + it * (RED_MAX_N + 1);
#pragma unroll
        for (int i = 0; i < RED_MAX_N; ++i) w[i] = acc[i];
        w[RED_MAX_N] = have;
      } else {
        finish_output<KIND>(A, &TB, o, acc, have);
      }
    }
    if constexpr (G == 256) __syncthreads();  // part[] is reused by the next item
  }
}

// Second launch for segmented rows: a wavefront per output, its lanes folding every 64th segment's value, then the
// lanes' values across the wavefront and the init values.
template <int KIND>
__global__ void __launch_bounds__(256) reduce_body_finish_kernel(const ReduceBodyArgs A) {
  __shared__ EwTables TB;
  if constexpr (KIND == ARG_NONE) stage_tables(A.body, &TB);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int64_t o = (int64_t)blockIdx.x * 4 + wave; o < A.outer; o += (int64_t)gridDim.x * 4) {
    uint32_t acc[RED_MAX_N] = {};
    bool have = false;
    auto take = [&](const uint32_t* y, bool yh) {
      if (have && yh) {
        fold<KIND>(A, &TB, acc, y);
      } else if (yh) {
#pragma unroll
        for (int i = 0; i < RED_MAX_N; ++i) acc[i] = y[i];
        have = true;
      }
    };
    for (int64_t seg = lane; seg < A.segs; seg += 64) {
      const uint32_t* w = (const uint32_t*)A.ws + (o * A.segs + seg) * (RED_MAX_N + 1);
      uint32_t y[RED_MAX_N];
#pragma unroll
      for (int i = 0; i < RED_MAX_N; ++i) y[i] = w[i];
      take(y, w[RED_MAX_N] != 0);
    }
    for (int off = 32; off > 0; off >>= 1) {
      uint32_t y[RED_MAX_N];
#pragma unroll
      for (int i = 0; i < RED_MAX_N; ++i) y[i] = (uint32_t)__shfl_xor((int)acc[i], off, 64);
      take(y, __shfl_xor((int)have, off, 64) != 0);
    }
    if (lane == 0) finish_output<KIND>(A, &TB, o, acc, have);
  }
}

template <int G, int KIND>
static void launch_reduce_body_g(const ReduceBodyArgs& a, bool coords, int mode, dim3 grid, hipStream_t stream,
                                 hipEvent_t done) {
  dim3 block(256);
  if constexpr (KIND != ARG_NONE) {
    if (mode == 2) return launch_k(done, reduce_body_kernel<G, false, KIND, 2>, grid, block, 0, stream, a);
    if (mode == 3) return launch_k(done, reduce_body_kernel<G, false, KIND, 3>, grid, block, 0, stream, a);
    if (mode == 4) return launch_k(done, reduce_body_kernel<G, false, KIND, 4>, grid, block, 0, stream, a);
    if (mode == 5) return launch_k(done, reduce_body_kernel<G, false, KIND, 5>, grid, block, 0, stream, a);
  }
  if (mode == 1) {
    if (coords) launch_k(done, reduce_body_kernel<G, true, KIND, 1>, grid, block, 0, stream, a);
    else launch_k(done, reduce_body_kernel<G, false, KIND, 1>, grid, block, 0, stream, a);
  } else {
    if (coords) launch_k(done, reduce_body_kernel<G, true, KIND, 0>, grid, block, 0, stream, a);
    else launch_k(done, reduce_body_kernel<G, false, KIND, 0>, grid, block, 0, stream, a);
  }
}

template <int KIND>
static void launch_reduce_body_kind(const ReduceBodyArgs& a0, hipStream_t stream, hipEvent_t done) {
  ReduceBodyArgs a = a0;
  // VEC elements per program run when the rows and segments are whole VEC-element chunks and the prologue's leaves
  // can be read VEC-wide
  const bool vect = a.inner % VEC == 0 && a.seg_len % VEC == 0 && prepare_vec(a.prologue, false);
  int mode = vect ? 1 : 0;
  if (vect && KIND != ARG_NONE && a.prologue.n_instr == 1 && a.prologue.instr[0].op == EW_LOAD &&
      a.prologue.n_leaves == 1 && a.prologue.leaves[0].kind == EW_LEAF_IDENTITY &&
      a.prologue.leaves[0].vmode == EW_VEC_CONTIG) {
    // a plain load of the contiguous rows (aligned to whole chunks: prepare_vec checked the leaf)
    // (the leaf's type is the value's: a plain load converts nothing)
    const int dt = a.prologue.leaves[0].dtype;
    if (dt == DT_F32) mode = 2;
    else if (dt == DT_BF16) mode = 3;
    else if (dt == DT_S32) mode = 4;
    else if (dt == DT_U32) mode = 5;
  }
  const bool coords = a.prologue.needs_coords != 0;
  const bool two = a.segs > 1;
  hipEvent_t first = two ? nullptr : done;
  const int64_t items = a.outer * a.segs;
  if (a.seg_len >= 4096) {  // long segments: a workgroup per item
    dim3 grid((unsigned)(items < 256 * 16 ? items : 256 * 16));
    launch_reduce_body_g<256, KIND>(a, coords, mode, grid, stream, first);
  } else {  // a wavefront per item
    int64_t blocks = (items + 3) / 4;
    if (blocks > 256 * 16) blocks = 256 * 16;
    launch_reduce_body_g<64, KIND>(a, coords, mode, dim3((unsigned)blocks), stream, first);
  }
  dim3 block(256);
  if (two) {
    int64_t blocks = (a.outer + 3) / 4;
    if (blocks > 256 * 16) blocks = 256 * 16;
    launch_k(done, reduce_body_finish_kernel<KIND>, dim3((unsigned)blocks), block, 0, stream, a);
  }
}

void launch_reduce_body(const ReduceBodyArgs& a, hipStream_t stream, hipEvent_t done) {
  const bool arg = a.arg_kind != ARG_NONE;
  if (a.n < 1 || a.n > RED_MAX_N || a.prologue.n_out != (arg ? 1 : a.n) || (!arg && a.body.n_out != a.n) ||
      a.body.n_leaves != 0 || a.segs < 1 || a.seg_len < 1 || (a.segs > 1 && !a.ws) || a.seg_len * a.segs < a.inner ||
      (arg && (a.n != 2 || (a.val != 0 && a.val != 1) || a.inner > INT32_MAX)))
    fail(PJRT_Error_Code_INTERNAL, "reduce body step with inconsistent arguments");
  if (a.outer == 0) return record_done(done, stream);
  switch (a.arg_kind) {
    case ARG_MAX: launch_reduce_body_kind<ARG_MAX>(a, stream, done); break;
    case ARG_MIN: launch_reduce_body_kind<ARG_MIN>(a, stream, done); break;
    default: launch_reduce_body_kind<ARG_NONE>(a, stream, done); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail(PJRT_Error_Code_INTERNAL, std::string("reduce launch failed: ") + hipGetErrorString(e));
}

}  // namespace ryft
