// Elementwise programs and reductions (HBM-bound). Each thread evaluates the program's instruction list on VEC = 8
// consecutive elements of the innermost dimension at once, so the (uniform) instruction dispatch is paid once per 8
// elements and contiguous leaves / outputs move as 8- to 32-byte vectors; the program's registers stay in VGPRs.
// Shapes whose innermost dimension is not a multiple of 8 run the same program one element per thread (registers in
// VGPRs). Reductions give each output row a workgroup (long rows, e.g. RMSNorm's 4096) or one wavefront (shorter
// rows), combine within the thread, across lanes with shuffles and across wavefronts through LDS; the init value
// enters once at the end.
#include <hip/hip_runtime.h>

#include <string>
#include <type_traits>

#include "../common.h"
#include "ew_device.h"
#include "ew_vec.h"
#include "kernels.h"
#include "launch.h"

namespace ryft {

template <bool COORDS>
__global__ void __launch_bounds__(256) ew_kernel(const EwProgram P) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t lin = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; lin < P.total; lin += stride) {
    int32_t coord[EW_MAX_RANK];
    if (COORDS) decompose(lin, P, coord);
    RegFile1 R;
    ew_run(P, lin, coord, nullptr, R);
    if (COORDS && P.out_strided) {
      int64_t off = P.out_offset;
      for (int d = 0; d < P.rank; ++d) off += (int64_t)coord[d] * P.out_strides[d];
      store_bits(P.out_ptr[0], off, P.out_dtype[0], R.get(P.out_reg[0]), P.out_float_mask & 1);
      continue;
    }
    for (int o = 0; o < P.n_out; ++o)
      store_bits(P.out_ptr[o], lin, P.out_dtype[o], R.get(P.out_reg[o]), (P.out_float_mask >> o) & 1);
  }
}


// Stores V consecutive register values (float bits if `is_float`, else int32) as `dtype` at out[lin..lin+V).
// 16- / 8-byte vector store, non-temporal (streamed past the caches, for data no kernel re-reads soon) when NT.
template <bool NT, typename T>
__device__ __forceinline__ void vstore(char* p, const T& v) {
  if constexpr (NT) __builtin_nontemporal_store(v, (T*)p);
  else *(T*)p = v;
}

// N consecutive 32-bit words as 16-byte stores, then an 8- and a 4-byte store for the rest.
template <bool NT, int N>
__device__ __forceinline__ void store_words_nt(char* p, const uint32_t* w) {
#pragma unroll
  for (int i = 0; i + 4 <= N; i += 4) vstore<NT>(p + 4 * i, u32x4v{w[i], w[i + 1], w[i + 2], w[i + 3]});
  constexpr int R = N & ~3;
  if constexpr ((N & 3) >= 2) vstore<NT>(p + 4 * R, u32x2v{w[R], w[R + 1]});
  if constexpr (N & 1) vstore<NT>(p + 4 * (N - 1), w[N - 1]);
}

template <int V, bool NT = false>
__device__ __forceinline__ void store_vec(void* out, int64_t lin, int dtype, const uint32_t* v, bool is_float) {
  static_assert(V == 4 || V == 8, "vector stores are written for 4 or 8 elements");
  char* p = (char*)out;
  switch (dtype) {
    case DT_F32: case DT_S32: case DT_U32: {
      uint32_t w[V];
#pragma unroll
      for (int e = 0; e < V; ++e) w[e] = (dtype != DT_F32 || is_float) ? v[e] : __float_as_uint((float)(int32_t)v[e]);
      vstore<NT>(p + lin * 4, u32x4v{w[0], w[1], w[2], w[3]});
      if constexpr (V == 8) vstore<NT>(p + lin * 4 + 16, u32x4v{w[4], w[5], w[6], w[7]});
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
      if constexpr (V == 8) vstore<NT>(p + lin * 2, u32x4v{w[0], w[1], w[2], w[3]});
      else vstore<NT>(p + lin * 2, u32x2v{w[0], w[1]});
      break;
    }
    case DT_F8E4M3FN: case DT_F8E5M2: case DT_S8: case DT_U8: case DT_PRED: {
      // one uniform branch per vector, then straight-line conversion of its V elements
      if (dtype == DT_F8E4M3FN && is_float) {
        uint32_t w[V / 4];
#pragma unroll
        for (int q = 0; q < V / 4; ++q)
          w[q] = f32x4_to_e4m3fn_bits(__uint_as_float(v[4 * q]), __uint_as_float(v[4 * q + 1]),
                                      __uint_as_float(v[4 * q + 2]), __uint_as_float(v[4 * q + 3]));
        if constexpr (V == 8) vstore<NT>(p + lin, u32x2v{w[0], w[1]});
        else vstore<NT>(p + lin, w[0]);
        break;
      }
      uint32_t byte[V];
      if (dtype == DT_F8E4M3FN) {
#pragma unroll
        for (int e = 0; e < V; ++e) byte[e] = f32_to_e4m3fn_bits(is_float ? __uint_as_float(v[e]) : (float)(int32_t)v[e]);
      } else if (dtype == DT_F8E5M2) {
#pragma unroll
        for (int e = 0; e < V; ++e) byte[e] = f32_to_e5m2_bits(is_float ? __uint_as_float(v[e]) : (float)(int32_t)v[e]);
      } else if (dtype == DT_PRED) {
#pragma unroll
        for (int e = 0; e < V; ++e) byte[e] = v[e] != 0;
      } else if (is_float) {
#pragma unroll
        for (int e = 0; e < V; ++e) byte[e] = (uint32_t)f2i_sat(__uint_as_float(v[e]), dtype) & 0xffu;
      } else {
#pragma unroll
        for (int e = 0; e < V; ++e) byte[e] = v[e] & 0xffu;
      }
      uint32_t w[V / 4];
#pragma unroll
      for (int q = 0; q < V / 4; ++q)
        w[q] = byte[4 * q] | (byte[4 * q + 1] << 8) | (byte[4 * q + 2] << 16) | (byte[4 * q + 3] << 24);
      if constexpr (V == 8) vstore<NT>(p + lin, u32x2v{w[0], w[1]});
      else vstore<NT>(p + lin, w[0]);
      break;
    }
    default:
#pragma unroll
      for (int e = 0; e < V; ++e) store_bits(out, lin + e, dtype, v[e], is_float);
      break;
  }
}

template <bool COORDS, int NR>
__global__ void __launch_bounds__(VNT) ew_kernel_vec(const EwProgram P) {
  __shared__ EwTables T;
  stage_tables(P, &T);
  __syncthreads();
  SwitchRegFile<VEC, NR> R;
  const int64_t chunks = P.total / VEC;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < chunks; c += stride) {
    const int64_t lin = c * VEC;
    int32_t coord[EW_MAX_RANK];
    if (COORDS) decompose_fast(lin, P, coord);
    ew_run_v<VEC>(P, lin, coord, nullptr, R, 0, -1, &T);
    for (int o = 0; o < P.n_out; ++o) {
      uint32_t v[VEC];
      R.load(P.out_reg[o], v);
      store_vec<VEC>(P.out_ptr[o], lin, P.out_dtype[o], v, (P.out_float_mask >> o) & 1);
    }
  }
}

// Streaming form for maps without coordinates over at most two contiguous leaves of one element size ES (a negate,
// a convert, a scaled residual add): one chunk per thread over a grid that covers the whole iteration space, the raw
// leaf words fetched as straight-line vector loads (ES is a template parameter, so nothing touches their registers
// before the computation) and, for steps that stream more data than the caches hold (NT), loaded and stored
// non-temporally. Measured on MI355X, one 16-byte chunk per thread over an oversubscribed grid with non-temporal
// accesses streams a copy at ~6.6 TB/s, against ~5.5 TB/s for a grid-stride loop over a capped grid.
template <int ES, bool NT>
__device__ __forceinline__ void fetch_raw(const void* base, int64_t elem, uint32_t* w) {
  const char* p = (const char*)base + elem * ES;
  auto ld4 = [](const char* q) { return NT ? __builtin_nontemporal_load((const u32x4v*)q) : *(const u32x4v*)q; };
  if constexpr (ES == 4) {
    const u32x4v a = ld4(p), b = ld4(p + 16);
    w[0] = a.x, w[1] = a.y, w[2] = a.z, w[3] = a.w, w[4] = b.x, w[5] = b.y, w[6] = b.z, w[7] = b.w;
  } else if constexpr (ES == 2) {
    const u32x4v a = ld4(p);
    w[0] = a.x, w[1] = a.y, w[2] = a.z, w[3] = a.w;
  } else {
    const u32x2v a = NT ? __builtin_nontemporal_load((const u32x2v*)p) : *(const u32x2v*)p;
    w[0] = a.x, w[1] = a.y;
  }
}

template <int NR, int ES, bool NT>
__global__ void __launch_bounds__(VNT) ew_stream_kernel(const EwProgram P) {
  static_assert(ES == 1 || ES == 2 || ES == 4, "leaf element size");
  __shared__ EwTables T;
  stage_tables(P, &T);
  __syncthreads();
  SwitchRegFile<VEC, NR> R;
  const int64_t chunks = P.total / VEC;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const bool two = P.n_leaves > 1;
  const char* p0 = (const char*)P.leaves[0].ptr + P.leaves[0].offset * ES;
  const char* p1 = (const char*)P.leaves[two ? 1 : 0].ptr + P.leaves[two ? 1 : 0].offset * ES;
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < chunks; c += stride) {
    uint32_t a[2 * VEC];  // (the second half is set and read only with two leaves)
    fetch_raw<ES, NT>(p0, c * VEC, a);
    if (two) fetch_raw<ES, NT>(p1, c * VEC, a + VEC);
    ew_run_v<VEC, SwitchRegFile<VEC, NR>, true>(P, c * VEC, nullptr, a, R, 0, -1, &T);
    for (int o = 0; o < P.n_out; ++o) {
      uint32_t v[VEC];
      R.load(P.out_reg[o], v);
      store_vec<VEC, NT>(P.out_ptr[o], c * VEC, P.out_dtype[o], v, (P.out_float_mask >> o) & 1);
    }
  }
}

// Direct form of the commonest streaming maps: one float operation (negate, abs, add, subtract, multiply, divide,
// maximum, minimum, convert) over one or two contiguous leaves of one type (f32 or bf16), or a leaf and a constant,
// written as f32 or bf16 — with no interpreter: the operation is picked by a uniform switch outside the element
// loop, each thread takes one 16-byte vector per leaf, and the grid covers the iteration space (a probe of this
// shape streams a 256 MiB copy at ~6.6 TB/s). Same arithmetic and rounding as the interpreter's instructions.
struct MapArgs {
  const void* a;
  const void* b;      // second leaf, or null (constant operand or unary)
  void* out;
  uint32_t imm;       // constant operand (f32 bits)
  int32_t op;         // EwOp
  int32_t b_kind;     // 0 none, 1 leaf, 2 constant
  int32_t b_first;    // the leaf / constant is the first operand (a - b with the constant on the left)
  int64_t chunks;     // 16-byte input vectors
};

template <int OP>
__device__ __forceinline__ float map_op(float x, float y) {
  if constexpr (OP == EW_NEG) return -x;
  else if constexpr (OP == EW_ABS) return fabsf(x);
  else if constexpr (OP == EW_CVT_F2F) return x;
  else if constexpr (OP == EW_ADD) return x + y;
  else if constexpr (OP == EW_SUB) return x - y;
  else if constexpr (OP == EW_MUL) return x * y;
  else if constexpr (OP == EW_DIV) return x / y;
  else if constexpr (OP == EW_MAX) return (x != x || y != y) ? __uint_as_float(0x7fc00000u) : fmaxf(x, y);
  else return (x != x || y != y) ? __uint_as_float(0x7fc00000u) : fminf(x, y);  // EW_MIN
}

// ES: leaf element size (4: f32, 2: bf16); OUT_BF16: results rounded to and stored as bf16
template <int OP, int ES, bool OUT_BF16, bool NT>
__device__ __forceinline__ void map_loop(const MapArgs& A) {
  constexpr int V = 16 / ES;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < A.chunks; c += stride) {
    const u32x4v wa = NT ? __builtin_nontemporal_load((const u32x4v*)A.a + c) : ((const u32x4v*)A.a)[c];
    u32x4v wb = u32x4v{A.imm, A.imm, A.imm, A.imm};
    if (A.b_kind == 1) wb = NT ? __builtin_nontemporal_load((const u32x4v*)A.b + c) : ((const u32x4v*)A.b)[c];
    float r[V];
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const uint32_t ua = ES == 4 ? wa[e] : ((e & 1) ? (wa[e >> 1] & 0xffff0000u) : (wa[e >> 1] << 16));
      const uint32_t ub = A.b_kind != 1 ? A.imm : ES == 4 ? wb[e] : ((e & 1) ? (wb[e >> 1] & 0xffff0000u) : (wb[e >> 1] << 16));
      const float x = __uint_as_float(ua), y = __uint_as_float(ub);
      r[e] = A.b_first ? map_op<OP>(y, x) : map_op<OP>(x, y);
    }
    if constexpr (OUT_BF16) {
      uint32_t w[V / 2];
#pragma unroll
      for (int q = 0; q < V / 2; ++q) w[q] = f32x2_to_bf16x2_bits(r[2 * q], r[2 * q + 1]);
      store_words_nt<NT, V / 2>((char*)A.out + c * (V * 2), w);
    } else {
      uint32_t w[V];
#pragma unroll
      for (int e = 0; e < V; ++e) w[e] = __float_as_uint(r[e]);
      store_words_nt<NT, V>((char*)A.out + c * (V * 4), w);
    }
  }
}

template <int ES, bool OUT_BF16, bool NT>
__global__ void __launch_bounds__(256) ew_map_kernel(const MapArgs A) {
  switch (A.op) {
    case EW_NEG: map_loop<EW_NEG, ES, OUT_BF16, NT>(A); break;
    case EW_ABS: map_loop<EW_ABS, ES, OUT_BF16, NT>(A); break;
    case EW_CVT_F2F: map_loop<EW_CVT_F2F, ES, OUT_BF16, NT>(A); break;
    case EW_ADD: map_loop<EW_ADD, ES, OUT_BF16, NT>(A); break;
    case EW_SUB: map_loop<EW_SUB, ES, OUT_BF16, NT>(A); break;
    case EW_MUL: map_loop<EW_MUL, ES, OUT_BF16, NT>(A); break;
    case EW_DIV: map_loop<EW_DIV, ES, OUT_BF16, NT>(A); break;
    case EW_MAX: map_loop<EW_MAX, ES, OUT_BF16, NT>(A); break;
    case EW_MIN: map_loop<EW_MIN, ES, OUT_BF16, NT>(A); break;
    default: break;
  }
}

// Recognises a program of that form: loads and constants, then one such operation whose result is the one output.
static bool map_args(const EwProgram& v, MapArgs* m) {
  if (v.n_out != 1 || v.needs_coords || v.out_strided || v.n_leaves < 1 || v.n_leaves > 2 || v.n_instr < 2) return false;
  const int ldt = v.leaves[0].dtype;
  if (ldt != DT_F32 && ldt != DT_BF16) return false;
  const int es = ldt == DT_F32 ? 4 : 2;
  for (int i = 0; i < v.n_leaves; ++i) {
    const EwLeaf& L = v.leaves[i];
    if (L.dtype != ldt || L.kind == EW_LEAF_SCALAR || L.vmode != EW_VEC_CONTIG) return false;
    if (((uintptr_t)L.ptr + (uintptr_t)(L.offset * es)) % 16) return false;
  }
  // sources of the registers before the operation: leaf index (>= 0), constant (-2), undefined (-1)
  int src[EW_MAX_REGS];
  uint32_t imm[EW_MAX_REGS];
  for (int r = 0; r < EW_MAX_REGS; ++r) src[r] = -1, imm[r] = 0;
  for (int i = 0; i + 1 < v.n_instr; ++i) {
    const EwInstr& I = v.instr[i];
    if (I.dst >= EW_MAX_REGS) return false;
    if (I.op == EW_LOAD && (I.round == 0 || I.round == ldt)) src[I.dst] = I.a;
    else if (I.op == EW_CONST) src[I.dst] = -2, imm[I.dst] = I.imm.u;
    else return false;
  }
  const EwInstr& I = v.instr[v.n_instr - 1];
  const bool unary = I.op == EW_NEG || I.op == EW_ABS || I.op == EW_CVT_F2F;
  const bool binary = I.op == EW_ADD || I.op == EW_SUB || I.op == EW_MUL || I.op == EW_DIV || I.op == EW_MAX ||
                      I.op == EW_MIN;
  if (!(unary || binary) || I.dst != v.out_reg[0] || I.a >= EW_MAX_REGS || (binary && I.b >= EW_MAX_REGS)) return false;
  const int round = I.round == 0 ? DT_F32 : I.round;
  if ((round != DT_F32 && round != DT_BF16) || v.out_dtype[0] != round || !(v.out_float_mask & 1)) return false;
  if ((uintptr_t)v.out_ptr[0] % 16) return false;
  if (v.total % (16 / es)) return false;
  // the first operand comes from a leaf; the second (binary) from a leaf or a constant, either side
  int sa = src[I.a], sb = binary ? src[I.b] : -3;
  bool b_first = false;
  if (binary && sa == -2 && sb >= 0) std::swap(sa, sb), b_first = true;
  if (sa < 0 || (binary && sb == -1)) return false;
  m->a = (const char*)v.leaves[sa].ptr + v.leaves[sa].offset * es;
  m->out = v.out_ptr[0];
  m->b = nullptr;
  m->imm = 0;
  m->b_kind = 0;
  if (binary && sb >= 0) m->b = (const char*)v.leaves[sb].ptr + v.leaves[sb].offset * es, m->b_kind = 1;
  if (binary && sb == -2) m->imm = imm[b_first ? I.a : I.b], m->b_kind = 2;
  m->b_first = b_first;
  m->op = I.op;
  m->chunks = v.total / (16 / es);
  return true;
}

// Registers a program touches (one past the highest register it reads or writes).
constexpr int EW_SMALL_REGS = 4;
static int program_regs(const EwProgram& p) {
  int n = 0;
  for (int i = 0; i < p.n_instr; ++i) {
    const EwInstr& I = p.instr[i];
    n = std::max(n, (int)I.dst + 1);
    const int src = ew_nsrc(I.op);
    if (src >= 1) n = std::max(n, (int)I.a + 1);
    if (src >= 2) n = std::max(n, (int)I.b + 1);
    if (src >= 3) n = std::max(n, (int)I.c + 1);
  }
  for (int o = 0; o < p.n_out; ++o) n = std::max(n, (int)p.out_reg[o] + 1);
  return n;
}

static int grid_for(int64_t total, int threads) {
  int64_t blocks = (total + threads - 1) / threads;
  const int64_t cap = 256 * 32;  // 32 blocks per CU is plenty for a grid-stride loop
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  return (int)blocks;
}

void launch_elementwise(const EwProgram& p, hipStream_t stream, hipEvent_t done) {
  if (p.total == 0) return record_done(done, stream);
  if (p.out_strided && (p.n_out != 1 || !p.needs_coords))
    fail(PJRT_Error_Code_INTERNAL, "strided-output elementwise step needs one output and coordinates");
  EwProgram v = p;
  if (!p.out_strided && prepare_vec(v, true)) {
    dim3 grid(grid_for(v.total / VEC, VNT)), block(VNT);
    const bool small = program_regs(v) <= EW_SMALL_REGS;
    bool streaming = !v.needs_coords && v.n_leaves >= 1 && v.n_leaves <= 2 && small;
    const int les = v.n_leaves >= 1 ? elem_size(v.leaves[0].dtype) : 0;
    for (int i = 0; streaming && i < v.n_leaves; ++i)
      streaming = v.leaves[i].vmode == EW_VEC_CONTIG && elem_size(v.leaves[i].dtype) == les;
    for (int i = 0; streaming && i < v.n_instr; ++i) streaming = !ew_is_heavy(v.instr[i].op);
    MapArgs m;
    if (map_args(v, &m)) {
      int64_t bytes = v.total * (int64_t)(elem_size(v.leaves[0].dtype) * (m.b_kind == 1 ? 2 : 1) + elem_size(v.out_dtype[0]));
      const bool nt = bytes >= ((int64_t)256 << 20);
      const bool f32in = v.leaves[0].dtype == DT_F32, bf16out = v.out_dtype[0] == DT_BF16;
      dim3 mgrid((unsigned)std::min<int64_t>((m.chunks + 255) / 256, (int64_t)1 << 20)), mblock(256);
#define RYFT_MAP(ES, OB)                                                                            \
  (nt ? launch_k(done, ew_map_kernel<ES, OB, true>, mgrid, mblock, 0, stream, m)                     \
      : launch_k(done, ew_map_kernel<ES, OB, false>, mgrid, mblock, 0, stream, m))
      if (f32in) { if (bf16out) RYFT_MAP(4, true); else RYFT_MAP(4, false); }
      else { if (bf16out) RYFT_MAP(2, true); else RYFT_MAP(2, false); }
#undef RYFT_MAP
    } else if (streaming) {
      // a chunk per thread (the grid covers the iteration space up to 2^20 workgroups); non-temporal accesses when
      // the step streams more than the 256 MB last-level cache could keep for its consumer anyway
      const int64_t sblocks = grid_for(v.total / VEC, VNT);
      int64_t bytes = 0;
      for (int i = 0; i < v.n_leaves; ++i) bytes += v.total * elem_size(v.leaves[i].dtype);
      for (int o = 0; o < v.n_out; ++o) bytes += v.total * elem_size(v.out_dtype[o]);
      const bool nt = bytes >= ((int64_t)256 << 20);
      dim3 sgrid((unsigned)std::max<int64_t>(sblocks, 1));
#define RYFT_STREAM(ES)                                                                                  \
  (nt ? launch_k(done, ew_stream_kernel<EW_SMALL_REGS, ES, true>, sgrid, block, 0, stream, v)           \
      : launch_k(done, ew_stream_kernel<EW_SMALL_REGS, ES, false>, sgrid, block, 0, stream, v))
      if (les == 4) RYFT_STREAM(4);
      else if (les == 2) RYFT_STREAM(2);
      else RYFT_STREAM(1);
#undef RYFT_STREAM
    } else if (v.needs_coords) {
      if (small) launch_k(done, ew_kernel_vec<true, EW_SMALL_REGS>, grid, block, 0, stream, v);
      else launch_k(done, ew_kernel_vec<true, EW_MAX_REGS>, grid, block, 0, stream, v);
    } else {
      if (small) launch_k(done, ew_kernel_vec<false, EW_SMALL_REGS>, grid, block, 0, stream, v);
      else launch_k(done, ew_kernel_vec<false, EW_MAX_REGS>, grid, block, 0, stream, v);
    }
  } else {
    dim3 grid(grid_for(p.total, 256)), block(256);
    if (p.needs_coords) launch_k(done, ew_kernel<true>, grid, block, 0, stream, p);
    else launch_k(done, ew_kernel<false>, grid, block, 0, stream, p);
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
  __shared__ EwTables T;
  VRegs R;
  const EwProgram& P = A.prologue;
  stage_tables(P, &T);
  __syncthreads();
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
      ew_run_v<VEC>(P, lin, coord, nullptr, R, 0, -1, &T);
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

void launch_reduce(const ReduceArgs& a, hipStream_t stream, hipEvent_t done) {
  if (a.outer == 0) return record_done(done, stream);
  ReduceArgs v = a;
  if (a.inner % VEC == 0 && prepare_vec(v.prologue, false)) {
    const bool coords = v.prologue.needs_coords != 0;
    if (a.inner / VEC >= 2 * VNT) {  // long rows: a workgroup per row
      dim3 grid((unsigned)(a.outer < 256 * 16 ? a.outer : 256 * 16)), block(VNT);
      if (coords) launch_k(done, reduce_kernel_vec<VNT, true>, grid, block, 0, stream, v);
      else launch_k(done, reduce_kernel_vec<VNT, false>, grid, block, 0, stream, v);
    } else {  // a wavefront per row
      int64_t blocks = (a.outer + VNT / 64 - 1) / (VNT / 64);
      if (blocks > 256 * 16) blocks = 256 * 16;
      dim3 grid((unsigned)blocks), block(VNT);
      if (coords) launch_k(done, reduce_kernel_vec<64, true>, grid, block, 0, stream, v);
      else launch_k(done, reduce_kernel_vec<64, false>, grid, block, 0, stream, v);
    }
  } else {
    int64_t blocks = (a.outer + 3) / 4;
    if (blocks > 256 * 16) blocks = 256 * 16;
    dim3 grid((unsigned)blocks), block(256);
    if (a.prologue.needs_coords) launch_k(done, reduce_kernel<true>, grid, block, 0, stream, a);
    else launch_k(done, reduce_kernel<false>, grid, block, 0, stream, a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail(PJRT_Error_Code_INTERNAL, std::string("reduce launch failed: ") + hipGetErrorString(e));
}

}  // namespace ryft

namespace ryft {

// ------------------------------------------------------------------------------------------------ row fusion
// G threads per row (VNT: a workgroup per row, for long rows; 64: a wavefront per row), V consecutive elements per
// program run. Each reduction folds its phase's value over the row within the thread, across lanes with shuffles and
// across wavefronts through LDS; every thread of the row then holds the same row value (one association order,
// broadcast from lane 0 / read from LDS in wave order), combines the init value and rounds to the reduce's type.
// The consumer phase reads the row values through EW_ACC. Rows are short enough to stay in L2 between phases.
template <int G, int V, bool COORDS>
__global__ void __launch_bounds__(VNT) row_kernel(const RowArgs A) {
  __shared__ uint32_t part[VNT / 64];
  __shared__ EwTables T;
  typename std::conditional<V == 1, RegFile1, SwitchRegFile<V>>::type R;
  const EwProgram& P = A.prog;
  stage_tables(P, &T);
  __syncthreads();
  constexpr int RB = VNT / G;  // rows per workgroup
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = threadIdx.x / G, t = threadIdx.x % G;
  const int64_t chunks = A.inner / V;
  for (int64_t o = (int64_t)blockIdx.x * RB + g; o < A.rows; o += (int64_t)gridDim.x * RB) {
    uint32_t rv[ROW_MAX_RED] = {0u, 0u};
    // passes 0 .. n_red-1 fold the reductions, pass n_red runs the consumer; one program-run site keeps the
    // interpreter's code once in the instruction cache
    for (int k = 0; k <= A.n_red; ++k) {
      const bool red = k < A.n_red;
      const bool fl = red && A.is_float[k] != 0;
      const int kind = red ? A.kind[k] : 0;
      const int pb = k == 0 ? 0 : A.phase_end[k - 1], pe = A.phase_end[k];
      uint32_t acc = red ? red_identity(kind, fl) : 0u;
      for (int64_t c = t; c < chunks; c += G) {
        const int64_t lin = o * A.inner + c * V;
        int32_t coord[EW_MAX_RANK];
        if (COORDS) decompose_fast(lin, P, coord);
        ew_run_v<V>(P, lin, coord, rv, R, pb, pe, &T);
        if (red) {
          uint32_t v[V];
          R.load(A.red_reg[k], v);
#pragma unroll
          for (int e = 0; e < V; ++e) acc = red_combine(acc, v[e], kind, fl);
        } else {
          for (int q = 0; q < P.n_out; ++q) {
            uint32_t v[V];
            R.load(P.out_reg[q], v);
            if constexpr (V == 1) store_bits(P.out_ptr[q], lin, P.out_dtype[q], v[0], (P.out_float_mask >> q) & 1);
            else store_vec<V>(P.out_ptr[q], lin, P.out_dtype[q], v, (P.out_float_mask >> q) & 1);
          }
        }
      }
      if (!red) break;
      for (int off = 32; off > 0; off >>= 1) acc = red_combine(acc, (uint32_t)__shfl_xor((int)acc, off, 64), kind, fl);
      acc = (uint32_t)__shfl((int)acc, 0, 64);
      if constexpr (G == VNT) {
        if (lane == 0) part[wave] = acc;
        __syncthreads();
        acc = part[0];
        for (int w = 1; w < VNT / 64; ++w) acc = red_combine(acc, part[w], kind, fl);
        __syncthreads();  // part[] is reused by the next reduction
      }
      acc = red_combine(acc, A.init[k], kind, fl);
      const uint32_t val = fl ? __float_as_uint(round_float(__uint_as_float(acc), A.red_dtype[k]))
                              : (uint32_t)wrap_int((int32_t)acc, A.red_dtype[k]);
      if (k == 0) rv[0] = val;
      else rv[1] = val;
    }
  }
}

// ------------------------------------------------------------------------------------------------ row-norm path
// Eight consecutive elements of a float row as f32 (f32, bf16 or f16 storage; 16-byte aligned groups).
// Raw words of 8 consecutive f32 / bf16 / f16 elements (8 words for f32, 4 for the 16-bit types).
__device__ __forceinline__ void load8_raw(const void* p, int64_t i, int dt, uint32_t* w) {
  const char* c = (const char*)p;
  if (dt == DT_F32) {
    const u32x4v a = *(const u32x4v*)(c + i * 4), b = *(const u32x4v*)(c + i * 4 + 16);
    w[0] = a.x, w[1] = a.y, w[2] = a.z, w[3] = a.w, w[4] = b.x, w[5] = b.y, w[6] = b.z, w[7] = b.w;
  } else {
    const u32x4v a = *(const u32x4v*)(c + i * 2);
    w[0] = a.x, w[1] = a.y, w[2] = a.z, w[3] = a.w;
  }
}

__device__ __forceinline__ void decode8_f32(int dt, const uint32_t* w, float* v) {
  if (dt == DT_F32) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = __uint_as_float(w[e]);
  } else if (dt == DT_BF16) {
#pragma unroll
    for (int q = 0; q < 4; ++q) v[2 * q] = __uint_as_float(w[q] << 16), v[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[2 * q] = (float)__builtin_bit_cast(_Float16, (uint16_t)w[q]);
      v[2 * q + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[q] >> 16));
    }
  }
}

__device__ __forceinline__ void load8_f32(const void* p, int64_t i, int dt, float* v) {
  uint32_t w[8];
  load8_raw(p, i, dt, w);
  decode8_f32(dt, w, v);
}

// Rounds 8 floats to the precision of `dtype` (a no-op for f32): one switch, straight-line element work.
__device__ __forceinline__ void round8(float* y, int dtype) {
  switch (dtype) {
    case DT_BF16:
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const uint32_t pk = f32x2_to_bf16x2_bits(y[e], y[e + 1]);
        y[e] = __uint_as_float(pk << 16), y[e + 1] = __uint_as_float(pk & 0xffff0000u);
      }
      break;
    case DT_F16:
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = round_float(y[e], DT_F16);
      break;
    case DT_F8E4M3FN:
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = round_float(y[e], DT_F8E4M3FN);
      break;
    case DT_F8E5M2:
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = round_float(y[e], DT_F8E5M2);
      break;
    default: break;
  }
}

// The scale 1/√(Σx²·α + ε) of a row from its folded Σx² (the init value enters last, as in the interpreted kernel).
__device__ __forceinline__ float rownorm_scale(const RowArgs& A, float acc) {
  const RowNormArgs& N = A.norm;
  acc = acc + __uint_as_float(A.init[0]);
  float t = N.alpha_div ? acc / N.alpha : acc * N.alpha;
  t = t + N.eps;
  return 1.0f / sqrtf(t);
}

// y = round(x·s·w) for 8 elements, stored as the output type; uniform branches once per vector of 8, straight-line
// element work inside each. NAN_FREE: the caller has shown that no y is a NaN, so an f8E4M3FN output needs no NaN
// sign repair after the hardware conversion.
template <bool NAN_FREE = false>
__device__ __forceinline__ void rownorm_emit(const RowNormArgs& N, int64_t lin, const float* v, const float* wv, float s,
                                             int out_dtype) {
#pragma clang fp contract(off)
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = v[e] * s;
  if (N.w) {
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = y[e] * wv[e];
  }
  round8(y, N.mid_round);
  if (NAN_FREE && out_dtype == DT_F8E4M3FN) {
    // v_cvt_pk_fp8_f32 gives the f8E4M3FN bits of every non-NaN input
    uint32_t w0 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
    w0 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], (int)w0, true);
    uint32_t w1 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(y[4], y[5], 0, false);
    w1 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(y[6], y[7], (int)w1, true);
    vstore<false>((char*)N.out + lin, u32x2v{w0, w1});
    return;
  }
  uint32_t b[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) b[e] = __float_as_uint(y[e]);
  store_vec<8>(N.out, lin, out_dtype, b, true);
}

// RMSNorm rows of at most 64·8·NCW elements, one wavefront per row: lane l owns chunks l, l + 64, ... of 8
// elements, loads them all at once (raw words, XB bytes per element) and keeps them in registers, folds Σx² in
// element order, then across lanes by shuffles and a broadcast from lane 0 — the order of the interpreted row kernel
// for such rows, so both paths give the same bits. No barrier sits between rows, so a compute unit has as many rows
// in flight as it holds waves. The weight row, shared by all rows, is staged once per workgroup in LDS. Products
// and sums are separately rounded f32 operations (no contraction into FMAs), as the program specifies.
template <int NCW, int XB>
__global__ void __launch_bounds__(VNT) rownorm_wave_kernel(const RowArgs A) {
#pragma clang fp contract(off)
  extern __shared__ __attribute__((aligned(16))) char wrow[];
  const RowNormArgs& N = A.norm;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t chunks = A.inner / 8;
  constexpr int W = XB * 2;  // raw words per chunk
  uint32_t xr[NCW][W];
  auto fetch = [&](int64_t o) {
    const char* xrow = (const char*)N.x + o * A.inner * XB;
#pragma unroll
    for (int q = 0; q < NCW; ++q) {
      const int c = lane + 64 * q;
      if (c < chunks) {
#pragma unroll
        for (int h = 0; h < W / 4; ++h) {
          const u32x4v a = *(const u32x4v*)(xrow + (int64_t)c * 8 * XB + 16 * h);
          xr[q][4 * h] = a.x, xr[q][4 * h + 1] = a.y, xr[q][4 * h + 2] = a.z, xr[q][4 * h + 3] = a.w;
        }
      }
    }
  };
  // the first row's words are requested before the weight row is staged (and the barrier that follows it)
  const int64_t first = (int64_t)blockIdx.x * (VNT / 64) + wave;
  if (first < A.rows) fetch(first);
  if (N.w) {
    const int64_t nbytes = A.inner * (N.w_dtype == DT_F32 ? 4 : 2);
    for (int64_t b = threadIdx.x * 16; b < nbytes; b += VNT * 16)
      *(u32x4v*)(wrow + b) = *(const u32x4v*)((const char*)N.w + b);
  }
  __syncthreads();
  auto decode_x = [&](const uint32_t* w, float* v) {
    if constexpr (XB == 4) {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = __uint_as_float(w[e]);
    } else {
      decode8_f32(N.x_dtype, w, v);
    }
  };
  for (int64_t o = first; o < A.rows; o += (int64_t)gridDim.x * (VNT / 64)) {
    if (o != first) fetch(o);
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < NCW; ++q)
      if (lane + 64 * q < chunks) {
        float v[8];
        decode_x(xr[q], v);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = acc + v[e] * v[e];
      }
    for (int off = 32; off > 0; off >>= 1) acc = acc + __shfl_xor(acc, off, 64);
    acc = __shfl(acc, 0, 64);
    const float s = rownorm_scale(A, acc);
    // one loop per output type, so each unrolled loop body holds that type's conversion only
    auto emit_all = [&](auto odt) {
#pragma unroll
      for (int q = 0; q < NCW; ++q) {
        const int c = lane + 64 * q;
        if (c < chunks) {
          float v[8], wv[8];
          decode_x(xr[q], v);
          if (N.w) load8_f32(wrow, (int64_t)c * 8, N.w_dtype, wv);
          rownorm_emit(N, o * A.inner + (int64_t)c * 8, v, wv, s, decltype(odt)::value);
        }
      }
    };
    switch (N.out_dtype) {
      case DT_F32: emit_all(std::integral_constant<int, DT_F32>{}); break;
      case DT_BF16: emit_all(std::integral_constant<int, DT_BF16>{}); break;
      case DT_F16: emit_all(std::integral_constant<int, DT_F16>{}); break;
      case DT_F8E4M3FN: emit_all(std::integral_constant<int, DT_F8E4M3FN>{}); break;
      default: emit_all(std::integral_constant<int, DT_F8E5M2>{}); break;
    }
  }
}

// RMSNorm of many bf16 rows (bf16 weights, or none: W) of at most 64·8·NCW elements, a wavefront per row like
// rownorm_wave_kernel, for grids that give each wavefront several rows: its lanes' weight chunks are loaded once and
// kept in registers (raw words; no LDS staging and no barrier), and a wavefront moves on to its next row without
// waiting for the others. The square of a bf16 value is exact in f32, so Σx² folds with FMAs (one rounding each, the
// same as the separate multiply and add) in the same order, and the output bits equal rownorm_wave_kernel's. The
// output type is chosen once, outside the row loop.
template <int NCW, bool W, int ODT>
__device__ __forceinline__ void rownorm_rows(const RowArgs& A) {
#pragma clang fp contract(off)
  const RowNormArgs& N = A.norm;
  const int lane = threadIdx.x & 63;
  const int64_t chunks = A.inner / 8;
  const int64_t stride = (int64_t)gridDim.x * (VNT / 64);
  int64_t o = (int64_t)blockIdx.x * (VNT / 64) + (threadIdx.x >> 6);
  if (o >= A.rows) return;
  uint32_t x[NCW][4], w[W ? NCW : 1][4];  // raw bf16 inputs and weights
  auto fetch = [&](int64_t r) __attribute__((always_inline)) {
    const char* xrow = (const char*)N.x + r * A.inner * 2;
#pragma unroll
    for (int q = 0; q < NCW; ++q) {
      const int c = lane + 64 * q;
      if (c < chunks) {
        const u32x4v a = *(const u32x4v*)(xrow + (int64_t)c * 16);
        x[q][0] = a.x, x[q][1] = a.y, x[q][2] = a.z, x[q][3] = a.w;
      }
    }
  };
  fetch(o);
  if constexpr (W) {
#pragma unroll
    for (int q = 0; q < NCW; ++q) {
      const int c = lane + 64 * q;
      if (c < chunks) {
        const u32x4v a = *(const u32x4v*)((const char*)N.w + (int64_t)c * 16);
        w[q][0] = a.x, w[q][1] = a.y, w[q][2] = a.z, w[q][3] = a.w;
      }
    }
  }
  // f8E4M3FN output: whether every weight is finite (bf16 exponent field not all ones), once per wavefront
  bool w_finite = true;
  if constexpr (W && ODT == DT_F8E4M3FN) {
    bool ok = true;
#pragma unroll
    for (int q = 0; q < NCW; ++q)
      if (lane + 64 * q < chunks)
#pragma unroll
        for (int h = 0; h < 4; ++h)
          ok = ok && (w[q][h] & 0x7f80u) != 0x7f80u && (w[q][h] & 0x7f800000u) != 0x7f800000u;
    w_finite = __all(ok);
  }
  for (;;) {
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < NCW; ++q)
      if (lane + 64 * q < chunks) {
        float v[8];
        decode8_f32(DT_BF16, x[q], v);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(v[e], v[e], acc);
      }
    for (int off = 32; off > 0; off >>= 1) acc = acc + __shfl_xor(acc, off, 64);
    acc = __shfl(acc, 0, 64);
    const float sc = rownorm_scale(A, acc);
    auto emit_row = [&](auto nan_free) __attribute__((always_inline)) {
#pragma unroll
      for (int q = 0; q < NCW; ++q) {
        const int c = lane + 64 * q;
        if (c < chunks) {
          // decoded here from raw words the compiler cannot see through, rather than kept decoded from the Σx²
          // pass (x) or from before the row loop (w): that would hold 16·NCW more registers per lane
          uint32_t xw[4] = {x[q][0], x[q][1], x[q][2], x[q][3]};
          __asm__ __volatile__("" : "+v"(xw[0]), "+v"(xw[1]), "+v"(xw[2]), "+v"(xw[3]));
          float v[8], wv[8];
          decode8_f32(DT_BF16, xw, v);
          if constexpr (W) {
            uint32_t ww[4] = {w[q][0], w[q][1], w[q][2], w[q][3]};
            __asm__ __volatile__("" : "+v"(ww[0]), "+v"(ww[1]), "+v"(ww[2]), "+v"(ww[3]));
            decode8_f32(DT_BF16, ww, wv);
          }
          rownorm_emit<decltype(nan_free)::value>(N, o * A.inner + (int64_t)c * 8, v, wv, sc, ODT);
        }
      }
    };
    // No y = round(x·s·w) is a NaN when Σx² and s are finite (so is every x, and |x·s| ≤ √Σx²·s), √Σx²·s stays
    // far below the f32 overflow threshold (x·s finite) and every weight is finite: (x·s)·w is then finite or
    // infinite, and so is its rounding. Such rows skip the NaN sign repair of the f8E4M3FN conversion.
    if (ODT == DT_F8E4M3FN && w_finite && __builtin_isfinite(acc) && __builtin_isfinite(sc) &&
        sqrtf(acc) * sc < 1e37f)
      emit_row(std::true_type{});
    else
      emit_row(std::false_type{});
    o += stride;
    if (o >= A.rows) break;
    fetch(o);
  }
}

template <int NCW, bool W>
__global__ void __launch_bounds__(VNT) rownorm_rows_kernel(const RowArgs A) {
  switch (A.norm.out_dtype) {
    case DT_F32: return rownorm_rows<NCW, W, DT_F32>(A);
    case DT_BF16: return rownorm_rows<NCW, W, DT_BF16>(A);
    case DT_F16: return rownorm_rows<NCW, W, DT_F16>(A);
    case DT_F8E4M3FN: return rownorm_rows<NCW, W, DT_F8E4M3FN>(A);
    default: return rownorm_rows<NCW, W, DT_F8E5M2>(A);
  }
}

// One workgroup per row (rows too long for a wavefront, or too few rows to fill the chip that way). A thread owns
// chunks t, t + 256, ... of 8 elements; with NC > 0 (rows of at most NC·2048 elements) it loads them — and the
// matching weight chunks — once, up front, and keeps them in registers; NC = 0 reads the row again (from L2) for the
// scaling pass. Σx² is folded per thread in element order, then across lanes and wavefronts (through LDS) in the
// order of the interpreted row kernel for such rows.
template <int NC>
__global__ void __launch_bounds__(VNT) rownorm_block_kernel(const RowArgs A) {
#pragma clang fp contract(off)
  __shared__ float part[VNT / 64];
  const RowNormArgs& N = A.norm;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t chunks = A.inner / 8;
  constexpr int NQ = NC > 0 ? NC : 1;
  for (int64_t o = blockIdx.x; o < A.rows; o += gridDim.x) {
    const int64_t base = o * A.inner;
    float acc = 0.0f;
    float xs[NQ][8], ws[NQ][8];
    if constexpr (NC > 0) {
#pragma unroll
      for (int q = 0; q < NC; ++q) {
        const int64_t c = threadIdx.x + (int64_t)q * VNT;
        if (c < chunks) {
          load8_f32(N.x, base + c * 8, N.x_dtype, xs[q]);
          if (N.w) load8_f32(N.w, c * 8, N.w_dtype, ws[q]);
        }
      }
#pragma unroll
      for (int q = 0; q < NC; ++q)
        if (threadIdx.x + (int64_t)q * VNT < chunks) {
#pragma unroll
          for (int e = 0; e < 8; ++e) acc = acc + xs[q][e] * xs[q][e];
        }
    } else {
      for (int64_t c = threadIdx.x; c < chunks; c += VNT) {
        float v[8];
        load8_f32(N.x, base + c * 8, N.x_dtype, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = acc + v[e] * v[e];
      }
    }
    for (int off = 32; off > 0; off >>= 1) acc = acc + __shfl_xor(acc, off, 64);
    acc = __shfl(acc, 0, 64);
    if (lane == 0) part[wave] = acc;
    __syncthreads();
    acc = part[0];
    for (int w = 1; w < VNT / 64; ++w) acc = acc + part[w];
    __syncthreads();
    const float s = rownorm_scale(A, acc);
    if constexpr (NC > 0) {
#pragma unroll
      for (int q = 0; q < NC; ++q) {
        const int64_t c = threadIdx.x + (int64_t)q * VNT;
        if (c < chunks) rownorm_emit(N, base + c * 8, xs[q], ws[q], s, N.out_dtype);
      }
    } else {
      for (int64_t c = threadIdx.x; c < chunks; c += VNT) {
        float v[8], wv[8];
        load8_f32(N.x, base + c * 8, N.x_dtype, v);
        if (N.w) load8_f32(N.w, c * 8, N.w_dtype, wv);
        rownorm_emit(N, base + c * 8, v, wv, s, N.out_dtype);
      }
    }
  }
}

// Whether a [rows, inner] row step gives each row one wavefront (else one workgroup), in the interpreted row kernel
// and in the RMSNorm kernels alike, so both fold a row's sums in the same order: short rows always; rows of up to
// ROW_WAVE_CHUNKS 8-element vectors when there are enough of them to keep every compute unit's waves busy (with few
// rows, splitting each row over a workgroup's four waves finishes sooner).
constexpr int64_t ROW_WAVE_CHUNKS = 64 * 16;
constexpr int64_t ROW_WAVE_MIN_ROWS = 2048;
static bool row_per_wave(int64_t rows, int64_t inner) {
  return inner / VEC < VNT || (inner / VEC <= ROW_WAVE_CHUNKS && rows >= ROW_WAVE_MIN_ROWS);
}

// Workgroups of rownorm_rows_kernel<NCW, W> one compute unit holds at once (asked of the runtime once per
// instantiation; gfx950 only, so one answer serves every device).
template <int NCW, bool W>
static int rownorm_rows_per_cu() {
  static const int n = [] {
    int v = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, rownorm_rows_kernel<NCW, W>, VNT, 0) != hipSuccess || v < 1)
      v = 1;
    return v;
  }();
  return n;
}

static bool rownorm_launchable(const RowArgs& a) {
  const RowNormArgs& n = a.norm;
  auto float_ok = [](int dt) { return dt == DT_F32 || dt == DT_BF16 || dt == DT_F16; };
  auto aligned = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  return a.inner % 8 == 0 && float_ok(n.x_dtype) && (!n.w || float_ok(n.w_dtype)) && aligned(n.x) &&
         (!n.w || aligned(n.w)) && ((uintptr_t)n.out % (uintptr_t)(8 * elem_size(n.out_dtype))) == 0 &&
         (n.out_dtype == DT_F32 || n.out_dtype == DT_BF16 || n.out_dtype == DT_F16 || n.out_dtype == DT_F8E4M3FN ||
          n.out_dtype == DT_F8E5M2);
}

template <int G, int V>
static void launch_row_g(const RowArgs& a, hipStream_t stream, hipEvent_t done) {
  constexpr int RB = VNT / G;
  int64_t blocks = (a.rows + RB - 1) / RB;
  if (blocks > 256 * 16) blocks = 256 * 16;
  dim3 grid((unsigned)blocks), block(VNT);
  if (a.prog.needs_coords) launch_k(done, row_kernel<G, V, true>, grid, block, 0, stream, a);
  else launch_k(done, row_kernel<G, V, false>, grid, block, 0, stream, a);
}

void launch_row(const RowArgs& a, hipStream_t stream, hipEvent_t done) {
  if (a.rows == 0 || a.inner == 0) return record_done(done, stream);
  if (a.n_red < 1 || a.n_red > ROW_MAX_RED || a.prog.rank < 1 || a.prog.shape[a.prog.rank - 1] != a.inner ||
      a.rows * a.inner != a.prog.total)
    fail(PJRT_Error_Code_INTERNAL, "row-fused step: arguments do not describe a [rows, inner] space");
  for (int k = 0; k <= a.n_red; ++k)
    if (a.phase_end[k] < (k ? a.phase_end[k - 1] : 0) || a.phase_end[k] > a.prog.n_instr)
      fail(PJRT_Error_Code_INTERNAL, "row-fused step: phase bounds outside the program");
  if (a.fast == ROW_FAST_NORM && rownorm_launchable(a)) {
    const int64_t chunks = a.inner / 8;
    const dim3 block(VNT);
    const int ncw = (int)((chunks + 63) / 64);
    if (row_per_wave(a.rows, a.inner) && a.norm.x_dtype == DT_BF16 && (!a.norm.w || a.norm.w_dtype == DT_BF16) &&
        ncw <= 8) {
      // a wavefront per row, the weights in registers; as many workgroups as the compute units hold at once (each
      // wavefront then takes every stride-th row), or fewer when there are fewer rows
      auto go = [&](auto ncw_c, auto w_c) {
        constexpr int K = decltype(ncw_c)::value;
        constexpr bool W = decltype(w_c)::value;
        const int64_t per_cu = rownorm_rows_per_cu<K, W>();
        int64_t blocks = (a.rows + 3) / 4;
        if (blocks > 256 * per_cu) blocks = 256 * per_cu;
        launch_k(done, rownorm_rows_kernel<K, W>, dim3((unsigned)blocks), block, 0, stream, a);
      };
      auto go_w = [&](auto ncw_c) {
        if (a.norm.w) go(ncw_c, std::true_type{});
        else go(ncw_c, std::false_type{});
      };
      if (ncw <= 1) go_w(std::integral_constant<int, 1>{});
      else if (ncw <= 2) go_w(std::integral_constant<int, 2>{});
      else if (ncw <= 4) go_w(std::integral_constant<int, 4>{});
      else go_w(std::integral_constant<int, 8>{});
    } else if (row_per_wave(a.rows, a.inner)) {
      // a wavefront per row, four rows per workgroup, the weight row in dynamic LDS
      int64_t blocks = (a.rows + 3) / 4;
      if (blocks > 256 * 64) blocks = 256 * 64;
      const dim3 grid((unsigned)blocks);
      const uint32_t lds = a.norm.w ? (uint32_t)(a.inner * (a.norm.w_dtype == DT_F32 ? 4 : 2)) : 0u;
      auto go = [&](auto kernel) { launch_k(done, kernel, grid, block, lds, stream, a); };
      if (a.norm.x_dtype == DT_F32) {
        if (ncw <= 1) go(rownorm_wave_kernel<1, 4>);
        else if (ncw <= 2) go(rownorm_wave_kernel<2, 4>);
        else if (ncw <= 4) go(rownorm_wave_kernel<4, 4>);
        else if (ncw <= 8) go(rownorm_wave_kernel<8, 4>);
        else go(rownorm_wave_kernel<16, 4>);
      } else {
        if (ncw <= 1) go(rownorm_wave_kernel<1, 2>);
        else if (ncw <= 2) go(rownorm_wave_kernel<2, 2>);
        else if (ncw <= 4) go(rownorm_wave_kernel<4, 2>);
        else if (ncw <= 8) go(rownorm_wave_kernel<8, 2>);
        else go(rownorm_wave_kernel<16, 2>);
      }
    } else {
      const dim3 grid((unsigned)(a.rows < 256 * 16 ? a.rows : 256 * 16));
      const int64_t per_thread = (chunks + VNT - 1) / VNT;
      if (per_thread <= 1) launch_k(done, rownorm_block_kernel<1>, grid, block, 0, stream, a);
      else if (per_thread <= 2) launch_k(done, rownorm_block_kernel<2>, grid, block, 0, stream, a);
      else if (per_thread <= 4) launch_k(done, rownorm_block_kernel<4>, grid, block, 0, stream, a);
      else launch_k(done, rownorm_block_kernel<0>, grid, block, 0, stream, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) fail(PJRT_Error_Code_INTERNAL, std::string("row-norm launch failed: ") + hipGetErrorString(e));
    return;
  }
  RowArgs v = a;
  if (prepare_vec(v.prog, true)) {
    if (row_per_wave(a.rows, a.inner)) launch_row_g<64, VEC>(v, stream, done);
    else launch_row_g<VNT, VEC>(v, stream, done);
  } else {
    if (a.inner >= 4 * VNT) launch_row_g<VNT, 1>(a, stream, done);
    else launch_row_g<64, 1>(a, stream, done);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail(PJRT_Error_Code_INTERNAL, std::string("row-fused launch failed: ") + hipGetErrorString(e));
}

}  // namespace ryft
