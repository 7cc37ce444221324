// GEMM dispatch for gfx950: picks an MFMA instantiation (gemm_mfma.h, one translation unit per operand type) when
// the operand types, layouts, alignments, epilogue and output types fit one, and otherwise runs the generic path —
// a 64×64 LDS-tiled FMA kernel that reads any element type through any strides (bounds-checked), used for shapes
// and type mixes the MFMA instantiations do not cover.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>
#include <type_traits>

#include "../common.h"
#include "gemm_epilogue.h"
#include "gemm_mfma.h"
#include "kernels.h"
#include "launch.h"

namespace ryft {

typedef __bf16 bf16x8_t __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef _Float16 f16x8_t __attribute__((__vector_size__(8 * sizeof(_Float16))));
typedef float f32x16_t __attribute__((__vector_size__(16 * sizeof(float))));
typedef int i32x16_t __attribute__((__vector_size__(16 * sizeof(int))));
typedef int i32x4_t __attribute__((__vector_size__(4 * sizeof(int))));
typedef int i32x8_t __attribute__((__vector_size__(8 * sizeof(int))));

// ------------------------------------------------------------------------------------------------ generic GEMM
template <bool INT_ACC, bool DUAL>
__global__ void __launch_bounds__(256) gemm_generic_kernel(const GemmArgs G) {
  __shared__ uint32_t As[16][65];
  __shared__ uint32_t Bs[16][65];
  __shared__ uint32_t B2s[DUAL ? 16 : 1][65];
  const int b = blockIdx.z;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  float acc[4][4] = {}, acc2[4][4] = {};
  int32_t iacc[4][4] = {};
  const bool a_float = dt_is_float(G.A.dtype), b_float = dt_is_float(G.B.dtype);
  for (int k0 = 0; k0 < G.K; k0 += 16) {
    for (int i = threadIdx.x; i < 64 * 16; i += 256) {
      int r = i >> 4, kk = i & 15, k = k0 + kk;
      uint32_t va = 0, vb = 0, vb2 = 0;
      if (m0 + r < G.M && k < G.K) {
        va = load_bits(G.A.ptr, (int64_t)b * G.A.sb + (int64_t)(m0 + r) * G.A.sr + (int64_t)k * G.A.sk, G.A.dtype);
        if (!INT_ACC && !a_float) va = __float_as_uint((float)(int32_t)va);
      }
      if (n0 + r < G.N && k < G.K) {
        vb = load_bits(G.B.ptr, (int64_t)b * G.B.sb + (int64_t)(n0 + r) * G.B.sr + (int64_t)k * G.B.sk, G.B.dtype);
        if (!INT_ACC && !b_float) vb = __float_as_uint((float)(int32_t)vb);
        if (DUAL) {
          vb2 = load_bits(G.B2.ptr, (int64_t)b * G.B2.sb + (int64_t)(n0 + r) * G.B2.sr + (int64_t)k * G.B2.sk, G.B2.dtype);
          if (!dt_is_float(G.B2.dtype)) vb2 = __float_as_uint((float)(int32_t)vb2);
        }
      }
      As[kk][r] = va;
      Bs[kk][r] = vb;
      if (DUAL) B2s[kk][r] = vb2;
    }
    __syncthreads();
#pragma unroll 4
    for (int kk = 0; kk < 16; ++kk) {
      uint32_t a[4], bb[4], b2[4];
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
      for (int j = 0; j < 4; ++j) bb[j] = Bs[kk][tx * 4 + j];
      if (DUAL)
        for (int j = 0; j < 4; ++j) b2[j] = B2s[kk][tx * 4 + j];
      for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 4; ++j) {
          if (INT_ACC) {
            iacc[i][j] += (int32_t)a[i] * (int32_t)bb[j];
          } else {
            acc[i][j] = fmaf(__uint_as_float(a[i]), __uint_as_float(bb[j]), acc[i][j]);
            if (DUAL) acc2[i][j] = fmaf(__uint_as_float(a[i]), __uint_as_float(b2[j]), acc2[i][j]);
          }
        }
    }
    __syncthreads();
  }
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 4; ++j) {
      int m = m0 + ty * 4 + i, n = n0 + tx * 4 + j;
      if (m < G.M && n < G.N) gemm_epilogue<INT_ACC>(G, b, m, n, acc[i][j], iacc[i][j], acc2[i][j]);
    }
}

// ------------------------------------------------------------------------------------------------ dispatch
// ------------------------------------------------------------------------------------------------ split-K
// Sums the K ranges' partial accumulators in range order and applies the epilogue (splitk_epilogue_oct, shared with
// the in-kernel finish of the MFMA kernels, so the two give the same bits). Each thread owns 8 consecutive elements
// of the result (N is a multiple of 16 on every split-K plan): S (the number of ranges, a template argument so that
// every range's two 16-byte loads are in flight together) × 2 loads per accumulator set, then one vector store per
// output.
template <bool INT, bool DUAL, int S>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const GemmArgs G) {
  const int64_t octs = (int64_t)G.batch * G.M * G.N / 8;
  const int64_t slice = (int64_t)G.batch * G.M * G.N;  // elements of one accumulator set
  constexpr int NB = DUAL ? 2 : 1;
  auto add = [](uint32_t a, uint32_t x) {
    return INT ? (uint32_t)((int32_t)a + (int32_t)x) : __float_as_uint(__uint_as_float(a) + __uint_as_float(x));
  };
  for (int64_t oc = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; oc < octs; oc += (int64_t)gridDim.x * blockDim.x) {
    const int64_t e0 = oc * 8;
    const int n = (int)(e0 % G.N);
    const int64_t bm = e0 / G.N;
    const int m = (int)(bm % G.M), b = (int)(bm / G.M);
    u32x4 w[S][NB][2];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int k = 0; k < NB; ++k) {
        const u32x4* p = (const u32x4*)((const uint32_t*)G.ws + ((int64_t)s * NB + k) * slice + e0);
        w[s][k][0] = p[0];
        w[s][k][1] = p[1];
      }
    uint32_t v[8], v2[8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      v[4 * h] = w[0][0][h].x, v[4 * h + 1] = w[0][0][h].y, v[4 * h + 2] = w[0][0][h].z, v[4 * h + 3] = w[0][0][h].w;
      if constexpr (DUAL)
        v2[4 * h] = w[0][1][h].x, v2[4 * h + 1] = w[0][1][h].y, v2[4 * h + 2] = w[0][1][h].z,
        v2[4 * h + 3] = w[0][1][h].w;
    }
#pragma unroll
    for (int s = 1; s < S; ++s)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        v[4 * h] = add(v[4 * h], w[s][0][h].x), v[4 * h + 1] = add(v[4 * h + 1], w[s][0][h].y);
        v[4 * h + 2] = add(v[4 * h + 2], w[s][0][h].z), v[4 * h + 3] = add(v[4 * h + 3], w[s][0][h].w);
        if constexpr (DUAL) {
          v2[4 * h] = add(v2[4 * h], w[s][1][h].x), v2[4 * h + 1] = add(v2[4 * h + 1], w[s][1][h].y);
          v2[4 * h + 2] = add(v2[4 * h + 2], w[s][1][h].z), v2[4 * h + 3] = add(v2[4 * h + 3], w[s][1][h].w);
        }
      }
    splitk_epilogue_oct<INT, DUAL>(G, e0, b, m, n, v, v2);
  }
}

template <bool INT, bool DUAL>
static void launch_splitk_reduce(const GemmArgs& g, hipStream_t stream, hipEvent_t done) {
  const int64_t octs = (int64_t)g.batch * g.M * g.N / 8;
  const dim3 grid((unsigned)std::min<int64_t>((octs + 255) / 256, 256 * 16)), block(256);
  switch (g.splits) {
    case 2: return launch_k(done, splitk_reduce_kernel<INT, DUAL, 2>, grid, block, 0, stream, g);
    case 4: return launch_k(done, splitk_reduce_kernel<INT, DUAL, 4>, grid, block, 0, stream, g);
    case 8: return launch_k(done, splitk_reduce_kernel<INT, DUAL, 8>, grid, block, 0, stream, g);
    case 16: return launch_k(done, splitk_reduce_kernel<INT, DUAL, 16>, grid, block, 0, stream, g);
    default: fail(PJRT_Error_Code_INTERNAL, "split-K over " + std::to_string(g.splits) + " ranges");
  }
}

static int mma_kind(const GemmArgs& g) {
  if (g.dual && g.B2.dtype != g.B.dtype) return -1;
  // bf16 × f8E4M3FN (weight-only quantisation): f8 widens exactly to bf16, so the bf16 MFMA computes the same dot
  if (g.A.dtype == DT_BF16 && g.B.dtype == DT_F8E4M3FN) return g.acc_is_int ? -1 : MMA_BF16_F8;
  if (g.A.dtype != g.B.dtype) return -1;
  switch (g.A.dtype) {
    case DT_BF16: return g.acc_is_int ? -1 : MMA_BF16;
    case DT_F16: return g.acc_is_int ? -1 : MMA_F16;
    case DT_S8: return g.acc_is_int ? MMA_I8 : -1;
    case DT_F8E4M3FN: return g.acc_is_int ? -1 : MMA_FP8;
    case DT_F32: return g.acc_is_int ? -1 : MMA_F32;
    default: return -1;
  }
}

// Operands (bit 0: A, 1: B, 2: B2) whose layout the MFMA kernels cannot read: neither K-contiguous nor contiguous
// along their free dimension in 16-byte vectors (`kbytes`-byte pieces along k for a K-contiguous f8 B widened to
// bf16), misaligned, or with rows too far apart for the 32-bit buffer offsets of a tile.
static unsigned layout_gaps(const GemmArgs& g, int kind, int* ar, int* br) {
  const int es = kind == MMA_BF16 || kind == MMA_F16 || kind == MMA_BF16_F8 ? 2 : (kind == MMA_F32 ? 4 : 1);
  const int bes = kind == MMA_BF16_F8 ? 1 : es;  // B's element size in HBM
  auto layout = [&](const GemmOperand& o, int oes, int kbytes, int* r) -> bool {
    const int ve = 16 / oes, vk = kbytes / oes;
    if (((uintptr_t)o.ptr & 15) != 0) return false;
    // tiles (≤ 256 rows / k-rows) are read through 32-bit buffer offsets from the tile origin
    if ((o.sr > o.sk ? o.sr : o.sk) * (int64_t)oes * 256 >= ((int64_t)1 << 31)) return false;
    if (o.sk == 1 && (o.sr % vk) == 0 && (o.sb % vk) == 0) { *r = 0; return true; }
    if (o.sr == 1 && (o.sk % ve) == 0 && (o.sb % ve) == 0) { *r = 1; return true; }
    return false;
  };
  const int bkb = kind == MMA_BF16_F8 ? 8 : 16;
  unsigned gaps = 0;
  int br2 = -1;
  if (!layout(g.A, es, 16, ar)) gaps |= 1;
  if (!layout(g.B, bes, bkb, br)) gaps |= 2;
  if (g.dual && (!layout(g.B2, bes, bkb, &br2) || (!(gaps & 2) && br2 != *br))) gaps |= 4;
  return gaps;
}

// Returns true and fills `c` when an MFMA instantiation covers these arguments.
static bool pick_mfma(const GemmArgs& g, Choice* c) {
  // MFMA epilogues implement store / scale / SwiGLU; generic programs run on the generic kernel
  if (g.epilogue == EPI_PROGRAM || (g.dual && g.epilogue != EPI_SWIGLU)) return false;
  int kind = mma_kind(g);
  if (kind < 0) return false;
  // output types the MFMA epilogue writes (outputs are whole device allocations, so 16-byte aligned)
  const bool int_acc = kind == MMA_I8;
  if (!mfma_out_supported(g.out_dtype[0], int_acc, g.epilogue, false)) return false;
  if (g.epilogue == EPI_SCALE && g.raw_out && !mfma_out_supported(g.out_dtype[1], int_acc, g.epilogue, true))
    return false;
  if (g.epilogue != EPI_STORE && !mfma_mid_round_supported(g.mid_round, g.raw_out != 0)) return false;
  if (g.epilogue == EPI_STORE && g.mid_round) return false;
  const int es = kind == MMA_BF16 || kind == MMA_F16 || kind == MMA_BF16_F8 ? 2 : (kind == MMA_F32 ? 4 : 1);
  const int bes = kind == MMA_BF16_F8 ? 1 : es;  // B's element size in HBM
  int ar = 0, br = 0;
  if (layout_gaps(g, kind, &ar, &br)) return false;
  bool ok = false;
  switch (kind) {
    case MMA_BF16: ok = pick_bf16(g, ar, br, c); break;
    case MMA_F16: ok = pick_f16(g, ar, br, c); break;
    case MMA_I8: ok = pick_i8(g, ar, br, c); break;
    case MMA_FP8: ok = pick_fp8(g, ar, br, c); break;
    case MMA_F32: ok = pick_f32(g, ar, br, c); break;
    case MMA_BF16_F8: ok = pick_bf16f8(g, ar, br, c); break;
  }
  if (ok && c->edge) {
    // the edge kernels zero k positions past K a load at a time: K must end on a load boundary of each
    // K-contiguous operand (16-byte vectors; 8-byte pieces for a widened f8 B)
    int kgran = 1;
    if (ar == 0) kgran = 16 / es;
    if (br == 0) kgran = std::max(kgran, kind == MMA_BF16_F8 ? 8 : 16 / bes);
    if (g.K % kgran) ok = false;
  }
  return ok;
}

int gemm_mfma_layout_gaps(const GemmArgs& a) {
  GemmArgs g = a;
  g.splits = 1;
  if (g.epilogue == EPI_PROGRAM) g.epilogue = EPI_STORE;
  const int kind = mma_kind(g);
  if (kind < 0 || (g.dual && g.epilogue != EPI_SWIGLU)) return -1;
  int ar = 0, br = 0;
  unsigned gaps = layout_gaps(g, kind, &ar, &br);
  // K-contiguous operands of the edge kernels are read a vector (8-byte piece for a widened f8 B) at a time up to K
  const int es = kind == MMA_BF16 || kind == MMA_F16 || kind == MMA_BF16_F8 ? 2 : (kind == MMA_F32 ? 4 : 1);
  const int bes = kind == MMA_BF16_F8 ? 1 : es;
  if (!(gaps & 1) && ar == 0 && g.K % (16 / es)) gaps |= 1;
  if (!(gaps & 2) && br == 0 && g.K % (kind == MMA_BF16_F8 ? 8 : 16 / bes)) gaps |= g.dual ? 6 : 2;
  if (gaps) return (int)gaps;
  Choice c;
  return pick_mfma(g, &c) ? 0 : -1;
}

const char* gemm_kernel_name(const GemmArgs& a) {
  Choice c;
  if (pick_mfma(a, &c)) return c.name;
  return "gemm_generic";
}

int gemm_plan_splits(const GemmArgs& a) {
  GemmArgs g = a;
  g.splits = 1;
  Choice c;
  if (!pick_mfma(g, &c)) return 1;
  const int64_t tiles = (int64_t)((g.M + c.bm - 1) / c.bm) * ((g.N + c.bn - 1) / c.bn) * g.batch;
  const bool f32 = g.A.dtype == DT_F32;
  // the 64-row tile (chosen when 128×128 tiles would not cover the chip) reads twice the operand bytes per FLOP of a
  // 128×128 tile, from L2 as well as LDS: splitting K over 128×128 tiles beats it
  const bool small_tile = !f32 && c.bm < 128;
  if (tiles >= 192 && !small_tile) return 1;  // the chip (256 CUs) is already covered well enough
  if (g.dual) return 1;
  // the split tile: the one the picker runs over each K range (probed with two ranges); at least 4 k-tiles per range
  GemmArgs probe = g;
  probe.splits = 2;
  Choice sc;
  if (!pick_mfma(probe, &sc)) return 1;
  const int64_t tiles_s = (int64_t)(g.M / sc.bm) * (g.N / sc.bn) * g.batch;
  int best = 1;
  for (int s = 2; s <= 16; s *= 2) {
    if (tiles_s * s > 256 || g.K % (sc.bk * s) || g.K / (sc.bk * s) < 4) break;
    best = s;
  }
  if (best < 2 || (!small_tile && tiles_s * best <= tiles)) return 1;
  g.splits = best;
  return pick_mfma(g, &c) ? best : 1;
}

void launch_gemm(const GemmArgs& g, hipStream_t stream, hipEvent_t done) {
  if (g.M == 0 || g.N == 0 || g.batch == 0) return record_done(done, stream);
  Choice c;
  hipError_t e;
  if (g.K > 0 && pick_mfma(g, &c)) {
    // shape invariants the MFMA kernels rely on (checked again here, right before the launch)
    if (!c.edge && (g.M % c.bm || g.N % c.bn)) fail(PJRT_Error_Code_INTERNAL, "gemm tile mismatch");
    if (c.lds > 65536) {
      e = hipFuncSetAttribute(c.fn, hipFuncAttributeMaxDynamicSharedMemorySize, c.lds);
      if (e != hipSuccess) fail(PJRT_Error_Code_INTERNAL, std::string("LDS attribute failed: ") + hipGetErrorString(e));
    }
    const int splits = g.splits > 1 ? g.splits : 1;
    if (splits > 1 && (!g.ws || g.K % (splits * 16) || g.N % 16 || c.edge))
      fail(PJRT_Error_Code_INTERNAL, "split-K without a workspace, on partial tiles or with N not a multiple of 16");
    if (splits > 1 && g.tile_counters && (g.dual || (splits & (splits - 1)) || splits > 16))
      fail(PJRT_Error_Code_INTERNAL, "in-kernel split-K finish for a dual GEMM or " + std::to_string(splits) + " ranges");
    int64_t blocks = (int64_t)((g.M + c.bm - 1) / c.bm) * ((g.N + c.bn - 1) / c.bn) * g.batch * splits;
    if (blocks > INT32_MAX) fail(PJRT_Error_Code_UNIMPLEMENTED, "too many GEMM tiles");
    void* args[] = {(void*)&g};
    // split-K finished by a reduction launch: that launch carries the completion event
    const bool reduce = splits > 1 && !g.tile_counters;
    hipEvent_t main_done = reduce ? nullptr : done;
    hipEvent_t start = take_start();
    e = main_done || start ? hipExtLaunchKernel(c.fn, dim3((unsigned)blocks), dim3(c.threads), args, (size_t)c.lds,
                                                stream, start, main_done, 0)
                           : hipLaunchKernel(c.fn, dim3((unsigned)blocks), dim3(c.threads), args, (size_t)c.lds, stream);
    if (e == hipSuccess && reduce) {
      if (g.acc_is_int) launch_splitk_reduce<true, false>(g, stream, done);
      else if (g.dual) launch_splitk_reduce<false, true>(g, stream, done);
      else launch_splitk_reduce<false, false>(g, stream, done);
      e = hipGetLastError();
    }
  } else {
    dim3 grid((g.N + 63) / 64, (g.M + 63) / 64, g.batch), block(256);
    if (g.batch > 65535) fail(PJRT_Error_Code_UNIMPLEMENTED, "batch too large for the generic GEMM");
    if (g.acc_is_int) {
      if (g.dual) fail(PJRT_Error_Code_UNIMPLEMENTED, "integer dual GEMM");
      launch_k(done, gemm_generic_kernel<true, false>, grid, block, 0, stream, g);
    } else if (g.dual) {
      launch_k(done, gemm_generic_kernel<false, true>, grid, block, 0, stream, g);
    } else {
      launch_k(done, gemm_generic_kernel<false, false>, grid, block, 0, stream, g);
    }
    e = hipGetLastError();
  }
  if (e != hipSuccess) fail(PJRT_Error_Code_INTERNAL, std::string("gemm launch failed: ") + hipGetErrorString(e));
}

}  // namespace ryft
