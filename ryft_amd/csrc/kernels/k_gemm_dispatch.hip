// GEMM dispatch for gfx950: picks an MFMA instantiation (gemm_mfma.h, one translation unit per operand type) when
// the operand types, layouts, alignments, epilogue and output types fit one, and otherwise runs the generic path —
// a 64×64 LDS-tiled FMA kernel that reads any element type through any strides (bounds-checked), used for shapes
// and type mixes the MFMA instantiations do not cover.
#include <hip/hip_runtime.h>

#include <string>
#include <type_traits>

#include "../common.h"
#include "gemm_epilogue.h"
#include "gemm_mfma.h"
#include "kernels.h"

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
static int mma_kind(const GemmArgs& g) {
  auto t = [](int d) { return d; };
  if (g.dual && g.B2.dtype != g.B.dtype) return -1;
  if (t(g.A.dtype) != t(g.B.dtype)) return -1;
  switch (g.A.dtype) {
    case DT_BF16: return g.acc_is_int ? -1 : MMA_BF16;
    case DT_F16: return g.acc_is_int ? -1 : MMA_F16;
    case DT_S8: return g.acc_is_int ? MMA_I8 : -1;
    case DT_F8E4M3FN: return g.acc_is_int ? -1 : MMA_FP8;
    case DT_F32: return g.acc_is_int ? -1 : MMA_F32;
    default: return -1;
  }
}

// Returns true and fills `c` when an MFMA instantiation covers these arguments.
static bool pick_mfma(const GemmArgs& g, Choice* c) {
  // MFMA epilogues implement store / scale / SwiGLU; generic programs run on the generic kernel
  if (g.epilogue == EPI_PROGRAM || (g.dual && g.epilogue != EPI_SWIGLU)) return false;
  if (g.N % 16) return false;  // 16-element row segments in the epilogue
  int kind = mma_kind(g);
  if (kind < 0) return false;
  // output types the MFMA epilogue writes (outputs are whole device allocations, so 16-byte aligned)
  const bool int_acc = kind == MMA_I8;
  if (!mfma_out_supported(g.out_dtype[0], int_acc, g.epilogue, false)) return false;
  if (g.epilogue == EPI_SCALE && g.raw_out && !mfma_out_supported(g.out_dtype[1], int_acc, g.epilogue, true))
    return false;
  if (g.epilogue != EPI_STORE && !mfma_mid_round_supported(g.mid_round, g.raw_out != 0)) return false;
  if (g.epilogue == EPI_STORE && g.mid_round) return false;
  const int es = kind == MMA_BF16 || kind == MMA_F16 ? 2 : (kind == MMA_F32 ? 4 : 1);
  const int ve = 16 / es;
  // operand layouts: K-contiguous (sk == 1) or row-contiguous (sr == 1)
  auto layout = [&](const GemmOperand& o, int rows, int* r) -> bool {
    if (((uintptr_t)o.ptr & 15) != 0) return false;
    // tiles (≤ 256 rows / k-rows) are read through 32-bit buffer offsets from the tile origin
    if ((o.sr > o.sk ? o.sr : o.sk) * (int64_t)es * 256 >= ((int64_t)1 << 31)) return false;
    if (o.sk == 1 && (o.sr % ve) == 0 && (o.sb % ve) == 0) { *r = 0; return true; }
    if (o.sr == 1 && (o.sk % ve) == 0 && (o.sb % ve) == 0) { *r = 1; return true; }
    (void)rows;
    return false;
  };
  int ar, br, br2 = -1;
  if (!layout(g.A, g.M, &ar) || !layout(g.B, g.N, &br)) return false;
  if (g.dual && (!layout(g.B2, g.N, &br2) || br2 != br)) return false;
  if (ar != 0) return false;  // m-contiguous A tiles are not instantiated
  auto fits = [&](int bm, int bn, int bk) { return g.M % bm == 0 && g.N % bn == 0 && g.K % bk == 0; };
  const bool dual = g.dual != 0;
  const int64_t tiles256 = (int64_t)(g.M / 256) * (g.N / 256) * g.batch;
  switch (kind) {
    case MMA_BF16: return pick_bf16(g, br, c);
    case MMA_F16: return pick_f16(g, br, c);
    case MMA_I8: return pick_i8(g, br, c);
    case MMA_FP8: return pick_fp8(g, br, c);
    case MMA_F32: return pick_f32(g, br, c);
  }
  return false;
}

const char* gemm_kernel_name(const GemmArgs& a) {
  Choice c;
  if (pick_mfma(a, &c)) return c.name;
  return "gemm_generic";
}

void launch_gemm(const GemmArgs& g, hipStream_t stream) {
  if (g.M == 0 || g.N == 0 || g.batch == 0) return;
  Choice c;
  hipError_t e;
  if (g.K > 0 && pick_mfma(g, &c)) {
    // shape invariants the MFMA kernels rely on (checked again here, right before the launch)
    if (g.M % c.bm || g.N % c.bn) fail(PJRT_Error_Code_INTERNAL, "gemm tile mismatch");
    if (c.lds > 65536) {
      e = hipFuncSetAttribute(c.fn, hipFuncAttributeMaxDynamicSharedMemorySize, c.lds);
      if (e != hipSuccess) fail(PJRT_Error_Code_INTERNAL, std::string("LDS attribute failed: ") + hipGetErrorString(e));
    }
    int64_t blocks = (int64_t)(g.M / c.bm) * (g.N / c.bn) * g.batch;
    if (blocks > INT32_MAX) fail(PJRT_Error_Code_UNIMPLEMENTED, "too many GEMM tiles");
    void* args[] = {(void*)&g};
    e = hipLaunchKernel(c.fn, dim3((unsigned)blocks), dim3(c.threads), args, (size_t)c.lds, stream);
  } else {
    dim3 grid((g.N + 63) / 64, (g.M + 63) / 64, g.batch), block(256);
    if (g.batch > 65535) fail(PJRT_Error_Code_UNIMPLEMENTED, "batch too large for the generic GEMM");
    if (g.acc_is_int) {
      if (g.dual) fail(PJRT_Error_Code_UNIMPLEMENTED, "integer dual GEMM");
      hipLaunchKernelGGL((gemm_generic_kernel<true, false>), grid, block, 0, stream, g);
    } else if (g.dual) {
      hipLaunchKernelGGL((gemm_generic_kernel<false, true>), grid, block, 0, stream, g);
    } else {
      hipLaunchKernelGGL((gemm_generic_kernel<false, false>), grid, block, 0, stream, g);
    }
    e = hipGetLastError();
  }
  if (e != hipSuccess) fail(PJRT_Error_Code_INTERNAL, std::string("gemm launch failed: ") + hipGetErrorString(e));
}

}  // namespace ryft
