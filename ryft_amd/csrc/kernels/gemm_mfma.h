// MFMA GEMM kernel template for gfx950, shared by the per-type translation units (k_gemm_<type>.hip).
#pragma once
// GEMM kernels for gfx950 (see also k_gemm_dispatch.hip).
//
// MFMA path: one workgroup computes a BM×BN tile of C[b] = A[b]·B[b]ᵀ (B addressed as [n, k]); WM×WN wavefronts
// each own a (BM/WM)×(BN/WN) sub-tile made of 32×32 MFMA tiles. Operand tiles are staged through LDS in a
// K-packed layout (each row holds BK consecutive k of one m or n), double-buffered so that the global loads of
// k-tile t+1 are in flight while the MFMAs of k-tile t run. Operands whose contiguous dimension is m / n (row-major
// [K, N] weights, for example) are transposed in registers with v_perm_b32 on their way into LDS, so no separate
// transpose pass over HBM is needed. Workgroups are mapped onto the 8 XCDs so that the tiles one XCD computes
// share A row-panels and B column-panels in that XCD's L2.
//
// Instruction per compute type (all dense, f32 or i32 accumulation):
//   bf16  v_mfma_f32_32x32x16_bf16      f16  v_mfma_f32_32x32x16_f16
//   i8    v_mfma_i32_32x32x32_i8        fp8  v_mfma_f32_32x32x64_f8f6f4 (e4m3 × e4m3, unit scales)
//   f32   v_mfma_f32_32x32x2_f32
//
// Generic path: a 64×64 LDS-tiled FMA kernel that reads any element type through any strides (bounds-checked); it
// serves shapes and type mixes the MFMA instantiations do not cover.
#include <hip/hip_runtime.h>

#include <string>
#include <type_traits>

#include "../common.h"
#include "gemm_epilogue.h"
#include "kernels.h"

namespace ryft {

typedef __bf16 bf16x8_t __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef _Float16 f16x8_t __attribute__((__vector_size__(8 * sizeof(_Float16))));
typedef float f32x16_t __attribute__((__vector_size__(16 * sizeof(float))));
typedef int i32x16_t __attribute__((__vector_size__(16 * sizeof(int))));
typedef int i32x4_t __attribute__((__vector_size__(4 * sizeof(int))));
typedef int i32x8_t __attribute__((__vector_size__(8 * sizeof(int))));
// 16-byte register vector. A native vector type rather than HIP's uint4 struct: copies of the struct lower to
// memcpy, which keeps register arrays of it (prefetched tiles, fragments) in private memory.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------------------------------------ MFMA GEMM
enum MmaKind { MMA_BF16 = 0, MMA_F16 = 1, MMA_I8 = 2, MMA_FP8 = 3, MMA_F32 = 4 };

template <int KIND> struct Mma;
template <> struct Mma<MMA_BF16> {
  static constexpr int ESIZE = 2, KPACK = 8;
  using Acc = f32x16_t;
  static constexpr bool INT = false;
  __device__ static Acc mma(const u32x4& a, const u32x4& b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
};
template <> struct Mma<MMA_F16> {
  static constexpr int ESIZE = 2, KPACK = 8;
  using Acc = f32x16_t;
  static constexpr bool INT = false;
  __device__ static Acc mma(const u32x4& a, const u32x4& b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
};
template <> struct Mma<MMA_I8> {
  static constexpr int ESIZE = 1, KPACK = 16;
  using Acc = i32x16_t;
  static constexpr bool INT = true;
  __device__ static Acc mma(const u32x4& a, const u32x4& b, Acc c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4_t, a), __builtin_bit_cast(i32x4_t, b), c, 0, 0, 0);
  }
};
struct U8x32 { u32x4 lo, hi; };
template <> struct Mma<MMA_FP8> {
  static constexpr int ESIZE = 1, KPACK = 32;
  using Acc = f32x16_t;
  static constexpr bool INT = false;
  __device__ static Acc mma(const U8x32& a, const U8x32& b, Acc c) {
    i32x8_t av = {(int)a.lo.x, (int)a.lo.y, (int)a.lo.z, (int)a.lo.w, (int)a.hi.x, (int)a.hi.y, (int)a.hi.z, (int)a.hi.w};
    i32x8_t bv = {(int)b.lo.x, (int)b.lo.y, (int)b.lo.z, (int)b.lo.w, (int)b.hi.x, (int)b.hi.y, (int)b.hi.z, (int)b.hi.w};
    // format 0 = fp8 e4m3 for both operands; zero scale operands select the unscaled instruction
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, c, 0, 0, 0, 0, 0, 0);
  }
};
template <> struct Mma<MMA_F32> {
  static constexpr int ESIZE = 4, KPACK = 1;
  using Acc = f32x16_t;
  static constexpr bool INT = false;
  __device__ static Acc mma(float a, float b, Acc c) { return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0); }
};

// Fragment type and LDS read for KPACK·ESIZE bytes per lane.
template <int BYTES> struct Frag;
template <> struct Frag<4> {
  using T = float;
  __device__ static T load(const char* p) { return *(const float*)p; }
};
template <> struct Frag<16> {
  using T = u32x4;
  __device__ static T load(const char* p) { return *(const u32x4*)p; }
};
template <> struct Frag<32> {
  using T = U8x32;
  __device__ static T load(const char* p) { return U8x32{*(const u32x4*)p, *(const u32x4*)(p + 16)}; }
};

// v_perm_b32 helper: result bytes picked from {lo: bytes 0-3, hi: bytes 4-7} by `sel`.
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// One operand tile (R rows × BK k) global → registers → LDS (K-packed rows of LDK bytes).
template <int ESIZE, int R, int BK, int THREADS, bool RCONTIG>
struct TileLoader {
  static constexpr int VE = 16 / ESIZE;                       // elements per 16-byte vector
  static constexpr int KP = ESIZE == 2 ? 8 : (ESIZE == 1 ? 4 : 1);  // k rows per transposed block
  static constexpr int NTOT = RCONTIG ? (BK / KP) * (R / VE) : R * BK / VE;  // vectors / blocks per tile
  static constexpr int NVEC = (NTOT + THREADS - 1) / THREADS;
  static constexpr bool PARTIAL = (NTOT % THREADS) != 0;  // some threads idle on the last round
  static constexpr int NREG = RCONTIG ? NVEC * KP : NVEC;
  static_assert(!PARTIAL || NVEC == 1, "uneven tile split");
  u32x4 regs[NREG];

  // base: element pointer of (row 0, k 0) of this tile; sr / sk: element strides
  __device__ __forceinline__ void load(const char* base, int64_t sr, int64_t sk, int tid) {
#pragma unroll
    for (int i = 0; i < NVEC; ++i) {
      int v = tid + i * THREADS;
      if (PARTIAL && v >= NTOT) break;
      if (!RCONTIG) {
        int row = v / (BK / VE), kv = v % (BK / VE);
        regs[i] = *(const u32x4*)(base + ((int64_t)row * sr + (int64_t)kv * VE) * ESIZE);
      } else {
        // consecutive lanes take consecutive k-blocks of one row group: their transposed LDS stores then land in
        // distinct banks (lanes 8 rows apart would share banks), and each global row is still read in 128-byte runs
        int kb = v % (BK / KP), rv = v / (BK / KP);
#pragma unroll
        for (int q = 0; q < KP; ++q)
          regs[i * KP + q] = *(const u32x4*)(base + ((int64_t)(kb * KP + q) * sk + (int64_t)rv * VE) * ESIZE);
      }
    }
  }

  template <int LDK>
  __device__ __forceinline__ void store(char* lds, int tid) {
#pragma unroll
    for (int i = 0; i < NVEC; ++i) {
      int v = tid + i * THREADS;
      if (PARTIAL && v >= NTOT) break;
      if (!RCONTIG) {
        int row = v / (BK / VE), kv = v % (BK / VE);
        *(u32x4*)(lds + row * LDK + kv * 16) = regs[i];
      } else {
        // consecutive lanes take consecutive k-blocks of one row group: their transposed LDS stores then land in
        // distinct banks (lanes 8 rows apart would share banks), and each global row is still read in 128-byte runs
        int kb = v % (BK / KP), rv = v / (BK / KP);
#define IN(q) regs[i * KP + (q)]
        if (ESIZE == 2) {
          // 8 k-rows × 8 elements → 8 rows (one per element) of 8 consecutive k
          uint32_t w[8][4];
#pragma unroll
          for (int q = 0; q < 8; ++q) { w[q][0] = IN(q).x; w[q][1] = IN(q).y; w[q][2] = IN(q).z; w[q][3] = IN(q).w; }
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            u32x4 lo, hi;
            lo.x = perm(w[1][t], w[0][t], 0x05040100u); hi.x = perm(w[1][t], w[0][t], 0x07060302u);
            lo.y = perm(w[3][t], w[2][t], 0x05040100u); hi.y = perm(w[3][t], w[2][t], 0x07060302u);
            lo.z = perm(w[5][t], w[4][t], 0x05040100u); hi.z = perm(w[5][t], w[4][t], 0x07060302u);
            lo.w = perm(w[7][t], w[6][t], 0x05040100u); hi.w = perm(w[7][t], w[6][t], 0x07060302u);
            *(u32x4*)(lds + (rv * VE + 2 * t) * LDK + kb * 16) = lo;
            *(u32x4*)(lds + (rv * VE + 2 * t + 1) * LDK + kb * 16) = hi;
          }
        } else if (ESIZE == 1) {
          // 4 k-rows × 16 bytes → 16 rows of 4 consecutive k
          uint32_t w[4][4];
#pragma unroll
          for (int q = 0; q < 4; ++q) { w[q][0] = IN(q).x; w[q][1] = IN(q).y; w[q][2] = IN(q).z; w[q][3] = IN(q).w; }
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            uint32_t p01l = perm(w[1][t], w[0][t], 0x05010400u), p01h = perm(w[1][t], w[0][t], 0x07030602u);
            uint32_t p23l = perm(w[3][t], w[2][t], 0x05010400u), p23h = perm(w[3][t], w[2][t], 0x07030602u);
            int r = rv * VE + 4 * t;
            *(uint32_t*)(lds + (r + 0) * LDK + kb * 4) = perm(p23l, p01l, 0x05040100u);
            *(uint32_t*)(lds + (r + 1) * LDK + kb * 4) = perm(p23l, p01l, 0x07060302u);
            *(uint32_t*)(lds + (r + 2) * LDK + kb * 4) = perm(p23h, p01h, 0x05040100u);
            *(uint32_t*)(lds + (r + 3) * LDK + kb * 4) = perm(p23h, p01h, 0x07060302u);
          }
        } else {
          // one k-row × 4 floats → 4 rows
          *(uint32_t*)(lds + (rv * VE + 0) * LDK + kb * 4) = IN(0).x;
          *(uint32_t*)(lds + (rv * VE + 1) * LDK + kb * 4) = IN(0).y;
          *(uint32_t*)(lds + (rv * VE + 2) * LDK + kb * 4) = IN(0).z;
          *(uint32_t*)(lds + (rv * VE + 3) * LDK + kb * 4) = IN(0).w;
#undef IN
        }
      }
    }
  }
};

template <int KIND, int BM, int BN, int BK, int WM, int WN, bool A_R, bool B_R, bool DUAL>
struct MfmaCfg {
  using M = Mma<KIND>;
  static constexpr int ESIZE = M::ESIZE, KPACK = M::KPACK, MK = 2 * KPACK;
  static constexpr int THREADS = 64 * WM * WN;
  static constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 32, TN = WTN / 32;
  static constexpr int LDK = BK * ESIZE + 16;  // LDS row pitch in bytes (16-byte pad)
  static constexpr int NB = DUAL ? 2 : 1;
  static constexpr int STAGE = (BM + NB * BN) * LDK;
  static constexpr int LDS_BYTES = 2 * STAGE;
  static_assert(BK % MK == 0, "BK must be a multiple of the MFMA K");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32");
  // epilogue rounds: the largest number of 32-row tile-rows (dividing TM) whose f32 patches fit in the LDS
  static constexpr int epi_bytes(int rows) { return WM * WN * NB * rows * 32 * (WTN + 1) * 4; }
  static constexpr int EPI_ROWS = (TM % 4 == 0 && epi_bytes(4) <= LDS_BYTES)   ? 4
                                  : (TM % 2 == 0 && epi_bytes(2) <= LDS_BYTES) ? 2
                                                                               : 1;
  static_assert(epi_bytes(EPI_ROWS) <= LDS_BYTES, "LDS too small for the epilogue patches");
};

// Stores 16 consecutive values of one output row with 16-byte vector stores.
__device__ __forceinline__ void store_row16(void* out, int64_t lin, int dtype, const uint32_t* v, bool is_float) {
  switch (dtype) {
    case DT_F32: case DT_S32: case DT_U32: {
      u32x4* p = (u32x4*)((char*)out + lin * 4);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          uint32_t x = v[4 * q + e];
          w[e] = (dtype == DT_F32) ? (is_float ? x : __float_as_uint((float)(int32_t)x)) : x;
        }
        p[q] = u32x4{w[0], w[1], w[2], w[3]};
      }
      break;
    }
    case DT_BF16: case DT_F16: {
      uint32_t w[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float a = is_float ? __uint_as_float(v[2 * e]) : (float)(int32_t)v[2 * e];
        float c = is_float ? __uint_as_float(v[2 * e + 1]) : (float)(int32_t)v[2 * e + 1];
        if (dtype == DT_BF16) {
          w[e] = (uint32_t)f32_to_bf16_bits(a) | ((uint32_t)f32_to_bf16_bits(c) << 16);
        } else {
          _Float16 ha = (_Float16)a, hc = (_Float16)c;
          w[e] = (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hc) << 16);
        }
      }
      u32x4* p = (u32x4*)((char*)out + lin * 2);
      p[0] = u32x4{w[0], w[1], w[2], w[3]};
      p[1] = u32x4{w[4], w[5], w[6], w[7]};
      break;
    }
    case DT_F8E4M3FN: case DT_F8E5M2: case DT_S8: case DT_U8: {
      uint32_t w[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t x = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          uint32_t bits = v[4 * q + e], byte;
          float f = is_float ? __uint_as_float(bits) : (float)(int32_t)bits;
          if (dtype == DT_F8E4M3FN) byte = f32_to_e4m3fn_bits(f);
          else if (dtype == DT_F8E5M2) byte = f32_to_e5m2_bits(f);
          else byte = is_float ? (uint32_t)f2i_sat(f, dtype) & 0xffu : bits & 0xffu;
          x |= byte << (8 * e);
        }
        w[q] = x;
      }
      *(u32x4*)((char*)out + lin) = u32x4{w[0], w[1], w[2], w[3]};
      break;
    }
    default:
#pragma unroll
      for (int e = 0; e < 16; ++e) store_bits(out, lin + e, dtype, v[e], is_float);
      break;
  }
}

// Bits of accumulator element r (f32 → its bit pattern, i32 → itself).
__device__ __forceinline__ uint32_t acc_elem_bits(const f32x16_t& v, int r) {
  float x = v[r];
  return __float_as_uint(x);
}
__device__ __forceinline__ uint32_t acc_elem_bits(const i32x16_t& v, int r) {
  int x = v[r];
  return (uint32_t)x;
}

template <int I> using int_c = std::integral_constant<int, I>;
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(int_c<I>{});
    static_for<I + 1, N>(f);
  }
}

// Epilogue of 16 consecutive accumulators of output row m, columns [n, n+16): `seg` points at them in LDS, `seg2`
// at the second accumulator of a dual GEMM. Handles EPI_STORE / EPI_SCALE / EPI_SWIGLU; programs (EPI_PROGRAM) run
// on the generic kernel.
template <bool INT, bool DUAL>
__device__ __forceinline__ void epilogue_row16(const GemmArgs& G, int b, int m, int n, const uint32_t* seg,
                                               const uint32_t* seg2) {
  const int64_t lin = ((int64_t)b * G.M + m) * (int64_t)G.N + n;
  uint32_t raw[16], v[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) raw[c] = seg[c];
  if (G.epilogue == EPI_STORE) {
    store_row16(G.out_ptr[0], lin, G.out_dtype[0], raw, !INT);
    return;
  }
  if (G.epilogue == EPI_SCALE) {
    float rs = G.alpha;
    if (G.row) rs *= G.row[(int64_t)b * G.row_sb + (int64_t)m * G.row_sm];
    const float* col = G.col ? G.col + (int64_t)b * G.col_sb + (int64_t)n * G.col_sn : nullptr;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      float x = INT ? (float)(int32_t)raw[c] : __uint_as_float(raw[c]);
      x *= rs;
      if (col) x *= col[(int64_t)c * G.col_sn];
      if (G.mid_round) x = round_float(x, G.mid_round);
      v[c] = __float_as_uint(x);
    }
    store_row16(G.out_ptr[0], lin, G.out_dtype[0], v, true);
    if (G.raw_out) store_row16(G.out_ptr[1], lin, G.out_dtype[1], raw, !INT);
    return;
  }
  if constexpr (DUAL) {  // EPI_SWIGLU
    const float* c1 = G.col ? G.col + (int64_t)b * G.col_sb + (int64_t)n * G.col_sn : nullptr;
    const float* c2 = G.col2 ? G.col2 + (int64_t)b * G.col2_sb + (int64_t)n * G.col2_sn : nullptr;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      float a = __uint_as_float(raw[c]);
      float u = __uint_as_float(seg2[c]);
      if (c1) a *= c1[(int64_t)c * G.col_sn];
      if (c2) u *= c2[(int64_t)c * G.col2_sn];
      float lg = 1.0f / (1.0f + expf(-a));
      float x = (a * lg) * u;
      if (G.mid_round) x = round_float(x, G.mid_round);
      v[c] = __float_as_uint(x);
    }
    store_row16(G.out_ptr[0], lin, G.out_dtype[0], v, true);
  }
}

template <int KIND, int BM, int BN, int BK, int WM, int WN, bool A_R, bool B_R, bool DUAL>
__global__ void __launch_bounds__(64 * WM * WN) gemm_mfma_kernel(const GemmArgs G) {
  using C = MfmaCfg<KIND, BM, BN, BK, WM, WN, A_R, B_R, DUAL>;
  using M = typename C::M;
  using Acc = typename M::Acc;
  using F = Frag<C::KPACK * C::ESIZE>;
  constexpr int ES = C::ESIZE;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // XCD-aware tile order: consecutive workgroup ids land on different XCDs (round-robin), so regroup them such that
  // each XCD owns a contiguous run of (batch, tile-row, tile-col) tiles.
  const int tiles_n = G.N / BN, tiles_m = G.M / BM;
  const int total = tiles_n * tiles_m * G.batch;
  int bid = blockIdx.x;
  if ((total & 7) == 0) bid = (bid & 7) * (total >> 3) + (bid >> 3);
  const int tn = bid % tiles_n;
  const int tm = (bid / tiles_n) % tiles_m;
  const int b = bid / (tiles_n * tiles_m);
  const int m0 = tm * BM, n0 = tn * BN;

  const char* Ab = (const char*)G.A.ptr + ((int64_t)b * G.A.sb + (int64_t)m0 * G.A.sr) * ES;
  const char* Bb = (const char*)G.B.ptr + ((int64_t)b * G.B.sb + (int64_t)n0 * G.B.sr) * ES;
  const char* B2b = DUAL ? (const char*)G.B2.ptr + ((int64_t)b * G.B2.sb + (int64_t)n0 * G.B2.sr) * ES : nullptr;

  TileLoader<ES, BM, BK, C::THREADS, A_R> la;
  TileLoader<ES, BN, BK, C::THREADS, B_R> lb;
  TileLoader<ES, BN, BK, C::THREADS, B_R> lb2;

  Acc acc[C::TM][C::TN];
  Acc acc2[DUAL ? C::TM : 1][DUAL ? C::TN : 1];
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j) {
      acc[i][j] = Acc{};
      if constexpr (DUAL) acc2[i][j] = Acc{};
    }

  const int KT = G.K / BK;
  auto gload = [&](int kt) {
    const int64_t ko = (int64_t)kt * BK;
    la.load(Ab + ko * G.A.sk * ES, G.A.sr, G.A.sk, tid);
    lb.load(Bb + ko * G.B.sk * ES, G.B.sr, G.B.sk, tid);
    if constexpr (DUAL) lb2.load(B2b + ko * G.B2.sk * ES, G.B2.sr, G.B2.sk, tid);
  };
  auto lstore = [&](int buf) {
    char* s = smem + buf * C::STAGE;
    la.template store<C::LDK>(s, tid);
    lb.template store<C::LDK>(s + BM * C::LDK, tid);
    if constexpr (DUAL) lb2.template store<C::LDK>(s + (BM + BN) * C::LDK, tid);
  };

  gload(0);
  lstore(0);
  __syncthreads();
  const int lrow = lane & 31;
  const int lk = (lane >> 5) * C::KPACK * ES;  // byte offset of this lane's k-pack within an MFMA k-step
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
    const char* sA = smem + cur * C::STAGE + (wm * C::WTM + lrow) * C::LDK + lk;
    const char* sB = smem + cur * C::STAGE + BM * C::LDK + (wn * C::WTN + lrow) * C::LDK + lk;
    const char* sB2 = sB + BN * C::LDK;
#pragma unroll
    for (int s = 0; s < BK / C::MK; ++s) {
      const int ko = s * C::MK * ES;
      typename F::T af[C::TM], bf[C::TN], bf2[DUAL ? C::TN : 1];
#pragma unroll
      for (int i = 0; i < C::TM; ++i) af[i] = F::load(sA + i * 32 * C::LDK + ko);
#pragma unroll
      for (int j = 0; j < C::TN; ++j) {
        bf[j] = F::load(sB + j * 32 * C::LDK + ko);
        if constexpr (DUAL) bf2[j] = F::load(sB2 + j * 32 * C::LDK + ko);
      }
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j) {
          acc[i][j] = M::mma(af[i], bf[j], acc[i][j]);
          if constexpr (DUAL) acc2[i][j] = M::mma(af[i], bf2[j], acc2[i][j]);
        }
    }
    if (kt + 1 < KT) lstore(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: acc register r of lane l holds C[8·(r/4) + 4·(l/32) + r%4][l%32] of its 32×32 tile. The wave's
  // accumulators go to LDS in rounds of EPI_ROWS tile-rows (compile-time indices keep them in registers until then);
  // a rolled loop then hands each lane 16-column row segments, so stores are contiguous and the epilogue body is
  // compiled once.
  constexpr int PITCH = C::WTN + 1;  // words per LDS row (+1 against bank conflicts)
  constexpr int EPI_ROWS = C::EPI_ROWS;
  constexpr int REGION = EPI_ROWS * 32 * PITCH;
  uint32_t* patch = (uint32_t*)smem + wave * C::NB * REGION;
  static_for<0, C::TM / EPI_ROWS>([&](auto rd) {
    constexpr int round = decltype(rd)::value;
    static_for<0, EPI_ROWS * C::TN>([&](auto t) {
      constexpr int il = decltype(t)::value / C::TN, j = decltype(t)::value % C::TN;
      constexpr int i = round * EPI_ROWS + il;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = il * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        // (element reads through the vector subscript, then a value conversion: a bit-cast of the subscript
        //  expression was lowered to element 0 for every r)
        patch[row * PITCH + j * 32 + (lane & 31)] = acc_elem_bits(acc[i][j], r);
        if constexpr (DUAL) patch[REGION + row * PITCH + j * 32 + (lane & 31)] = acc_elem_bits(acc2[i][j], r);
      }
    });
    __syncthreads();
    constexpr int SEGS = EPI_ROWS * 32 * (C::WTN / 16);
    for (int s = lane; s < SEGS; s += 64) {
      const int row = s / (C::WTN / 16), c0 = (s % (C::WTN / 16)) * 16;
      const uint32_t* seg = patch + row * PITCH + c0;
      epilogue_row16<M::INT, DUAL>(G, b, m0 + wm * C::WTM + round * EPI_ROWS * 32 + row, n0 + wn * C::WTN + c0, seg,
                                   DUAL ? seg + REGION : nullptr);
    }
    __syncthreads();
  });
}


// ------------------------------------------------------------------------------------------------ dispatch
struct Choice {
  const void* fn = nullptr;
  int threads = 256;
  int lds = 0;
  int bm = 0, bn = 0;
  const char* name = "gemm_generic";
};

template <int KIND, int BM, int BN, int BK, int WM, int WN, bool A_R, bool B_R, bool DUAL>
Choice make_choice(const char* name) {
  using C = MfmaCfg<KIND, BM, BN, BK, WM, WN, A_R, B_R, DUAL>;
  Choice c;
  c.fn = (const void*)&gemm_mfma_kernel<KIND, BM, BN, BK, WM, WN, A_R, B_R, DUAL>;
  c.threads = C::THREADS;
  c.lds = C::LDS_BYTES;
  c.bm = BM;
  c.bn = BN;
  c.name = name;
  return c;
}

// Per-type instantiation pickers (one translation unit each, so the build parallelises). `br`: B is n-contiguous.
bool pick_bf16(const GemmArgs& g, bool br, Choice* c);
bool pick_f16(const GemmArgs& g, bool br, Choice* c);
bool pick_i8(const GemmArgs& g, bool br, Choice* c);
bool pick_fp8(const GemmArgs& g, bool br, Choice* c);
bool pick_f32(const GemmArgs& g, bool br, Choice* c);

}  // namespace ryft
