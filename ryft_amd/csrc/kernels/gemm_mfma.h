// MFMA GEMM kernel template for gfx950, shared by the per-type translation units (k_gemm_<type>.hip).
#pragma once
// GEMM kernels for gfx950 (see also k_gemm_dispatch.hip).
//
// MFMA path: one workgroup computes a BM×BN tile of C[b] = A[b]·B[b]ᵀ (B addressed as [n, k]); WM×WN wavefronts
// each own a (BM/WM)×(BN/WN) sub-tile made of 32×32 MFMA tiles. Full tiles of a K-contiguous A go from global memory
// straight into LDS (buffer_load ... lds) in unpadded, XOR-swizzled K-packed rows (each row holds BK consecutive k of
// one m), together with B — K-packed the same way, or, when its contiguous dimension is n (row-major [K, N] weights),
// as unchanged [k][n] rows read back with transposing LDS reads — in two or three LDS stages, so no register staging
// and no LDS store instructions are needed. Edge tiles and m-contiguous A operands take a register-staged path
// instead: buffer loads one k-tile ahead into registers, padded LDS rows, m / n-contiguous operands transposed in
// registers with v_perm_b32 on their way into LDS. Either way LDS fragments are double-buffered in registers across
// k-steps and across the one barrier per k-tile, and no separate transpose pass over HBM is needed. Workgroups are
// mapped onto the 8 XCDs so that the tiles one XCD computes share A row-panels and B column-panels in that XCD's L2.
//
// Instruction per compute type (all dense, f32 or i32 accumulation):
//   bf16  v_mfma_f32_32x32x16_bf16      f16  v_mfma_f32_32x32x16_f16
//   i8    v_mfma_i32_32x32x32_i8        fp8  v_mfma_f32_32x32x64_f8f6f4 (e4m3 × e4m3, unit scales)
//   f32   v_mfma_f32_32x32x2_f32
//   bf16 × f8E4M3FN (weight-only quantised B): B is read from HBM as f8E4M3FN bytes and widened exactly to bf16
//   (v_cvt_scalef32_pk_bf16_fp8, unit scale) between its registers and LDS; the MFMA is the bf16 one
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
enum MmaKind { MMA_BF16 = 0, MMA_F16 = 1, MMA_I8 = 2, MMA_FP8 = 3, MMA_F32 = 4, MMA_BF16_F8 = 5 };

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
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
template <> struct Mma<MMA_FP8> {
  static constexpr int ESIZE = 1, KPACK = 32;
  using Acc = f32x16_t;
  static constexpr bool INT = false;
  __device__ static Acc mma(const u32x8& a, const u32x8& b, Acc c) {
    // format 0 = fp8 e4m3 for both operands; zero scale operands select the unscaled instruction
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(__builtin_bit_cast(i32x8_t, a), __builtin_bit_cast(i32x8_t, b),
                                                           c, 0, 0, 0, 0, 0, 0);
  }
};
template <> struct Mma<MMA_F32> {
  static constexpr int ESIZE = 4, KPACK = 1;
  using Acc = f32x16_t;
  static constexpr bool INT = false;
  __device__ static Acc mma(float a, float b, Acc c) { return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0); }
};
// bf16 activations × f8E4M3FN weights: the bf16 MFMA on B tiles widened to bf16 in LDS.
template <> struct Mma<MMA_BF16_F8> : Mma<MMA_BF16> {};

// Element size of B in HBM (differs from the LDS / MFMA element size only for widened B operands).
template <int KIND> constexpr int b_hbm_size() { return KIND == MMA_BF16_F8 ? 1 : Mma<KIND>::ESIZE; }

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
  using T = u32x8;
  __device__ static T load(const char* p) {
    u32x4 lo = *(const u32x4*)p, hi = *(const u32x4*)(p + 16);
    return u32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
  }
};

// v_perm_b32 helper: result bytes picked from {lo: bytes 0-3, hi: bytes 4-7} by `sel`.
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// Bounds of one k-tile's loads in the edge kernels (shapes that are not tile multiples): the buffer resource covers
// `nrec` bytes from the tile origin (rows past the operand's last byte read as zero instead of faulting), and the k
// positions at or beyond `kvalid` are loaded as zeros (an offset past `nrec`, which the hardware returns as 0), so the
// last, partial k-tile contributes nothing beyond K. Rows past M / N inside the operand's memory only feed output rows
// / columns that are never stored.
struct LoadBounds {
  int nrec = -1;     // bytes from the tile origin (-1: unchecked)
  int kvalid = 1 << 30;
};
__device__ __forceinline__ int masked_off(int64_t off, bool valid) { return valid ? (int)off : (int)0x80000000u; }

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

  // base: element pointer of (row 0, k 0) of this tile; sr / sk: element strides. Loads go through a buffer
  // resource whose base is this k-tile's origin (scalar registers), so the per-lane byte offsets are loop-invariant
  // 32-bit values (the host checks that one tile spans less than 2 GiB).
  template <bool EDGE = false>
  __device__ __forceinline__ void load(const char* base, int64_t sr, int64_t sk, int tid, LoadBounds lb = {}) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, EDGE ? lb.nrec : -1, 0x00020000);
#pragma unroll
    for (int i = 0; i < NVEC; ++i) {
      int v = tid + i * THREADS;
      if (PARTIAL && v >= NTOT) break;
      if (!RCONTIG) {
        int row = v / (BK / VE), kv = v % (BK / VE);
        const int64_t off = ((int64_t)row * sr + (int64_t)kv * VE) * ESIZE;
        regs[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, EDGE ? masked_off(off, kv * VE < lb.kvalid) : (int)off, 0, 0);
      } else {
        // consecutive lanes take consecutive k-blocks of one row group: their transposed LDS stores then land in
        // distinct banks (lanes 8 rows apart would share banks), and each global row is still read in 128-byte runs
        int kb = v % (BK / KP), rv = v / (BK / KP);
#pragma unroll
        for (int q = 0; q < KP; ++q) {
          const int64_t off = ((int64_t)(kb * KP + q) * sk + (int64_t)rv * VE) * ESIZE;
          regs[i * KP + q] = __builtin_amdgcn_raw_buffer_load_b128(
              rs, EDGE ? masked_off(off, kb * KP + q < lb.kvalid) : (int)off, 0, 0);
        }
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

// One row-contiguous operand tile (BK k-rows × R elements) global → registers → LDS, copied unchanged ([k][R] rows
// of LDB bytes), read later with transposing LDS reads.
template <int ESIZE, int R, int BK, int THREADS>
struct TileCopyLoader {
  static constexpr int VE = 16 / ESIZE;
  static constexpr int NTOT = BK * (R / VE);
  static constexpr int NVEC = NTOT / THREADS;
  static_assert(NTOT % THREADS == 0, "uneven tile split");
  u32x4 regs[NVEC];
  template <bool EDGE = false>
  __device__ __forceinline__ void load(const char* base, int64_t sr, int64_t sk, int tid, LoadBounds lb = {}) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, EDGE ? lb.nrec : -1, 0x00020000);
    (void)sr;  // row-contiguous: the element stride along R is 1
#pragma unroll
    for (int i = 0; i < NVEC; ++i) {
      const int v = tid + i * THREADS;
      const int k = v / (R / VE), c = v % (R / VE);
      const int64_t off = ((int64_t)k * sk + (int64_t)c * VE) * ESIZE;
      regs[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, EDGE ? masked_off(off, k < lb.kvalid) : (int)off, 0, 0);
    }
  }
  template <int LDB>
  __device__ __forceinline__ void store(char* lds, int tid) {
#pragma unroll
    for (int i = 0; i < NVEC; ++i) {
      const int v = tid + i * THREADS;
      const int k = v / (R / VE), c = v % (R / VE);
      *(u32x4*)(lds + k * LDB + c * 16) = regs[i];
    }
  }
};

// f8E4M3FN → bf16, 8 values (one 8-byte piece → one 16-byte chunk): v_cvt_scalef32_pk_bf16_fp8 widens two bytes of
// a word per instruction. Exact: every f8E4M3FN value (subnormals included) is a bf16 value and the unit scale
// multiplies exactly; NaN stays NaN.
typedef uint32_t u32x2w __attribute__((__vector_size__(2 * sizeof(uint32_t))));
__device__ __forceinline__ u32x4 f8x8_to_bf16(const u32x2w& v) {
#define RYFT_W(x, s) __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((x), 1.0f, (s)))
  return u32x4{RYFT_W(v[0], false), RYFT_W(v[0], true), RYFT_W(v[1], false), RYFT_W(v[1], true)};
#undef RYFT_W
}

// An f8E4M3FN operand tile widened to bf16 on its way into LDS, in 8-byte pieces (one 16-byte bf16 chunk each):
// consecutive lanes take consecutive pieces of one LDS row, so each 16-lane group of a store writes 256 contiguous
// bytes (conflict-free) and each global read covers whole rows. ROWS rows of PIECES pieces. Used for a K-contiguous
// B (R n-rows × BK k in HBM → K-packed bf16 rows of LDK bytes, like a 16-bit K-packed operand); an n-contiguous f8 B
// is copied into LDS unchanged and widened after its transposing read.
template <int ROWS, int PIECES, int THREADS>
struct TileWidenPieces {
  static constexpr int NTOT = ROWS * PIECES;
  static constexpr int NVEC = (NTOT + THREADS - 1) / THREADS;
  static constexpr bool PARTIAL = (NTOT % THREADS) != 0;
  static_assert(!PARTIAL || NVEC == 1, "uneven tile split");
  u32x2w regs[NVEC];
  // stride_row: HBM bytes between consecutive LDS rows of the tile ([n][k] tiles: sr); pieces run along k
  template <bool EDGE = false>
  __device__ __forceinline__ void load(const char* base, int64_t stride_row, int tid, LoadBounds lb = {}) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, EDGE ? lb.nrec : -1, 0x00020000);
#pragma unroll
    for (int i = 0; i < NVEC; ++i) {
      const int v = tid + i * THREADS;
      if (PARTIAL && v >= NTOT) break;
      const int r = v / PIECES, c = v % PIECES;
      const int64_t off = (int64_t)r * stride_row + (int64_t)c * 8;
      regs[i] = __builtin_amdgcn_raw_buffer_load_b64(rs, EDGE ? masked_off(off, c * 8 < lb.kvalid) : (int)off, 0, 0);
    }
  }
  template <int PITCH>
  __device__ __forceinline__ void store(char* lds, int tid) {
#pragma unroll
    for (int i = 0; i < NVEC; ++i) {
      const int v = tid + i * THREADS;
      if (PARTIAL && v >= NTOT) break;
      const int r = v / PIECES, c = v % PIECES;
      *(u32x4*)(lds + r * PITCH + c * 16) = f8x8_to_bf16(regs[i]);
    }
  }
};

template <int R, int BK, int THREADS>
struct TileWidenLoader : TileWidenPieces<R, BK / 8, THREADS> {
  template <bool EDGE = false>
  __device__ __forceinline__ void load(const char* base, int64_t sr, int64_t sk, int tid, LoadBounds lb = {}) {
    (void)sk;  // K-contiguous
    TileWidenPieces<R, BK / 8, THREADS>::template load<EDGE>(base, sr, tid, lb);
  }
};

typedef short s16x4_t __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16. Within each group of 16 lanes, lane i receives element i % 4 of the 8-byte chunks addressed by
// lanes i/4, i/4 + 4, i/4 + 8, i/4 + 12 of the group (lane layout measured on gfx950). So when lane s of a group
// addresses row k0 + s/4, column c0 + 4·(s % 4) of a [k][n] tile, lane i receives B[k0 .. k0+3][c0 + i].
__device__ __forceinline__ uint2 lds_read_tr16(const char* p) {
  const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4_t*)p);
  return __builtin_bit_cast(uint2, v);
}
typedef int i32x2_t __attribute__((ext_vector_type(2)));
// ds_read_b64_tr_b8. Within each group of 16 lanes, lane i receives byte i % 8 of the 8-byte chunks addressed by
// lanes 2j + i/8 (j = 0..7) of the group (measured on gfx950). So when lane s of a group addresses row k0 + s/2,
// column c0 + 8·(s % 2) of a [k][n] byte tile, lane i receives B[k0 .. k0+7][c0 + i].
__device__ __forceinline__ uint2 lds_read_tr8(const char* p) {
  const i32x2_t v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) i32x2_t*)p);
  return __builtin_bit_cast(uint2, v);
}

// ------------------------------------------------------------------------------------------------ LDS-DMA tiles
// XOR swizzles of the DMA tile layouts: the 16-byte chunk c of tile row r sits at chunk position c ^ swz(r).
// K-packed rows of 128 bytes (A, K-contiguous B): a fragment read takes one chunk of each of 16 consecutive rows per
// 16 lanes (ds_read_b128); rows alternate between the two 128-byte halves of the 64 banks, so the 8 rows of a half
// need 8 distinct positions. Period 16 rows.
__device__ __forceinline__ int swz_k128(int r) { return (r >> 1) & 7; }
// [k][n] rows read with transposing reads (32 lanes per pass): 16-bit rows (≥ 256 bytes): 4 consecutive rows × 4
// consecutive chunks, so the 4 rows' chunk quads go to distinct quads (period 4); 8-bit rows of ≥ 256 bytes: 8 rows
// × 2 chunks (period 8); 8-bit rows of 128 bytes: the even and the odd rows of 8 fall in different bank halves, 4 rows
// × 2 chunks each (period 8).
template <int ES, int RB>
__device__ __forceinline__ int swz_tr(int r) {
  if constexpr (ES == 2) return 4 * (r & 3);
  else if constexpr (RB >= 256) return 2 * (r & 7);
  else return 2 * ((r >> 1) & 3);
}

typedef __attribute__((address_space(3))) void lds_void_t;
// One wave-wide load of 16 bytes per lane from a buffer straight into LDS: lane l's bytes (buffer offset voff + soff)
// land at lds + 16·l (lds and soff wave-uniform).
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, char* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds, 16, voff, soff, 0, 0);
}
// LDS fragment reads as inline assembly: the compiler cannot tell the stage they read from the stages the DMA loads
// are filling and would otherwise wait for every outstanding load before each read. Their completion is waited for
// explicitly (lgkm_wait), with the fragments passed through the wait so that their uses follow it.
template <int OFF>
__device__ __forceinline__ u32x4 lds_rd128(uint32_t a) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(a), "i"(OFF));
  return r;
}
template <int OFF>
__device__ __forceinline__ u32x2v lds_rd_tr16(uint32_t a) {
  u32x2v r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(a), "i"(OFF));
  return r;
}
template <int OFF>
__device__ __forceinline__ u32x2v lds_rd_tr8(uint32_t a) {
  u32x2v r;
  asm volatile("ds_read_b64_tr_b8 %0, %1 offset:%2" : "=v"(r) : "v"(a), "i"(OFF));
  return r;
}
// Waits until at most N of this wave's LDS reads are outstanding.
template <int N>
__device__ __forceinline__ void lgkm_wait() {
  asm volatile("s_waitcnt lgkmcnt(%[n])" ::[n] "n"(N));
}
// Orders the uses of a register after the preceding wait (volatile asm statements keep their order).
template <class T>
__device__ __forceinline__ void after_wait(T& r) {
  asm volatile("" : "+v"(r));
}
// Waits for this wave's DMA loads down to N outstanding and for its LDS reads, then joins the workgroup barrier.
template <int N>
__device__ __forceinline__ void dma_barrier() {
  asm volatile("s_waitcnt vmcnt(%[n]) lgkmcnt(0)\n\ts_barrier" ::[n] "n"(N) : "memory");
}

template <int KIND, int BM, int BN, int BK, int WM, int WN, bool A_R, bool B_R, bool DUAL, bool EDGE = false>
struct MfmaCfg {
  using M = Mma<KIND>;
  static constexpr int ESIZE = M::ESIZE, KPACK = M::KPACK, MK = 2 * KPACK;
  static constexpr int BES = b_hbm_size<KIND>();  // B's element size in HBM (1: f8 for the bf16 MFMA)
  static constexpr int THREADS = 64 * WM * WN;
  static constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 32, TN = WTN / 32;
  static constexpr int LDK = BK * ESIZE + 16;  // LDS row pitch in bytes (16-byte pad)
  static constexpr int NB = DUAL ? 2 : 1;
  // BTR: an n-contiguous 16- or 8-bit B operand is copied into LDS unchanged, [k][n] rows of pitch LDB (≡ 64 resp.
  // 32·odd bytes mod 256, so the rows one transposing read touches fall in distinct banks), and its fragments are read
  // with ds_read_b64_tr_b16 / _b8; otherwise B is K-packed like A ([n][k] rows of pitch LDK, transposed in registers
  // on the way)
  static constexpr bool BTR = B_R && ESIZE <= 2;
  // element size of B in LDS: an n-contiguous f8 B for the bf16 MFMA stays f8 in LDS (half the LDS bytes written
  // and read) and is widened in registers after its transposing read; a K-contiguous one is widened on its way in
  static constexpr int BLES = BTR ? BES : ESIZE;
  static constexpr int LDB = BN * BLES + (BLES == 2 ? 64 : 32);
  static constexpr int BREG = BTR ? BK * LDB : BN * LDK;  // bytes of one B operand tile
  // DMA: full tiles of a K-contiguous A and a B that reaches LDS unchanged (n-contiguous 16- / 8-bit, or K-contiguous
  // without widening) go from global memory straight into LDS (buffer_load ... lds, 16 bytes per lane): unpadded rows
  // whose 16-byte chunks are XOR-swizzled per row (so that the fragment reads stay conflict-free), no register
  // staging and no LDS stores; NST stages (three when they fit) keep the loads two k-tiles ahead.
  static constexpr int RBA = BK * ESIZE;                       // bytes per A row (and per K-contiguous B row)
  static constexpr int RBB = BTR ? BN * BLES : BK * ESIZE;     // bytes per B row ([k][n] rows when BTR)
  static constexpr bool DMA = !EDGE && !A_R && ESIZE <= 2 && (BTR || BES == ESIZE) && RBA == 128 &&
                              (BM * RBA) % (1024 * WM * WN) == 0 && (BTR ? BK : BN) * RBB % (1024 * WM * WN) == 0 &&
                              (!BTR || RBB == 128 || RBB == 256 || RBB == 512);
  static constexpr int BREG_D = BTR ? BK * RBB : BN * RBA;
  static constexpr int STAGE_D = BM * RBA + NB * BREG_D;
  // three stages when they fit the 160 KB of LDS and two stages would already leave room for one workgroup only
  static constexpr int NST = DMA && 3 * STAGE_D <= 163840 && 2 * STAGE_D > 163840 / 2 ? 3 : 2;
  static constexpr int STAGE = DMA ? STAGE_D : BM * LDK + NB * BREG;
  static_assert(BK % MK == 0, "BK must be a multiple of the MFMA K");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32");
  // epilogue rounds: the largest number of 32-row tile-rows (dividing TM) whose f32 patches fit in the LDS the two
  // stages occupy (at least one round's worth)
  static constexpr int epi_bytes(int rows) { return WM * WN * NB * rows * 32 * (WTN + 4) * 4; }
  static constexpr int LDS_BYTES = NST * STAGE > epi_bytes(1) ? NST * STAGE : epi_bytes(1);
  static constexpr int EPI_ROWS = (TM % 4 == 0 && epi_bytes(4) <= LDS_BYTES)   ? 4
                                  : (TM % 2 == 0 && epi_bytes(2) <= LDS_BYTES) ? 2
                                                                               : 1;
  static_assert(epi_bytes(EPI_ROWS) <= LDS_BYTES, "LDS too small for the epilogue patches");
};

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

// ------------------------------------------------------------------------------------------------ epilogue
// Output types the MFMA epilogue writes (others run on the generic kernel): f32 / bf16 / f16 / f8e4m3fn for
// float results, s32 / f32 (and, scaled, bf16 / f16) for integer accumulators.
template <int DT> constexpr int out_size() { return DT == DT_F32 || DT == DT_S32 ? 4 : (DT == DT_BF16 || DT == DT_F16 ? 2 : 1); }

// Element bits of one value in output type DT; `x` is an f32 bit pattern, or an i32 when !is_float.
template <int DT>
__device__ __forceinline__ uint32_t out_bits(uint32_t x, bool is_float) {
  if constexpr (DT == DT_S32) {
    return x;
  } else {
    const float f = is_float ? __uint_as_float(x) : (float)(int32_t)x;
    if constexpr (DT == DT_F32) return __float_as_uint(f);
    else if constexpr (DT == DT_BF16) return f32_to_bf16_bits(f);
    else if constexpr (DT == DT_F16) return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
    else return f32_to_e4m3fn_bits(f);
  }
}

// Device-scope (sc1) vector store and load for the partial sums of split-K ranges: the stores write through to the
// point of device coherence and the loads do not return stale L2 copies, whichever XCD each workgroup runs on, so no
// cache write-back or invalidation is needed between the ranges and the one that finishes the tile. The loads are
// not seen by the compiler's wait-count tracking: wait_loads() completes them.
__device__ __forceinline__ void store_coherent16(void* p, const u32x4& v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ u32x4 load_coherent16(const void* p) {
  u32x4 r;
  asm volatile("global_load_dwordx4 %0, %1, off sc1" : "=v"(r) : "v"(p) : "memory");
  return r;
}

// The first `nvalid` (at most 16 / OS) elements of a 16-byte output chunk packed in w, stored an element at a time.
template <int OS>
__device__ __forceinline__ void store_chunk_elements(char* p, const uint32_t (&w)[4], int nvalid) {
#pragma unroll
  for (int e = 0; e < 16 / OS; ++e) {
    if (e >= nvalid) break;
    const uint32_t word = w[e * OS / 4];
    if constexpr (OS == 4) *(uint32_t*)(p + 4 * e) = word;
    else if constexpr (OS == 2) *(uint16_t*)(p + 2 * e) = (uint16_t)(word >> (16 * (e & 1)));
    else *(uint8_t*)(p + e) = (uint8_t)(word >> (8 * (e & 3)));
  }
}

// One epilogue pass over a wave's staged accumulators: ROWS rows of WTN words at `reg` (and `reg2`, the second
// accumulator of a dual GEMM), row pitch PITCH words. Each lane owns one 16-byte output chunk column (16 / size(DT)
// values) and walks the rows in steps of 64 / chunks-per-row, so consecutive lanes write consecutive bytes of a row.
// KIND is EPI_STORE / EPI_SCALE / EPI_SWIGLU; the output type, the epilogue kind and the trip count are
// compile-time, so each pass is a short unrolled loop whose LDS reads can be issued ahead of the conversions. MIDR:
// the value is rounded to G.mid_round (bf16 or f16) before the output conversion.
template <int KIND, int DT, bool INT, bool MIDR, int WTN, int PITCH, int ROWS, bool EDGE = false, bool COH = false>
__device__ __forceinline__ void epi_pass(const GemmArgs& G, void* out, int b, int m0, int n0, const uint32_t* reg,
                                         const uint32_t* reg2, int lane) {
  constexpr int OS = out_size<DT>();
  constexpr int VPC = 16 / OS;  // values per chunk
  constexpr int CPR = WTN / VPC;
  static_assert(WTN % VPC == 0 && 64 % CPR == 0 && (ROWS * CPR) % 64 == 0, "epilogue chunk layout");
  constexpr int RSTEP = 64 / CPR, ITER = ROWS * CPR / 64;
  const int row0 = lane / CPR, col = (lane % CPR) * VPC;
  const int n = n0 + col;
  // partial edge tiles: columns past N and rows past M are neither read from the per-row / per-column operands nor
  // stored; a chunk that runs past N, or any chunk of rows that are not 16-byte aligned (N·size not a multiple of
  // 16), is stored an element at a time
  const int nvalid = EDGE ? G.N - n : VPC;
  const bool col_ok = nvalid > 0;
  const bool vec_ok = !EDGE || (nvalid >= VPC && ((int64_t)G.N * OS) % 16 == 0);
  char* optr = (char*)out + (((int64_t)b * G.M + m0 + row0) * (int64_t)G.N + n) * OS;
  const int64_t ostep = (int64_t)RSTEP * G.N * OS;
  // per-column operands are the same for every row this lane visits
  float cs[VPC], cs2[VPC];
  if constexpr (KIND == EPI_SCALE || KIND == EPI_SWIGLU) {
    const float* cp = G.col && col_ok ? G.col + (int64_t)b * G.col_sb + (int64_t)n * G.col_sn : nullptr;
#pragma unroll
    for (int e = 0; e < VPC; ++e) cs[e] = cp && e < nvalid ? cp[(int64_t)e * G.col_sn] : 1.0f;
  }
  if constexpr (KIND == EPI_SWIGLU) {
    const float* cp = G.col2 && col_ok ? G.col2 + (int64_t)b * G.col2_sb + (int64_t)n * G.col2_sn : nullptr;
#pragma unroll
    for (int e = 0; e < VPC; ++e) cs2[e] = cp && e < nvalid ? cp[(int64_t)e * G.col2_sn] : 1.0f;
  }
#pragma unroll 4
  for (int it = 0; it < ITER; ++it) {
    const int row = row0 + it * RSTEP;
    if (EDGE && (!col_ok || m0 + row >= G.M)) continue;
    uint32_t v[VPC];
#pragma unroll
    for (int q = 0; q < VPC / 4; ++q) {
      const u32x4 w = *(const u32x4*)(reg + row * PITCH + col + 4 * q);
      v[4 * q] = w.x, v[4 * q + 1] = w.y, v[4 * q + 2] = w.z, v[4 * q + 3] = w.w;
    }
    bool is_float = !INT;
    if constexpr (KIND == EPI_SCALE) {
      float rs = G.alpha;
      if (G.row) rs *= G.row[(int64_t)b * G.row_sb + (int64_t)(m0 + row) * G.row_sm];
#pragma unroll
      for (int e = 0; e < VPC; ++e) {
        float x = INT ? (float)(int32_t)v[e] : __uint_as_float(v[e]);
        x = x * rs * cs[e];
        if constexpr (MIDR) x = G.mid_round == DT_BF16 ? bf16_bits_to_f32(f32_to_bf16_bits(x)) : (float)(_Float16)x;
        v[e] = __float_as_uint(x);
      }
      is_float = true;
    } else if constexpr (KIND == EPI_SWIGLU) {
#pragma unroll
      for (int q = 0; q < VPC / 4; ++q) {
        const u32x4 w = *(const u32x4*)(reg2 + row * PITCH + col + 4 * q);
        const uint32_t u4[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          const int e = 4 * q + e4;
          const float a = __uint_as_float(v[e]) * cs[e];
          const float u = __uint_as_float(u4[e4]) * cs2[e];
          const float lg = 1.0f / (1.0f + expf(-a));
          float x = (a * lg) * u;
          if constexpr (MIDR) x = G.mid_round == DT_BF16 ? bf16_bits_to_f32(f32_to_bf16_bits(x)) : (float)(_Float16)x;
          v[e] = __float_as_uint(x);
        }
      }
      is_float = true;
    }
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if constexpr (OS == 4) {
        w[q] = out_bits<DT>(v[q], is_float);
      } else if constexpr (OS == 2 && DT == DT_BF16) {
        const float a = is_float ? __uint_as_float(v[2 * q]) : (float)(int32_t)v[2 * q];
        const float c = is_float ? __uint_as_float(v[2 * q + 1]) : (float)(int32_t)v[2 * q + 1];
        w[q] = f32x2_to_bf16x2_bits(a, c);
      } else if constexpr (OS == 2) {
        w[q] = out_bits<DT>(v[2 * q], is_float) | (out_bits<DT>(v[2 * q + 1], is_float) << 16);
      } else {
        w[q] = out_bits<DT>(v[4 * q], is_float) | (out_bits<DT>(v[4 * q + 1], is_float) << 8) |
               (out_bits<DT>(v[4 * q + 2], is_float) << 16) | (out_bits<DT>(v[4 * q + 3], is_float) << 24);
      }
    }
    if constexpr (COH) store_coherent16(optr + it * ostep, u32x4{w[0], w[1], w[2], w[3]});
    else if (vec_ok) *(u32x4*)(optr + it * ostep) = u32x4{w[0], w[1], w[2], w[3]};
    else store_chunk_elements<OS>(optr + it * ostep, w, nvalid);
  }
}

// ------------------------------------------------------------------------------------------------ split-K finish
// Eight consecutive summed accumulators of the result (element e0 = (b, m, n .. n+7)) through the epilogue and stored:
// the arithmetic and operation order of the MFMA kernels' epilogue passes. Shared by the reduction kernel and the
// in-kernel finish below, so both give the same bits.
template <int DT>
__device__ __forceinline__ void store_oct(void* out, int64_t e0, const uint32_t* v, bool is_float) {
  constexpr int OS = out_size<DT>();
  uint32_t w[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) w[e] = out_bits<DT>(v[e], is_float);
  char* p = (char*)out + e0 * OS;
  if constexpr (OS == 4) {
    *(u32x4*)p = u32x4{w[0], w[1], w[2], w[3]};
    *(u32x4*)(p + 16) = u32x4{w[4], w[5], w[6], w[7]};
  } else if constexpr (OS == 2) {
    *(u32x4*)p = u32x4{w[0] | w[1] << 16, w[2] | w[3] << 16, w[4] | w[5] << 16, w[6] | w[7] << 16};
  } else {
    *(uint2*)p = uint2{w[0] | w[1] << 8 | w[2] << 16 | w[3] << 24, w[4] | w[5] << 8 | w[6] << 16 | w[7] << 24};
  }
}

__device__ __forceinline__ void store_oct_any(void* out, int64_t e0, int dt, const uint32_t* v, bool is_float) {
  switch (dt) {
    case DT_F32: return store_oct<DT_F32>(out, e0, v, is_float);
    case DT_S32: return store_oct<DT_S32>(out, e0, v, is_float);
    case DT_BF16: return store_oct<DT_BF16>(out, e0, v, is_float);
    case DT_F16: return store_oct<DT_F16>(out, e0, v, is_float);
    case DT_F8E4M3FN: return store_oct<DT_F8E4M3FN>(out, e0, v, is_float);
    default:
#pragma unroll
      for (int e = 0; e < 8; ++e) store_bits(out, e0 + e, dt, v[e], is_float);
  }
}


template <bool INT, bool DUAL>
__device__ __forceinline__ void splitk_epilogue_oct(const GemmArgs& G, int64_t e0, int b, int m, int n, uint32_t (&v)[8],
                                                    const uint32_t (&v2)[8]) {
  uint32_t raw[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) raw[e] = v[e];
  bool is_float = !INT;
  if (G.epilogue == EPI_SCALE) {
    float rs = G.alpha;
    if (G.row) rs *= G.row[(int64_t)b * G.row_sb + (int64_t)m * G.row_sm];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float cs = G.col ? G.col[(int64_t)b * G.col_sb + (int64_t)(n + e) * G.col_sn] : 1.0f;
      float x = INT ? (float)(int32_t)v[e] : __uint_as_float(v[e]);
      x = x * rs * cs;
      if (G.mid_round) x = G.mid_round == DT_BF16 ? bf16_bits_to_f32(f32_to_bf16_bits(x)) : (float)(_Float16)x;
      v[e] = __float_as_uint(x);
    }
    is_float = true;
  } else if (DUAL && G.epilogue == EPI_SWIGLU) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float c1 = G.col ? G.col[(int64_t)b * G.col_sb + (int64_t)(n + e) * G.col_sn] : 1.0f;
      const float c2 = G.col2 ? G.col2[(int64_t)b * G.col2_sb + (int64_t)(n + e) * G.col2_sn] : 1.0f;
      const float a = __uint_as_float(v[e]) * c1;
      const float u = __uint_as_float(v2[e]) * c2;
      const float lg = 1.0f / (1.0f + expf(-a));
      float x = (a * lg) * u;
      if (G.mid_round) x = G.mid_round == DT_BF16 ? bf16_bits_to_f32(f32_to_bf16_bits(x)) : (float)(_Float16)x;
      v[e] = __float_as_uint(x);
    }
    is_float = true;
  }
  store_oct_any(G.out_ptr[0], e0, G.out_dtype[0], v, is_float);
  if (G.epilogue == EPI_SCALE && G.raw_out) store_oct_any(G.out_ptr[1], e0, G.out_dtype[1], raw, !INT);
}

// The K range that finishes a BM×BN tile last: sums the S ranges' partial sums in range order (the reduction
// kernel's order) and applies the epilogue, eight consecutive elements per thread and step, with the loads of
// 16 / S steps in flight together.
template <bool INT, int S, int BM, int BN, int THREADS>
__device__ __forceinline__ void splitk_finish_tile(const GemmArgs& G, int b, int m0, int n0, int tid) {
  constexpr int OCTS = BM * BN / 8, PER = OCTS / THREADS, B0 = S >= 16 ? 1 : 16 / S, BATCH = PER < B0 ? PER : B0;
  static_assert(OCTS % THREADS == 0 && PER % BATCH == 0, "finish layout");
  const int64_t slice = (int64_t)G.batch * G.M * G.N;
  const uint32_t* ws = (const uint32_t*)G.ws;
  auto add = [](uint32_t a, uint32_t x) {
    return INT ? (uint32_t)((int32_t)a + (int32_t)x) : __float_as_uint(__uint_as_float(a) + __uint_as_float(x));
  };
  for (int o0 = 0; o0 < PER; o0 += BATCH) {
    u32x4 w[BATCH][S][2];
    int64_t e0[BATCH];
#pragma unroll
    for (int q = 0; q < BATCH; ++q) {
      const int oc = tid + (o0 + q) * THREADS;
      const int r = oc / (BN / 8), c = (oc % (BN / 8)) * 8;
      e0[q] = ((int64_t)b * G.M + m0 + r) * G.N + n0 + c;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        w[q][s][0] = load_coherent16(ws + s * slice + e0[q]);
        w[q][s][1] = load_coherent16(ws + s * slice + e0[q] + 4);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int q = 0; q < BATCH; ++q)
#pragma unroll
      for (int s = 0; s < S; ++s) {
        asm volatile("" : "+v"(w[q][s][0]));
        asm volatile("" : "+v"(w[q][s][1]));
      }
#pragma unroll
    for (int q = 0; q < BATCH; ++q) {
      uint32_t v[8];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        v[4 * h] = w[q][0][h].x, v[4 * h + 1] = w[q][0][h].y, v[4 * h + 2] = w[q][0][h].z, v[4 * h + 3] = w[q][0][h].w;
      }
#pragma unroll
      for (int s = 1; s < S; ++s)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          v[4 * h] = add(v[4 * h], w[q][s][h].x), v[4 * h + 1] = add(v[4 * h + 1], w[q][s][h].y);
          v[4 * h + 2] = add(v[4 * h + 2], w[q][s][h].z), v[4 * h + 3] = add(v[4 * h + 3], w[q][s][h].w);
        }
      const int oc = tid + (o0 + q) * THREADS;
      splitk_epilogue_oct<INT, false>(G, e0[q], b, m0 + oc / (BN / 8), n0 + (oc % (BN / 8)) * 8, v, v);
    }
  }
}

// Output types each epilogue kind supports on the MFMA kernels (`raw`: the raw-accumulator second output).
__host__ __device__ inline bool mfma_mid_round_supported(int mid_round, bool raw_out) {
  return mid_round == 0 || ((mid_round == DT_BF16 || mid_round == DT_F16) && !raw_out);
}
__host__ __device__ inline bool mfma_out_supported(int dt, bool int_acc, int epilogue, bool raw) {
  if (raw) return int_acc ? dt == DT_S32 : (dt == DT_F32 || dt == DT_BF16);
  if (int_acc && epilogue == EPI_STORE) return dt == DT_S32 || dt == DT_F32;
  return dt == DT_F32 || dt == DT_BF16 || dt == DT_F16 || (!int_acc && dt == DT_F8E4M3FN);
}

// Epilogue of one staged round: dispatch (uniform) on the epilogue kind, the intermediate rounding and the output
// type to one compact pass.
template <bool INT, bool DUAL, bool MIDR, int WTN, int PITCH, int ROWS, bool EDGE>
__device__ __forceinline__ void epi_round_mr(const GemmArgs& G, int b, int m0, int n0, const uint32_t* reg,
                                             const uint32_t* reg2, int lane) {
#define RYFT_EPI(K, DT, OUT) epi_pass<K, DT, INT, MIDR, WTN, PITCH, ROWS, EDGE>(G, OUT, b, m0, n0, reg, reg2, lane)
  const int dt = G.out_dtype[0];
  if (!MIDR && G.epilogue == EPI_STORE) {
    if (INT && dt == DT_S32) RYFT_EPI(EPI_STORE, DT_S32, G.out_ptr[0]);
    else if (dt == DT_F32) RYFT_EPI(EPI_STORE, DT_F32, G.out_ptr[0]);
    else if (!INT && dt == DT_BF16) RYFT_EPI(EPI_STORE, DT_BF16, G.out_ptr[0]);
    else if (!INT && dt == DT_F16) RYFT_EPI(EPI_STORE, DT_F16, G.out_ptr[0]);
    else if (!INT && dt == DT_F8E4M3FN) RYFT_EPI(EPI_STORE, DT_F8E4M3FN, G.out_ptr[0]);
  } else if (G.epilogue == EPI_SCALE) {
    if (dt == DT_F32) RYFT_EPI(EPI_SCALE, DT_F32, G.out_ptr[0]);
    else if (dt == DT_BF16) RYFT_EPI(EPI_SCALE, DT_BF16, G.out_ptr[0]);
    else if (dt == DT_F16) RYFT_EPI(EPI_SCALE, DT_F16, G.out_ptr[0]);
    else if (!INT && dt == DT_F8E4M3FN) RYFT_EPI(EPI_SCALE, DT_F8E4M3FN, G.out_ptr[0]);
    if (!MIDR && G.raw_out) {
      const int rt = G.out_dtype[1];
      if (INT) RYFT_EPI(EPI_STORE, DT_S32, G.out_ptr[1]);
      else if (rt == DT_F32) RYFT_EPI(EPI_STORE, DT_F32, G.out_ptr[1]);
      else RYFT_EPI(EPI_STORE, DT_BF16, G.out_ptr[1]);
    }
  } else if constexpr (DUAL) {
    if (dt == DT_F32) RYFT_EPI(EPI_SWIGLU, DT_F32, G.out_ptr[0]);
    else if (dt == DT_BF16) RYFT_EPI(EPI_SWIGLU, DT_BF16, G.out_ptr[0]);
    else if (dt == DT_F16) RYFT_EPI(EPI_SWIGLU, DT_F16, G.out_ptr[0]);
    else RYFT_EPI(EPI_SWIGLU, DT_F8E4M3FN, G.out_ptr[0]);
  }
#undef RYFT_EPI
}

template <bool INT, bool DUAL, int WTN, int PITCH, int ROWS, bool EDGE>
__device__ __forceinline__ void epi_round(const GemmArgs& G, int b, int m0, int n0, const uint32_t* reg,
                                          const uint32_t* reg2, int lane) {
  if (G.mid_round) epi_round_mr<INT, DUAL, true, WTN, PITCH, ROWS, EDGE>(G, b, m0, n0, reg, reg2, lane);
  else epi_round_mr<INT, DUAL, false, WTN, PITCH, ROWS, EDGE>(G, b, m0, n0, reg, reg2, lane);
}

// EDGE: any M, N (partial tiles at the edges: bounded loads, masked stores) and any K that is a multiple of the
// 16-byte vector (the last k-tile loads zeros past K); no split-K.
template <int KIND, int BM, int BN, int BK, int WM, int WN, bool A_R, bool B_R, bool DUAL, bool EDGE>
__global__ void __launch_bounds__(64 * WM * WN) gemm_mfma_kernel(const GemmArgs G) {
  using C = MfmaCfg<KIND, BM, BN, BK, WM, WN, A_R, B_R, DUAL, EDGE>;
  using M = typename C::M;
  using Acc = typename M::Acc;
  using F = Frag<C::KPACK * C::ESIZE>;
  constexpr int ES = C::ESIZE;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // XCD-aware tile order: consecutive workgroup ids land on different XCDs (round-robin), so regroup them such that
  // each XCD owns a contiguous run of tile ids; within a batch, ids run column-major through groups of up to 8
  // tile-rows, so one XCD's run covers a compact block of tiles and each A row-panel / B column-panel is fetched
  // into that XCD's L2 by few XCDs (with a row-major order every XCD would stream every B panel).
  const int tiles_n = EDGE ? (G.N + BN - 1) / BN : G.N / BN, tiles_m = EDGE ? (G.M + BM - 1) / BM : G.M / BM;
  const int per_batch = tiles_n * tiles_m;
  const int total = per_batch * G.batch;
  // split-K: the K range is the slow index of the work order, so each XCD's run covers one K range (or a few) and
  // the tiles of that range fetch only its slices of A and B (with the range inside the XCD's run every XCD would
  // fetch the whole of A). A split finished in-kernel (small partial sums) keeps every K range of a tile on the
  // tile's XCD instead, so that the finishing range reads partial sums written on its own XCD.
  const int nsplit = G.splits > 1 ? G.splits : 1;
  int split, bid;
  if (nsplit > 1 && G.tile_counters) {
    split = (int)blockIdx.x / total;
    bid = (int)blockIdx.x % total;
    if ((total & 7) == 0) bid = (bid & 7) * (total >> 3) + (bid >> 3);
  } else {
    int work = (int)blockIdx.x;
    if (((total * nsplit) & 7) == 0) work = (work & 7) * ((total * nsplit) >> 3) + (work >> 3);
    split = nsplit > 1 ? work / total : 0;
    bid = nsplit > 1 ? work % total : work;
  }
  const int b = bid / per_batch, t = bid % per_batch;
  const int GM = tiles_m < 8 ? tiles_m : 8;
  const int first_m = (t / (GM * tiles_n)) * GM;
  const int gm = min(GM, tiles_m - first_m);  // the last group may hold fewer tile-rows
  const int tg = t - first_m * tiles_n;
  const int tm = first_m + tg % gm, tn = tg / gm;
  const int m0 = tm * BM, n0 = tn * BN;

  const char* Ab = (const char*)G.A.ptr + ((int64_t)b * G.A.sb + (int64_t)m0 * G.A.sr) * ES;
  constexpr int BES = C::BES;
  const char* Bb = (const char*)G.B.ptr + ((int64_t)b * G.B.sb + (int64_t)n0 * G.B.sr) * BES;
  const char* B2b = DUAL ? (const char*)G.B2.ptr + ((int64_t)b * G.B2.sb + (int64_t)n0 * G.B2.sr) * BES : nullptr;


  Acc acc[C::TM][C::TN];
  Acc acc2[DUAL ? C::TM : 1][DUAL ? C::TN : 1];
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j) {
      acc[i][j] = Acc{};
      if constexpr (DUAL) acc2[i][j] = Acc{};
    }

  // k-tiles of this workgroup's K range
  const int KT = EDGE ? (G.K + BK - 1) / BK : (G.splits > 1 ? G.K / BK / G.splits : G.K / BK);
  const int kt0 = split * KT;
  if constexpr (C::DMA) {
    // ---- operand tiles straight from global memory into LDS (buffer_load ... lds), NST stages
    constexpr int NW = WM * WN, NST = C::NST, RBA = C::RBA, RBB = C::RBB;
    constexpr int UA = RBA / 16, R1A = 1024 / RBA, PA = BM * RBA / 1024 / NW;  // chunks / row, rows / piece, pieces
    constexpr int BROWS = C::BTR ? BK : BN;
    constexpr int UB = RBB / 16, R1B = 1024 / RBB, PB = BROWS * RBB / 1024 / NW;
    constexpr int OPS = PA + C::NB * PB;  // DMA loads per wave per k-tile
    constexpr int BREG = C::BREG_D;
    static_assert((NW * R1A) % 16 == 0 && (NW * R1B) % (C::BTR ? 8 : 16) == 0, "piece rows must keep the swizzle");
    static_assert(OPS <= 63, "vmcnt range");
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    // per-lane source offsets of piece 0 (pieces i of a wave are i·NW·R1 rows further: a scalar offset)
    const int64_t a_rs = G.A.sr * ES;
    const int ra = wave_u * R1A + lane / UA;
    const int a_voff = (int)(ra * a_rs) + 16 * ((lane % UA) ^ swz_k128(ra));
    const int a_pstep = (int)(NW * R1A * a_rs);
    auto bsw = [&](int r) { if constexpr (C::BTR) return swz_tr<C::BLES, RBB>(r); else return swz_k128(r); };
    const int rb = wave_u * R1B + lane / UB;
    const int64_t b_rs = C::BTR ? G.B.sk * BES : G.B.sr * ES;
    const int b_voff = (int)(rb * b_rs) + 16 * ((lane % UB) ^ bsw(rb));
    const int b_pstep = (int)(NW * R1B * b_rs);
    int b2_voff = 0, b2_pstep = 0;
    if constexpr (DUAL) {
      const int64_t b2_rs = C::BTR ? G.B2.sk * BES : G.B2.sr * ES;
      b2_voff = (int)(rb * b2_rs) + 16 * ((lane % UB) ^ bsw(rb));
      b2_pstep = (int)(NW * R1B * b2_rs);
    }
    auto dma = [&](int t, int st) {
      const int64_t ko = (int64_t)(kt0 + t) * BK;
      char* sb = smem + st * C::STAGE;
      const __amdgpu_buffer_rsrc_t rsa =
          __builtin_amdgcn_make_buffer_rsrc((void*)(Ab + ko * G.A.sk * ES), (short)0, -1, 0x00020000);
      const __amdgpu_buffer_rsrc_t rsb =
          __builtin_amdgcn_make_buffer_rsrc((void*)(Bb + ko * G.B.sk * BES), (short)0, -1, 0x00020000);
#pragma unroll
      for (int i = 0; i < PA; ++i) lds_dma16(rsa, sb + (wave_u + i * NW) * 1024, a_voff, i * a_pstep);
#pragma unroll
      for (int i = 0; i < PB; ++i) lds_dma16(rsb, sb + BM * RBA + (wave_u + i * NW) * 1024, b_voff, i * b_pstep);
      if constexpr (DUAL) {
        const __amdgpu_buffer_rsrc_t rsb2 =
            __builtin_amdgcn_make_buffer_rsrc((void*)(B2b + ko * G.B2.sk * BES), (short)0, -1, 0x00020000);
#pragma unroll
        for (int i = 0; i < PB; ++i)
          lds_dma16(rsb2, sb + BM * RBA + BREG + (wave_u + i * NW) * 1024, b2_voff, i * b2_pstep);
      }
    };

    // ---- fragment read addresses (bytes from the stage base)
    constexpr int S = BK / C::MK;
    constexpr int CPL = C::KPACK * ES / 16;  // 16-byte chunks per lane per K-packed fragment (2 for fp8)
    const int half = lane >> 5, l32 = lane & 31;
    int a_rd[S][CPL];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int q = 0; q < CPL; ++q)
        a_rd[s][q] = (wm * C::WTM + l32) * RBA + 16 * ((s * 2 * CPL + half * CPL + q) ^ swz_k128(l32));
    constexpr int NBR = C::BTR ? C::TN : S * CPL;
    int b_rd[NBR];
    if constexpr (C::BTR) {
#pragma unroll
      for (int j = 0; j < C::TN; ++j) {
        if constexpr (C::BLES == 2) {
          const int kr = 8 * half + ((lane & 15) >> 2);
          const int ch = (wn * C::WTN + 32 * j) / 8 + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
          b_rd[j] = BM * RBA + kr * RBB + 16 * (ch ^ swz_tr<2, RBB>(kr)) + 8 * (lane & 1);
        } else {
          const int kr = C::KPACK * half + ((lane & 15) >> 1);
          const int ch = (wn * C::WTN + 32 * j) / 16 + ((lane >> 4) & 1);
          b_rd[j] = BM * RBA + kr * RBB + 16 * (ch ^ swz_tr<1, RBB>(kr)) + 8 * (lane & 1);
        }
      }
    } else {
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int q = 0; q < CPL; ++q)
          b_rd[s * CPL + q] = BM * RBA + (wn * C::WTN + l32) * RBA + 16 * ((s * 2 * CPL + half * CPL + q) ^ swz_k128(l32));
    }
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)smem;

    constexpr bool BWIDEN = C::BTR && C::BLES == 1 && ES == 2;
    using FT = typename F::T;
    using BF = std::conditional_t<BWIDEN, u32x2w, FT>;
    FT fa[2][C::TM];
    BF fb[2][C::TN], fb2[2][DUAL ? C::TN : 1];
    auto lfrag = [&](int st, auto sc, auto slot) {
      constexpr int SS = decltype(sc)::value, SL = decltype(slot)::value;
      const uint32_t sb = lds0 + st * C::STAGE;
      static_for<0, C::TM>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        if constexpr (CPL == 1) {
          fa[SL][i] = lds_rd128<i * 32 * RBA>(sb + a_rd[SS][0]);
        } else {
          const u32x4 lo = lds_rd128<i * 32 * RBA>(sb + a_rd[SS][0]), hi = lds_rd128<i * 32 * RBA>(sb + a_rd[SS][1]);
          fa[SL][i] = FT{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        }
      });
      static_for<0, C::TN>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        static_for<0, C::NB>([&](auto bc) {
          constexpr int bi = decltype(bc)::value;
          BF v;
          if constexpr (C::BTR) {
            constexpr int O = SS * C::MK * RBB + bi * BREG;
            const uint32_t ad = sb + b_rd[j];
            if constexpr (C::BLES == 2) {
              const u32x2v lo = lds_rd_tr16<O>(ad), hi = lds_rd_tr16<O + 4 * RBB>(ad);
              v = BF{lo.x, lo.y, hi.x, hi.y};
            } else if constexpr (BWIDEN) {
              const u32x2v a = lds_rd_tr8<O>(ad);
              v = BF{a.x, a.y};
            } else if constexpr (C::KPACK == 16) {
              const u32x2v a = lds_rd_tr8<O>(ad), b = lds_rd_tr8<O + 8 * RBB>(ad);
              v = BF{a.x, a.y, b.x, b.y};
            } else {
              const u32x2v a = lds_rd_tr8<O>(ad), b = lds_rd_tr8<O + 8 * RBB>(ad), c = lds_rd_tr8<O + 16 * RBB>(ad),
                           d = lds_rd_tr8<O + 24 * RBB>(ad);
              v = BF{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
            }
          } else {
            constexpr int O = j * 32 * RBA + bi * BREG;
            if constexpr (CPL == 1) {
              v = lds_rd128<O>(sb + b_rd[SS * CPL]);
            } else {
              const u32x4 lo = lds_rd128<O>(sb + b_rd[SS * CPL]), hi = lds_rd128<O>(sb + b_rd[SS * CPL + 1]);
              v = BF{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            }
          }
          if constexpr (bi == 0) fb[SL][j] = v;
          else fb2[SL][j] = v;
        });
      });
    };
    // LDS read instructions per k-step (the wait count that leaves the next step's reads in flight)
    constexpr int BREADS = !C::BTR ? CPL : (C::BLES == 2 ? 2 : (BWIDEN ? 1 : C::KPACK / 8));
    constexpr int NREAD = C::TM * CPL + C::TN * C::NB * BREADS;
    // (lgkmcnt counts to 15: with more reads per step the wait also covers some of the next step's reads)
    constexpr int NWAIT = NREAD < 15 ? NREAD : 15;
    // the reads into fragment slot SL are complete once at most N LDS reads are outstanding (N < 0: already waited
    // for); the slot's fragments pass through the wait
    auto wait_slot = [&](auto slot, auto n) {
      constexpr int SL = decltype(slot)::value, N = decltype(n)::value;
      if constexpr (N >= 0) lgkm_wait<N>();
#pragma unroll
      for (int i = 0; i < C::TM; ++i) after_wait(fa[SL][i]);
#pragma unroll
      for (int j = 0; j < C::TN; ++j) {
        after_wait(fb[SL][j]);
        if constexpr (DUAL) after_wait(fb2[SL][j]);
      }
    };

    // prologue: tiles 0 (and 1 with three stages) in flight, tile 0 waited for
    dma(0, 0);
    if constexpr (NST == 3) {
      if (KT > 1) {
        dma(1, 1);
        dma_barrier<OPS>();
      } else {
        dma_barrier<0>();
      }
    } else {
      dma_barrier<0>();
    }
    lfrag(0, int_c<0>{}, int_c<0>{});
    int cur = 0;
    for (int kt = 0; kt < KT; ++kt) {
      const int nxt = cur + 1 == NST ? 0 : cur + 1;
      static_for<0, S>([&](auto s) {
        constexpr int SS = decltype(s)::value;
        if constexpr (SS + 1 < S) {
          lfrag(cur, int_c<SS + 1>{}, int_c<(SS + 1) & 1>{});
          wait_slot(int_c<SS & 1>{}, int_c<NWAIT>{});
        } else {
          // tile kt + 1 complete in every wave's LDS, and every wave done reading stage cur
          if (NST == 3 && kt + 2 < KT) dma_barrier<NST == 3 ? OPS : 0>();
          else dma_barrier<0>();
          wait_slot(int_c<SS & 1>{}, int_c<-1>{});
          lfrag(nxt, int_c<0>{}, int_c<0>{});
        }
        __builtin_amdgcn_sched_barrier(0);
        typename F::T wb[C::TN], wb2[DUAL ? C::TN : 1];
#pragma unroll
        for (int j = 0; j < C::TN; ++j) {
          if constexpr (BWIDEN) {
            wb[j] = f8x8_to_bf16(fb[SS & 1][j]);
            if constexpr (DUAL) wb2[j] = f8x8_to_bf16(fb2[SS & 1][j]);
          } else {
            wb[j] = fb[SS & 1][j];
            if constexpr (DUAL) wb2[j] = fb2[SS & 1][j];
          }
        }
#pragma unroll
        for (int i = 0; i < C::TM; ++i)
#pragma unroll
          for (int j = 0; j < C::TN; ++j) {
            acc[i][j] = M::mma(wb[j], fa[SS & 1][i], acc[i][j]);
            if constexpr (DUAL) acc2[i][j] = M::mma(wb2[j], fa[SS & 1][i], acc2[i][j]);
          }
        if constexpr (SS == 0) {
          // tile kt + NST - 1 into the stage tile kt - 1 used (every wave finished reading it before the last barrier)
          const int t = kt + NST - 1;
          if (t < KT) {
            dma(t, t % NST);
            constexpr int NM = C::TM * C::TN * C::NB;
            static_for<0, (OPS < NM ? OPS : NM)>([&](auto) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
              __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read (DMA)
            });
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      });
      cur = nxt;
    }
  } else {
    // One register stage of global prefetch: tile kt + 2 is requested at the start of k-tile kt (right after tile
    // kt + 1 went from registers to LDS), so each load has a whole k-tile of MFMA work to arrive in. Two LDS stages.
    using BLoader = std::conditional_t<
        C::BTR, TileCopyLoader<C::BLES, BN, BK, C::THREADS>,
        std::conditional_t<BES != ES, TileWidenLoader<BN, BK, C::THREADS>, TileLoader<ES, BN, BK, C::THREADS, B_R>>>;
    TileLoader<ES, BM, BK, C::THREADS, A_R> la;
    BLoader lb;
    BLoader lb2;
    // edge kernels: one past the last byte of each operand their loads may read, as an address (the loads are
    // bounded to it). An operand contiguous along its rows / columns (sr == 1) is read in 16-byte vectors along them,
    // so the bound is the end of the vector holding the last element: a vector straddling the last element's byte
    // would otherwise read as zero whole. (That vector stays inside the row pitch, which the layout check keeps a
    // multiple of the vector.)
    auto op_end = [&](const GemmOperand& o, int rows, int es) -> const char* {
      const int ve = 16 / es;
      const int64_t r = o.sr == 1 ? ((int64_t)rows + ve - 1) / ve * ve : rows;
      return (const char*)o.ptr +
             ((int64_t)(G.batch - 1) * o.sb + (r - 1) * o.sr + (int64_t)(G.K - 1) * o.sk + 1) * es;
    };
    const char* const a_end = EDGE ? op_end(G.A, G.M, ES) : nullptr;
    const char* const b_end = EDGE ? op_end(G.B, G.N, BES) : nullptr;
    const char* const b2_end = EDGE && DUAL ? op_end(G.B2, G.N, BES) : nullptr;
    auto bounds = [&](const char* p, const char* end, int kvalid) {
      LoadBounds r;
      r.nrec = (int)min((int64_t)(end - p), (int64_t)0x7fffffff);
      r.kvalid = kvalid;
      return r;
    };
    auto gload = [&](int kt) {
      const int64_t ko = (int64_t)(kt0 + kt) * BK;
      const char* pa = Ab + ko * G.A.sk * ES;
      const char* pb = Bb + ko * G.B.sk * BES;
      if constexpr (EDGE) {
        const int kvalid = G.K - (int)ko;
        la.template load<true>(pa, G.A.sr, G.A.sk, tid, bounds(pa, a_end, kvalid));
        lb.template load<true>(pb, G.B.sr, G.B.sk, tid, bounds(pb, b_end, kvalid));
        if constexpr (DUAL) {
          const char* pb2 = B2b + ko * G.B2.sk * BES;
          lb2.template load<true>(pb2, G.B2.sr, G.B2.sk, tid, bounds(pb2, b2_end, kvalid));
        }
      } else {
        la.load(pa, G.A.sr, G.A.sk, tid);
        lb.load(pb, G.B.sr, G.B.sk, tid);
        if constexpr (DUAL) lb2.load(B2b + ko * G.B2.sk * BES, G.B2.sr, G.B2.sk, tid);
      }
    };
    auto lstore = [&](int buf) {
      char* s = smem + buf * C::STAGE;
      la.template store<C::LDK>(s, tid);
      constexpr int BP = C::BTR ? C::LDB : C::LDK;
      lb.template store<BP>(s + BM * C::LDK, tid);
      if constexpr (DUAL) lb2.template store<BP>(s + BM * C::LDK + C::BREG, tid);
    };

    // Fragments of MFMA k-step s live in register slot s & 1: step s + 1 is read from LDS while step s multiplies.
    constexpr int S = BK / C::MK;
    static_assert(S % 2 == 0, "k-steps per tile must be even (fragment slots alternate)");
    // f8 B in LDS for the bf16 MFMA: B fragments are kept as the raw bytes of their transposing read and widened
    // right before the MFMAs that use them, so their LDS reads stay in flight across the previous step's MFMAs
    constexpr bool BWIDEN = C::BTR && C::BLES == 1 && ES == 2;
    using BF = std::conditional_t<BWIDEN, u32x2w, typename F::T>;
    typename F::T fa[2][C::TM];
    BF fb[2][C::TN], fb2[2][DUAL ? C::TN : 1];
    const int lrow = lane & 31;
    const int lk = (lane >> 5) * C::KPACK * ES;  // byte offset of this lane's k-pack within an MFMA k-step
    const int a_off = (wm * C::WTM + lrow) * C::LDK + lk;
    // K-packed B: row n, k-pack of this lane. Transposed-read B: lane s of each 16-lane group addresses k-row
    // 8·(lane/32) + s/4 and column 16·((lane/16) % 2) + 4·(s % 4), so the pair of reads (k-rows +0 and +4) delivers
    // B[8·(lane/32) .. +7][lane % 32] — the MFMA operand fragment.
    // (8-bit: lane s addresses k-row KPACK·(lane/32) + s/2 and column 16·((lane/16) % 2) + 8·(s % 2); each read
    // delivers 8 consecutive k, KPACK / 8 reads make the fragment.)
    const int b_off = !C::BTR ? BM * C::LDK + (wn * C::WTN + lrow) * C::LDK + lk
                      : C::BLES == 2 ? BM * C::LDK + (8 * (lane >> 5) + ((lane & 15) >> 2)) * C::LDB +
                                           (wn * C::WTN + 16 * ((lane >> 4) & 1) + 4 * (lane & 3)) * 2
                                     : BM * C::LDK + (C::KPACK * (lane >> 5) + ((lane & 15) >> 1)) * C::LDB +
                                           (wn * C::WTN + 16 * ((lane >> 4) & 1) + 8 * (lane & 1));
    auto bfrag = [&](const char* p) -> BF {
      if constexpr (!C::BTR) {
        return F::load(p);
      } else if constexpr (C::BLES == 2) {
        const uint2 lo = lds_read_tr16(p), hi = lds_read_tr16(p + 4 * C::LDB);
        return u32x4{lo.x, lo.y, hi.x, hi.y};
      } else if constexpr (BWIDEN) {  // one transposing read gives the 8 k of the fragment
        const uint2 a = lds_read_tr8(p);
        return u32x2w{a.x, a.y};
      } else if constexpr (C::KPACK == 16) {
        const uint2 a = lds_read_tr8(p), b = lds_read_tr8(p + 8 * C::LDB);
        return u32x4{a.x, a.y, b.x, b.y};
      } else {
        const uint2 a = lds_read_tr8(p), b = lds_read_tr8(p + 8 * C::LDB), c = lds_read_tr8(p + 16 * C::LDB),
                    d = lds_read_tr8(p + 24 * C::LDB);
        return u32x8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
      }
    };
    auto lfrag = [&](int buf, auto s, auto slot) {
      constexpr int SL = decltype(slot)::value;
      constexpr int ko = decltype(s)::value * C::MK * ES;
      // B fragment j / k-step offset: K-packed rows are n (32 per tile) with k along the row; transposed rows are k
      constexpr int bko = C::BTR ? decltype(s)::value * C::MK * C::LDB : ko;
      constexpr int bjo = C::BTR ? 32 * C::BLES : 32 * C::LDK;
      const char* st = smem + buf * C::STAGE;
#pragma unroll
      for (int i = 0; i < C::TM; ++i) fa[SL][i] = F::load(st + a_off + i * 32 * C::LDK + ko);
#pragma unroll
      for (int j = 0; j < C::TN; ++j) {
        fb[SL][j] = bfrag(st + b_off + j * bjo + bko);
        if constexpr (DUAL) fb2[SL][j] = bfrag(st + b_off + C::BREG + j * bjo + bko);
      }
    };

    // prologue: tile 0 in LDS stage 0, tile 1 in flight in registers
    gload(0);
    lstore(0);
    gload(min(1, KT - 1));
    __syncthreads();
    lfrag(0, int_c<0>{}, int_c<0>{});

    // k-tile kt reads LDS stage kt & 1. Per k-step s: the fragments of step s + 1 are requested first and a
    // scheduling barrier keeps them ahead of the MFMAs of step s (the compiler would otherwise sink each read to just
    // before its first use and expose the LDS latency). After the MFMAs of step 0, tile kt + 1 goes from registers to
    // the other stage and tile kt + 2 is requested (past the last tile the last one is re-read: unconditional loads
    // keep the wait counters exact). The single barrier sits before the MFMAs of the last k-step: by then every wave
    // holds its last fragments of this stage and has stored tile kt + 1, so the first fragments of tile kt + 1 are read
    // while the last k-step multiplies; the barrier also orders the reads of this stage before its next overwrite.
    //
    // MFMA operands are swapped (B fragment first): each accumulator holds the transposed 32×32 tile, so a lane's
    // registers are 4 runs of 4 consecutive output columns of one row, which the epilogue writes as 16-byte words.
    for (int kt = 0; kt < KT; ++kt) {
      const int cur = kt & 1;
      static_for<0, S>([&](auto s) {
        constexpr int SS = decltype(s)::value;
        if constexpr (SS + 1 < S) {
          lfrag(cur, int_c<SS + 1>{}, int_c<(SS + 1) & 1>{});
        } else {
          __syncthreads();
          lfrag(cur ^ 1, int_c<0>{}, int_c<0>{});
        }
        __builtin_amdgcn_sched_barrier(0);
        typename F::T wb[C::TN], wb2[DUAL ? C::TN : 1];
#pragma unroll
        for (int j = 0; j < C::TN; ++j) {
          if constexpr (BWIDEN) {
            wb[j] = f8x8_to_bf16(fb[SS & 1][j]);
            if constexpr (DUAL) wb2[j] = f8x8_to_bf16(fb2[SS & 1][j]);
          } else {
            wb[j] = fb[SS & 1][j];
            if constexpr (DUAL) wb2[j] = fb2[SS & 1][j];
          }
        }
#pragma unroll
        for (int i = 0; i < C::TM; ++i)
#pragma unroll
          for (int j = 0; j < C::TN; ++j) {
            acc[i][j] = M::mma(wb[j], fa[SS & 1][i], acc[i][j]);
            if constexpr (DUAL) acc2[i][j] = M::mma(wb2[j], fa[SS & 1][i], acc2[i][j]);
          }
        // The LDS store of tile kt + 1 (step 0) and the loads of tile kt + 2 (step 1) are spread between this step's
        // MFMAs, one memory instruction per MFMA: issued as a burst they would queue in the memory pipeline and stall
        // the in-order issue of the MFMAs behind them.
        constexpr int NM = C::TM * C::TN * C::NB;
        if constexpr (SS == 0) {
          lstore(cur ^ 1);
          static_for<0, NM>([&](auto) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU (transposes, addresses)
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
          });
        }
        if constexpr (SS == (S > 2 ? 1 : 0)) {
          gload(min(kt + 2, KT - 1));
          static_for<0, NM>([&](auto) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load
          });
        }
        __builtin_amdgcn_sched_barrier(0);
      });
    }

  }  // main loop

  // Epilogue. With the swapped operands, register r of lane l holds C[l%32][8·(r/4) + 4·(l/32) + r%4] of its
  // 32×32 tile: registers 4g..4g+3 are 4 consecutive columns of one row. Each wave stages its accumulators in its own
  // LDS region, in rounds of EPI_ROWS tile-rows (compile-time indices keep them in registers until then), with one
  // 16-byte write per run; a short loop specialised for the epilogue kind and output type then hands each lane 16-byte output
  // chunks in row order, so global stores are contiguous.
  __syncthreads();  // the main loop's last fragment reads of the LDS stages are complete in every wave
  constexpr int PITCH = C::WTN + 4;  // words per LDS row (16-byte pad against bank conflicts)
  constexpr int EPI_ROWS = C::EPI_ROWS;
  constexpr int REGION = EPI_ROWS * 32 * PITCH;
  uint32_t* patch = (uint32_t*)smem + wave * C::NB * REGION;
  static_for<0, C::TM / EPI_ROWS>([&](auto rd) {
    constexpr int round = decltype(rd)::value;
    static_for<0, EPI_ROWS * C::TN>([&](auto t) {
      constexpr int il = decltype(t)::value / C::TN, j = decltype(t)::value % C::TN;
      constexpr int i = round * EPI_ROWS + il;
      const int row = il * 32 + (lane & 31);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int col = j * 32 + 8 * g + 4 * (lane >> 5);
        // (element reads through the vector subscript, then a value conversion: a bit-cast of the subscript
        //  expression was lowered to element 0 for every r)
        *(u32x4*)(patch + row * PITCH + col) =
            u32x4{acc_elem_bits(acc[i][j], 4 * g), acc_elem_bits(acc[i][j], 4 * g + 1),
                  acc_elem_bits(acc[i][j], 4 * g + 2), acc_elem_bits(acc[i][j], 4 * g + 3)};
        if constexpr (DUAL)
          *(u32x4*)(patch + REGION + row * PITCH + col) =
              u32x4{acc_elem_bits(acc2[i][j], 4 * g), acc_elem_bits(acc2[i][j], 4 * g + 1),
                    acc_elem_bits(acc2[i][j], 4 * g + 2), acc_elem_bits(acc2[i][j], 4 * g + 3)};
      }
    });
    // The region is private to this wave, and one wave's LDS operations execute in order: keeping the compiler from
    // moving the reads above the writes is all the ordering needed (a memory fence would also wait for the stores).
    __asm__ __volatile__("" ::: "memory");
    const int em0 = m0 + wm * C::WTM + round * EPI_ROWS * 32, en0 = n0 + wn * C::WTN;
    if (G.splits > 1) {  // raw partial sums of this K range
      constexpr int PDT = M::INT ? DT_S32 : DT_F32;
      const int64_t slice = (int64_t)G.batch * G.M * G.N * 4;
      char* ws = (char*)G.ws + (int64_t)split * C::NB * slice;
      if (G.tile_counters) {  // read back by the range that finishes the tile: device-scope stores
        epi_pass<EPI_STORE, PDT, M::INT, false, C::WTN, PITCH, EPI_ROWS * 32, false, true>(G, ws, b, em0, en0, patch,
                                                                                          nullptr, lane);
      } else {
        epi_pass<EPI_STORE, PDT, M::INT, false, C::WTN, PITCH, EPI_ROWS * 32>(G, ws, b, em0, en0, patch, nullptr, lane);
        if constexpr (DUAL)
          epi_pass<EPI_STORE, PDT, M::INT, false, C::WTN, PITCH, EPI_ROWS * 32>(G, ws + slice, b, em0, en0,
                                                                               patch + REGION, nullptr, lane);
      }
    } else {
      epi_round<M::INT, DUAL, C::WTN, PITCH, EPI_ROWS * 32, EDGE>(G, b, em0, en0, patch, patch + REGION, lane);
    }
    if constexpr (round + 1 < C::TM / EPI_ROWS) __asm__ __volatile__("" ::: "memory");  // reads before next writes
  });

  // Split-K with arrival counters: once every thread's partial stores are complete at device scope, the workgroup
  // counts its arrival at the tile; the last of the S ranges to arrive sums them all and applies the epilogue. No
  // workgroup waits for another, and no cache is flushed or invalidated (the partials are written and read at
  // device scope); the counter is back at zero when the launch ends.
  if constexpr (!EDGE && !DUAL) {
    if (G.splits > 1 && G.tile_counters) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      int* last = (int*)smem;
      if (tid == 0) {
        int32_t* cnt = G.tile_counters + ((int64_t)b * tiles_m + tm) * tiles_n + tn;
        const int arrived = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
        if (arrived == G.splits) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *last = arrived == G.splits;
      }
      __syncthreads();
      if (*(volatile int*)last) {
        switch (G.splits) {
          case 2: splitk_finish_tile<M::INT, 2, BM, BN, C::THREADS>(G, b, m0, n0, tid); break;
          case 4: splitk_finish_tile<M::INT, 4, BM, BN, C::THREADS>(G, b, m0, n0, tid); break;
          case 8: splitk_finish_tile<M::INT, 8, BM, BN, C::THREADS>(G, b, m0, n0, tid); break;
          case 16: splitk_finish_tile<M::INT, 16, BM, BN, C::THREADS>(G, b, m0, n0, tid); break;
        }
      }
    }
  }
}


// ------------------------------------------------------------------------------------------------ dispatch
struct Choice {
  const void* fn = nullptr;
  int threads = 256;
  int lds = 0;
  int bm = 0, bn = 0, bk = 0;
  bool edge = false;  // partial tiles allowed (grid rounds up)
  const char* name = "gemm_generic";
};

template <int KIND, int BM, int BN, int BK, int WM, int WN, bool A_R, bool B_R, bool DUAL, bool EDGE = false>
Choice make_choice(const char* name) {
  using C = MfmaCfg<KIND, BM, BN, BK, WM, WN, A_R, B_R, DUAL, EDGE>;
  Choice c;
  c.fn = (const void*)&gemm_mfma_kernel<KIND, BM, BN, BK, WM, WN, A_R, B_R, DUAL, EDGE>;
  c.edge = EDGE;
  c.threads = C::THREADS;
  c.lds = C::LDS_BYTES;
  c.bm = BM;
  c.bn = BN;
  c.bk = BK;
  c.name = name;
  return c;
}

// The edge instantiation of a tile for either layout of A (ar: m-contiguous) and B (br: n-contiguous).
template <int KIND, int BM, int BN, int BK, int WM, int WN, bool DUAL>
Choice edge_choice(bool ar, bool br, const char* name) {
  if (ar) return br ? make_choice<KIND, BM, BN, BK, WM, WN, true, true, DUAL, true>(name)
                    : make_choice<KIND, BM, BN, BK, WM, WN, true, false, DUAL, true>(name);
  return br ? make_choice<KIND, BM, BN, BK, WM, WN, false, true, DUAL, true>(name)
            : make_choice<KIND, BM, BN, BK, WM, WN, false, false, DUAL, true>(name);
}

// Per-type instantiation pickers (one translation unit each, so the build parallelises). `ar`: A is m-contiguous,
// `br`: B is n-contiguous. Tile-multiple shapes with a K-contiguous A get the full-tile kernels; any other shape (and
// an m-contiguous A) gets the edge kernel of a 128×128 tile (64×64 for f32). With g.splits > 1 a picker returns the
// tile it runs over each of the K ranges, or false (split-K runs full tiles only).
bool pick_bf16(const GemmArgs& g, bool ar, bool br, Choice* c);
bool pick_f16(const GemmArgs& g, bool ar, bool br, Choice* c);
bool pick_i8(const GemmArgs& g, bool ar, bool br, Choice* c);
bool pick_fp8(const GemmArgs& g, bool ar, bool br, Choice* c);
bool pick_f32(const GemmArgs& g, bool ar, bool br, Choice* c);
bool pick_bf16f8(const GemmArgs& g, bool ar, bool br, Choice* c);

}  // namespace ryft
