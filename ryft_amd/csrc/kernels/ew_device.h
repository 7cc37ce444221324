// Device-side helpers: typed loads/stores with StableHLO rounding rules, and the elementwise program interpreter
// shared by the elementwise, reduction-prologue and GEMM-epilogue kernels.
#pragma once

#include <hip/hip_runtime.h>

#include "../kernel_abi.h"

namespace ryft {

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));


// DType values (PJRT_Buffer_Type numbering; kept literal so kernels do not include the C API header).
enum : int {
  DT_PRED = 1, DT_S8 = 2, DT_S16 = 3, DT_S32 = 4, DT_S64 = 5, DT_U8 = 6, DT_U16 = 7, DT_U32 = 8, DT_U64 = 9,
  DT_F16 = 10, DT_F32 = 11, DT_F64 = 12, DT_BF16 = 13, DT_F8E5M2 = 16, DT_F8E4M3FN = 17,
};

__device__ __forceinline__ bool dt_is_float(int t) {
  return t == DT_F32 || t == DT_BF16 || t == DT_F16 || t == DT_F8E4M3FN || t == DT_F8E5M2 || t == DT_F64;
}

// ---- bit-exact conversions (round to nearest even; f8E4M3FN overflow → NaN, f8E5M2 overflow → inf)
// f32 → bf16 with v_cvt_pk_bf16_f32: round to nearest even, and a NaN keeps its sign and high payload bits with the
// quiet bit set ((bits >> 16) | 0x40) — the same bits as the integer formulation, checked over 2^20 random and
// special patterns on gfx950.
typedef __bf16 ew_bf16x2 __attribute__((ext_vector_type(2)));
typedef float ew_f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(ew_f32x2{lo, hi}, ew_bf16x2));
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) { return (uint16_t)f32x2_to_bf16x2_bits(f, 0.0f); }
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// f32 → f8E4M3FN with v_cvt_pk_fp8_f32: round to nearest even, subnormals on the 2^-9 grid, |x| ≥ 464 → NaN — the
// integer rule's bits on 2^20 random and special patterns on gfx950, except that the instruction writes every NaN
// input as 0xff; a NaN input keeps its sign here (0x7f / 0xff).
__device__ __forceinline__ uint8_t f32_to_e4m3fn_bits(float f) {
  uint32_t code = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(f, 0.0f, 0, false) & 0xffu;
  if (f != f) code = ((__float_as_uint(f) >> 24) & 0x80u) | 0x7fu;
  return (uint8_t)code;
}
// Four floats → four f8E4M3FN bytes (a, b, c, d from the low byte up): two v_cvt_pk_fp8_f32, each converting a pair.
// Only NaN inputs need more (their sign back), and the instruction writes those as 0xff: a word with no byte of 0x7f
// or 0xff (one zero-byte test on the low seven bits of each byte) is final, any other takes the per-element rule.
__device__ __forceinline__ uint32_t f32x4_to_e4m3fn_bits(float a, float b, float c, float d) {
  uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, (int)w, true);
  const uint32_t t = ~w & 0x7f7f7f7fu;
  if ((t - 0x01010101u) & ~t & 0x80808080u)
    w = (uint32_t)f32_to_e4m3fn_bits(a) | ((uint32_t)f32_to_e4m3fn_bits(b) << 8) |
        ((uint32_t)f32_to_e4m3fn_bits(c) << 16) | ((uint32_t)f32_to_e4m3fn_bits(d) << 24);
  return w;
}
__device__ __forceinline__ float e4m3fn_bits_to_f32(uint32_t v) {
  uint32_t s = (v & 0x80u) << 24, e = (v >> 3) & 15u, m = v & 7u;
  float r;
  if (e == 0) r = (float)m * 0.001953125f;  // 2^-9
  else r = __uint_as_float(((e + 120u) << 23) | (m << 20));
  if ((v & 0x7fu) == 0x7fu) r = __uint_as_float(0x7fc00000u);
  return __uint_as_float(__float_as_uint(r) | s);
}
__device__ __forceinline__ uint8_t f32_to_e5m2_bits(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint8_t)(sign | 0x7fu);
  if (a == 0x7f800000u) return (uint8_t)(sign | 0x7cu);
  uint32_t code;
  if (a < 0x38800000u) {  // |x| < 2^-14: subnormal grid of 2^-16
    code = (uint32_t)rintf(__uint_as_float(a) * 65536.0f);
  } else {
    uint32_t r = (a + 0xfffffu + ((a >> 21) & 1u)) >> 21;
    code = r - ((127u - 15u) << 2);
    if (code > 0x7bu) code = 0x7cu;
  }
  return (uint8_t)(sign | code);
}
__device__ __forceinline__ float e5m2_bits_to_f32(uint32_t v) {
  uint32_t s = (v & 0x80u) << 24, e = (v >> 2) & 31u, m = v & 3u;
  float r;
  if (e == 0) r = (float)m * 1.52587890625e-05f;  // 2^-16
  else if (e == 31) r = m ? __uint_as_float(0x7fc00000u) : __uint_as_float(0x7f800000u);
  else r = __uint_as_float(((e + 112u) << 23) | (m << 21));
  return __uint_as_float(__float_as_uint(r) | s);
}

// Round a float register to the precision of `dtype` (no-op for f32).
__device__ __forceinline__ float round_float(float v, int dtype) {
  switch (dtype) {
    case DT_BF16: return bf16_bits_to_f32(f32_to_bf16_bits(v));
    case DT_F16: return (float)(_Float16)v;
    case DT_F8E4M3FN: return e4m3fn_bits_to_f32(f32_to_e4m3fn_bits(v));
    case DT_F8E5M2: return e5m2_bits_to_f32(f32_to_e5m2_bits(v));
    default: return v;
  }
}
// Wrap an int32 register to the width of `dtype`.
__device__ __forceinline__ int32_t wrap_int(int32_t v, int dtype) {
  switch (dtype) {
    case DT_S8: return (int32_t)(int8_t)v;
    case DT_S16: return (int32_t)(int16_t)v;
    case DT_U8: return (int32_t)(uint8_t)v;
    case DT_U16: return (int32_t)(uint16_t)v;
    case DT_PRED: return v != 0;
    default: return v;
  }
}

// Load one element as a 32-bit register value: floats as f32 bits, integers as int32 (sign/zero extended).
__device__ __forceinline__ uint32_t load_bits(const void* p, int64_t i, int dtype) {
  switch (dtype) {
    case DT_F32: case DT_S32: case DT_U32: return ((const uint32_t*)p)[i];
    case DT_BF16: return (uint32_t)((const uint16_t*)p)[i] << 16;
    case DT_F16: return __float_as_uint((float)((const _Float16*)p)[i]);
    case DT_F8E4M3FN: return __float_as_uint(e4m3fn_bits_to_f32(((const uint8_t*)p)[i]));
    case DT_F8E5M2: return __float_as_uint(e5m2_bits_to_f32(((const uint8_t*)p)[i]));
    case DT_F64: return __float_as_uint((float)((const double*)p)[i]);
    case DT_S8: return (uint32_t)(int32_t)((const int8_t*)p)[i];
    case DT_U8: case DT_PRED: return (uint32_t)((const uint8_t*)p)[i];
    case DT_S16: return (uint32_t)(int32_t)((const int16_t*)p)[i];
    case DT_U16: return (uint32_t)((const uint16_t*)p)[i];
    case DT_S64: case DT_U64: return (uint32_t)((const int64_t*)p)[i];
    default: return 0;
  }
}
__device__ __forceinline__ float load_float(const void* p, int64_t i, int dtype) {
  uint32_t b = load_bits(p, i, dtype);
  return dt_is_float(dtype) ? __uint_as_float(b) : (float)(int32_t)b;
}

// Store a register value (float bits if `is_float`, else int32) as `dtype`.
__device__ __forceinline__ void store_bits(void* p, int64_t i, int dtype, uint32_t bits, bool is_float) {
  switch (dtype) {
    case DT_F32: ((float*)p)[i] = is_float ? __uint_as_float(bits) : (float)(int32_t)bits; break;
    case DT_BF16: ((uint16_t*)p)[i] = f32_to_bf16_bits(is_float ? __uint_as_float(bits) : (float)(int32_t)bits); break;
    case DT_F16: ((_Float16*)p)[i] = (_Float16)(is_float ? __uint_as_float(bits) : (float)(int32_t)bits); break;
    case DT_F8E4M3FN: ((uint8_t*)p)[i] = f32_to_e4m3fn_bits(is_float ? __uint_as_float(bits) : (float)(int32_t)bits); break;
    case DT_F8E5M2: ((uint8_t*)p)[i] = f32_to_e5m2_bits(is_float ? __uint_as_float(bits) : (float)(int32_t)bits); break;
    case DT_F64: ((double*)p)[i] = is_float ? (double)__uint_as_float(bits) : (double)(int32_t)bits; break;
    case DT_S32: case DT_U32: ((uint32_t*)p)[i] = bits; break;
    case DT_S8: case DT_U8: ((uint8_t*)p)[i] = (uint8_t)bits; break;
    case DT_PRED: ((uint8_t*)p)[i] = bits != 0; break;
    case DT_S16: case DT_U16: ((uint16_t*)p)[i] = (uint16_t)bits; break;
    case DT_S64: ((int64_t*)p)[i] = (int64_t)(int32_t)bits; break;
    case DT_U64: ((uint64_t*)p)[i] = (uint64_t)bits; break;
    default: break;
  }
}

__device__ __forceinline__ bool cmp_f(float x, float y, int dir) {
  switch (dir) {
    case 0: return x == y;
    case 1: return x != y;
    case 2: return x >= y;
    case 3: return x > y;
    case 4: return x <= y;
    default: return x < y;
  }
}
template <typename T>
__device__ __forceinline__ bool cmp_i(T x, T y, int dir) {
  switch (dir) {
    case 0: return x == y;
    case 1: return x != y;
    case 2: return x >= y;
    case 3: return x > y;
    case 4: return x <= y;
    default: return x < y;
  }
}

// The low `w` bits (w in 1..32).
__device__ __forceinline__ uint32_t width_mask(int w) { return w >= 32 ? 0xffffffffu : (1u << w) - 1u; }
// The low `w` bits read as a w-bit two's complement integer.
__device__ __forceinline__ int32_t sign_extend(uint32_t v, int w) {
  return w >= 32 ? (int32_t)v : (int32_t)(v << (32 - w)) >> (32 - w);
}

// bitcast_convert of one element between types of one width: the register form of `from` → the element's raw bits
// → the register form of `to` (floats as f32 values, bf16 as its bits in the high half, integers sign- or
// zero-extended).
__device__ __noinline__ uint32_t bitcast_reg(uint32_t r, int from, int to) {
  uint32_t bits;
  switch (from) {
    case DT_BF16: bits = r >> 16; break;
    case DT_F16: bits = __builtin_bit_cast(uint16_t, (_Float16)__uint_as_float(r)); break;
    case DT_F8E4M3FN: bits = f32_to_e4m3fn_bits(__uint_as_float(r)); break;
    case DT_F8E5M2: bits = f32_to_e5m2_bits(__uint_as_float(r)); break;
    case DT_S8: case DT_U8: bits = r & 0xffu; break;
    case DT_S16: case DT_U16: bits = r & 0xffffu; break;
    default: bits = r; break;  // 32-bit types
  }
  switch (to) {
    case DT_BF16: return bits << 16;
    case DT_F16: return __float_as_uint((float)__builtin_bit_cast(_Float16, (uint16_t)bits));
    case DT_F8E4M3FN: return __float_as_uint(e4m3fn_bits_to_f32(bits));
    case DT_F8E5M2: return __float_as_uint(e5m2_bits_to_f32(bits));
    case DT_S8: return (uint32_t)(int32_t)(int8_t)bits;
    case DT_S16: return (uint32_t)(int32_t)(int16_t)bits;
    default: return bits;  // 32-bit types, u8, u16
  }
}

// reduce_precision (casting.rs:259-300) of one element of type dt (f32, bf16 or f16; register form: an f32 value), on
// the element's own bits as XLA's emitter does: the mantissa rounded to m bits (ties to even; a carry moves into the
// exponent), then values whose exponent the e-bit format cannot hold overflow to ±inf or underflow to ±0 (the
// reduced format's subnormals included); a NaN comes back unchanged.
__device__ __noinline__ uint32_t reduce_precision_reg(uint32_t r, int dt, int e, int m) {
  const float v = __uint_as_float(r);
  if (v != v) return r;
  const int sm = dt == DT_BF16 ? 7 : (dt == DT_F16 ? 10 : 23), se = dt == DT_F16 ? 5 : 8;
  uint32_t x = dt == DT_BF16 ? r >> 16 : (dt == DT_F16 ? (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v) : r);
  if (m < sm) {
    const int shift = sm - m;
    const uint32_t last = 1u << shift;
    x = (x + ((x & last) >> shift) + ((last >> 1) - 1)) & ~(last - 1);
  }
  if (e < se) {
    const uint32_t exp_mask = ((1u << se) - 1) << sm, sign = 1u << (sm + se);
    const int bias = (1 << (se - 1)) - 1, rbias = (1 << (e - 1)) - 1;
    const uint32_t xe = x & exp_mask;
    if (xe > ((uint32_t)(bias + rbias) << sm)) x = (x & sign) | exp_mask;
    else if (xe <= ((uint32_t)(bias - rbias) << sm)) x = x & sign;
  }
  if (dt == DT_BF16) return x << 16;
  if (dt == DT_F16) return __float_as_uint((float)__builtin_bit_cast(_Float16, (uint16_t)x));
  return x;
}

__device__ __forceinline__ float f_logistic(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Saturating float → int conversion (NaN → 0), truncating toward zero.
__device__ __forceinline__ int32_t f2i_sat(float x, int dtype) {
  if (x != x) return 0;
  float lo, hi;
  switch (dtype) {
    case DT_S8: lo = -128.f; hi = 127.f; break;
    case DT_U8: lo = 0.f; hi = 255.f; break;
    case DT_S16: lo = -32768.f; hi = 32767.f; break;
    case DT_U16: lo = 0.f; hi = 65535.f; break;
    default: lo = -2147483648.f; hi = 2147483520.f; break;
  }
  x = fminf(fmaxf(x, lo), hi);
  return (int32_t)x;
}

// Offset of leaf `L` at the given iteration coordinates / linear index.
__device__ __forceinline__ int64_t leaf_offset(const EwLeaf& L, int64_t lin, const int32_t* coord, int rank) {
  if (L.kind == EW_LEAF_IDENTITY) return L.offset + lin;
  if (L.kind == EW_LEAF_SCALAR) return L.offset;
  int64_t off = L.offset;
#pragma unroll
  for (int d = 0; d < EW_MAX_RANK; ++d)  // constant indices: the leaf and coordinates stay in registers
    if (d < rank) off += (int64_t)coord[d] * L.strides[d];
  return off;
}

__device__ __forceinline__ void decompose(int64_t lin, const EwProgram& P, int32_t* coord) {
  for (int d = P.rank - 1; d >= 0; --d) {
    int64_t s = P.shape[d];
    coord[d] = (int32_t)(lin % s);
    lin /= s;
  }
}

// B bytes (4, 8, 16 or 32; B-aligned) into the first B/4 words of w.
template <int B>
__device__ __forceinline__ void load_words(const char* p, uint32_t* w) {
  if constexpr (B >= 16) {
#pragma unroll
    for (int q = 0; q < B / 16; ++q) {
      const u32x4v a = *(const u32x4v*)(p + 16 * q);
      w[4 * q] = a.x, w[4 * q + 1] = a.y, w[4 * q + 2] = a.z, w[4 * q + 3] = a.w;
    }
  } else if constexpr (B == 8) {
    const u32x2v a = *(const u32x2v*)p;
    w[0] = a.x, w[1] = a.y;
  } else {
    w[0] = *(const uint32_t*)p;
  }
}

// Raw words of V contiguous elements of a leaf starting at element `off` (V·size bytes, V·size-aligned): the first
// V·size/4 words of w.
template <int V>
__device__ __forceinline__ void fetch_contig(const EwLeaf& L, int64_t off, uint32_t* w) {
  static_assert(V == 4 || V == 8, "vector leaf loads are written for 4 or 8 elements");
  const char* p = (const char*)L.ptr;
  switch (L.dtype) {
    case DT_F32: case DT_S32: case DT_U32: load_words<V * 4>(p + off * 4, w); break;
    case DT_BF16: case DT_F16: case DT_S16: case DT_U16: load_words<V * 2>(p + off * 2, w); break;
    default: load_words<V>(p + off, w); break;
  }
}

// V register values (f32 bits / int32) from the raw words fetch_contig returned: one switch on the element type,
// then straight-line decoding of the V elements (no per-element branches).
template <int V>
__device__ __forceinline__ void decode_contig(int dtype, const uint32_t* w, uint32_t* r) {
  switch (dtype) {
    case DT_F32: case DT_S32: case DT_U32:
#pragma unroll
      for (int e = 0; e < V; ++e) r[e] = w[e];
      break;
    case DT_BF16:
#pragma unroll
      for (int e = 0; e < V; ++e) r[e] = (e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16);
      break;
    case DT_F16:
#pragma unroll
      for (int e = 0; e < V; ++e)
        r[e] = __float_as_uint((float)__builtin_bit_cast(_Float16, (uint16_t)(w[e >> 1] >> (16 * (e & 1)))));
      break;
    case DT_S16:
#pragma unroll
      for (int e = 0; e < V; ++e) r[e] = (uint32_t)(int32_t)(int16_t)(w[e >> 1] >> (16 * (e & 1)));
      break;
    case DT_U16:
#pragma unroll
      for (int e = 0; e < V; ++e) r[e] = (w[e >> 1] >> (16 * (e & 1))) & 0xffffu;
      break;
    case DT_F8E4M3FN:
#pragma unroll
      for (int e = 0; e < V; ++e) r[e] = __float_as_uint(e4m3fn_bits_to_f32((w[e >> 2] >> (8 * (e & 3))) & 0xffu));
      break;
    case DT_F8E5M2:
#pragma unroll
      for (int e = 0; e < V; ++e) r[e] = __float_as_uint(e5m2_bits_to_f32((w[e >> 2] >> (8 * (e & 3))) & 0xffu));
      break;
    case DT_S8:
#pragma unroll
      for (int e = 0; e < V; ++e) r[e] = (uint32_t)(int32_t)(int8_t)(w[e >> 2] >> (8 * (e & 3)));
      break;
    default:  // u8, pred
#pragma unroll
      for (int e = 0; e < V; ++e) r[e] = (w[e >> 2] >> (8 * (e & 3))) & 0xffu;
      break;
  }
}

// Element bits of a leaf at V consecutive innermost positions starting at linear index `lin` (coordinates `coord`).
template <int V>
__device__ __forceinline__ void load_leaf(const EwLeaf& L, int64_t lin, const int32_t* coord, int rank, uint32_t* r) {
  const int64_t off = leaf_offset(L, lin, coord, rank);
  if constexpr (V == 1) {
    r[0] = load_bits(L.ptr, off, L.dtype);
  } else {
    if (L.vmode == EW_VEC_BCAST) {
      const uint32_t x = load_bits(L.ptr, off, L.dtype);
#pragma unroll
      for (int e = 0; e < V; ++e) r[e] = x;
    } else if (L.vmode == EW_VEC_CONTIG) {
      // V elements of ≤ 4 bytes, aligned to V·size (checked by the launcher)
      uint32_t w[V];
      fetch_contig<V>(L, off, w);
      decode_contig<V>(L.dtype, w, r);
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e) r[e] = load_bits(L.ptr, off + (int64_t)e * L.vstride, L.dtype);
    }
  }
}

// Register files of the VM. Operands are moved as whole rows of V elements.
//  * RegFile1: one element per thread in a VGPR array (indexed with the uniform register number: indirect moves).
//  * SwitchRegFile<V, NR>: V elements per thread in NR (≤ twelve) named VGPR rows picked by a uniform switch (a
//    V-wide array indexed with the register number would be placed in private memory, turning every operand into a
//    scratch round trip). Programs that use only the first NR registers run with the smaller file, which leaves VGPRs
//    for more waves per SIMD.
struct RegFile1 {
  uint32_t v[EW_MAX_REGS];
  __device__ __forceinline__ void load(int r, uint32_t* out) const { out[0] = v[r]; }
  __device__ __forceinline__ void store(int r, const uint32_t* in) { v[r] = in[0]; }
  __device__ __forceinline__ uint32_t get(int r) const { return v[r]; }
};

template <int V, int NR = EW_MAX_REGS>
struct SwitchRegFile {
  // twelve named rows held as vector values and selected by a uniform switch: the merged switch arms become phis of
  // values, which stay in VGPRs (rows kept as arrays would be merged into a phi of pointers and spilled to private
  // memory)
  static_assert(EW_MAX_REGS == 12 && NR >= 1 && NR <= 12, "SwitchRegFile names up to twelve registers");
  typedef uint32_t row_t __attribute__((ext_vector_type(V)));
  row_t r0, r1, r2, r3, r4, r5, r6, r7, r8, r9, r10, r11;
#define RF_ROWS(X) X(0) X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8) X(9) X(10) X(11)
  __device__ __forceinline__ void load(int r, uint32_t* out) const {
    row_t v = r0;
    switch (r) {
#define RF_LOAD(i) case i: if constexpr (i < NR) v = r##i; break;
      RF_ROWS(RF_LOAD)
#undef RF_LOAD
      default: break;
    }
#pragma unroll
    for (int e = 0; e < V; ++e) out[e] = v[e];
  }
  __device__ __forceinline__ void store(int r, const uint32_t* in) {
    row_t v;
#pragma unroll
    for (int e = 0; e < V; ++e) v[e] = in[e];
    switch (r) {
#define RF_STORE(i) case i: if constexpr (i < NR) r##i = v; break;
      RF_ROWS(RF_STORE)
#undef RF_STORE
      default: break;
    }
  }
#undef RF_ROWS
};

// Number of register operands an instruction reads.
__host__ __device__ __forceinline__ int ew_nsrc(int op) {
  if (op == EW_LOAD || op == EW_CONST || op == EW_IOTA || op == EW_ACC) return 0;
  if (op == EW_SELECT || op == EW_FCLAMP || op == EW_ICLAMP) return 3;
  if (op >= EW_ADD) return 2;
  return 1;
}

// Operations with long instruction sequences, evaluated one element at a time from a single copy of their code (the
// interpreter's other operations are unrolled over its V elements).
__device__ __noinline__ uint32_t ew_heavy(int op, uint32_t a, uint32_t b, int round) {
  const float fa = __uint_as_float(a), fb = __uint_as_float(b);
  const int32_t ia = (int32_t)a, ib = (int32_t)b;
  switch (op) {
    case EW_LOG: return __float_as_uint(logf(fa));
    case EW_TANH: return __float_as_uint(tanhf(fa));
    case EW_EXPM1: return __float_as_uint(expm1f(fa));
    case EW_LOG1P: return __float_as_uint(log1pf(fa));
    case EW_SIN: return __float_as_uint(sinf(fa));
    case EW_COS: return __float_as_uint(cosf(fa));
    case EW_TAN: return __float_as_uint(tanf(fa));
    case EW_CBRT: return __float_as_uint(cbrtf(fa));
    case EW_ATAN2: return __float_as_uint(atan2f(fa, fb));
    case EW_CVT_F2I: return (uint32_t)f2i_sat(fa, round);
    case EW_POW: return __float_as_uint(powf(fa, fb));
    case EW_REM: return __float_as_uint(fmodf(fa, fb));
    case EW_IDIV: return (uint32_t)(ib == 0 ? -1 : (ia == (int32_t)0x80000000 && ib == -1) ? ia : ia / ib);
    case EW_IREM: return (uint32_t)(ib == 0 ? ia : (ib == -1 ? 0 : ia % ib));
    case EW_UDIV: return b == 0 ? 0xffffffffu : a / b;
    case EW_UREM: return b == 0 ? a : a % b;
    default: return 0u;
  }
}

// Runs the program on V consecutive elements of the innermost dimension (linear indices lin .. lin+V-1, all in one
// innermost row; `coord` are the coordinates of `lin`). `acc` holds the GEMM accumulators (bits) for EW_ACC (V = 1
// only unless the values are row-uniform). Instructions [pc_begin, pc_end) run (pc_end < 0: to the end). Results
// land in the register file R. The instruction dispatch is uniform across the wave, so its cost is
// paid once per V elements.
// The instruction and leaf tables of a program staged in LDS by the kernels that interpret it many times: a
// uniform LDS read (then readfirstlane into scalar registers) per instruction instead of a scalar load from the
// kernel-argument segment, whose latency the interpreter's dependent dispatch chain cannot hide.
struct EwTables {
  EwInstr instr[EW_MAX_INSTR];
  EwLeaf leaves[EW_MAX_LEAVES];
};

// Copies P's tables into `T` (LDS); every thread of the workgroup takes part, the caller synchronises.
__device__ __forceinline__ void stage_tables(const EwProgram& P, EwTables* T) {
  static_assert(sizeof(EwInstr) % 4 == 0 && sizeof(EwLeaf) % 4 == 0, "tables are copied as 32-bit words");
  const uint32_t* si = (const uint32_t*)P.instr;
  uint32_t* di = (uint32_t*)T->instr;
  const int ni = P.n_instr * (int)(sizeof(EwInstr) / 4);
  for (int i = threadIdx.x; i < ni; i += blockDim.x) di[i] = si[i];
  const uint32_t* sl = (const uint32_t*)P.leaves;
  uint32_t* dl = (uint32_t*)T->leaves;
  const int nl = P.n_leaves * (int)(sizeof(EwLeaf) / 4);
  for (int i = threadIdx.x; i < nl; i += blockDim.x) dl[i] = sl[i];
}

template <typename T>
__device__ __forceinline__ T uniform_read(const T* p) {
  static_assert(sizeof(T) % 4 == 0, "uniform reads move 32-bit words");
  struct W { uint32_t w[sizeof(T) / 4]; } v;
  const uint32_t* s = (const uint32_t*)p;
#pragma unroll
  for (int i = 0; i < (int)(sizeof(T) / 4); ++i) v.w[i] = __builtin_amdgcn_readfirstlane(s[i]);
  return __builtin_bit_cast(T, v);
}

// Ops evaluated out of line (ew_heavy).
__host__ __device__ inline bool ew_is_heavy(int op) {
  switch (op) {
    case EW_LOG: case EW_TANH: case EW_EXPM1: case EW_LOG1P: case EW_CVT_F2I: case EW_POW: case EW_REM:
    case EW_IDIV: case EW_IREM: case EW_UDIV: case EW_UREM: case EW_SIN: case EW_COS: case EW_TAN: case EW_CBRT:
    case EW_ATAN2: case EW_BITCAST: case EW_REDPREC:
      return true;
    default:
      return false;
  }
}

// PRE: the program's leaves (at most two, contiguous) were fetched ahead by the caller as raw words (fetch_contig),
// at acc[leaf · V ..]; EW_LOAD decodes them instead of reading memory (streaming kernels issue several chunks' loads
// before computing any of them).
template <int V, typename RF, bool PRE = false>
__device__ __forceinline__ void ew_run_v(const EwProgram& P, int64_t lin, const int32_t* coord, const uint32_t* acc,
                                         RF& R, int pc_begin = 0, int pc_end = -1, const EwTables* T = nullptr) {
#define EW_FOR _Pragma("unroll") for (int e = 0; e < V; ++e)
#define EW_FA __uint_as_float(ra[e])
#define EW_FB __uint_as_float(rb[e])
#define EW_IA ((int32_t)ra[e])
#define EW_IB ((int32_t)rb[e])
#define EW_UA (ra[e])
#define EW_UB (rb[e])
#define EW_F(OP, EXPR) case OP: EW_FOR r[e] = __float_as_uint(EXPR); break;
#define EW_U(OP, EXPR) case OP: EW_FOR r[e] = (uint32_t)(EXPR); break;
// (PRE: the out-of-line heavy ops are compiled out; the launcher streams only programs without them, and a call in
// the loop would force the prefetched words out of registers)
#define EW_HEAVY(OP) case OP: if constexpr (!PRE) { _Pragma("unroll 1") for (int e = 0; e < V; ++e) r[e] = ew_heavy(OP, ra[e], rb[e], I.round); } break;
  const int end = pc_end < 0 ? P.n_instr : pc_end;
  EwInstr next = T ? uniform_read(&T->instr[pc_begin]) : P.instr[pc_begin];
  for (int pc = pc_begin; pc < end; ++pc) {
    const EwInstr I = next;
    if (pc + 1 < end) next = T ? uniform_read(&T->instr[pc + 1]) : P.instr[pc + 1];  // requested while I executes
    uint32_t r[V], ra[V], rb[V], rc[V];
    const int nsrc = ew_nsrc(I.op);
    if (nsrc >= 1) R.load(I.a, ra);
    if (nsrc >= 2) R.load(I.b, rb);
    if (nsrc >= 3) R.load(I.c, rc);
    switch (I.op) {
      case EW_LOAD:
        if constexpr (PRE) {
          uint32_t w[V];
          EW_FOR w[e] = I.a == 0 ? acc[e] : acc[V + e];
          decode_contig<V>(T ? uniform_read(&T->leaves[I.a].dtype) : P.leaves[I.a].dtype, w, r);
        } else {
          if (T) load_leaf<V>(uniform_read(&T->leaves[I.a]), lin, coord, P.rank, r);
          else load_leaf<V>(P.leaves[I.a], lin, coord, P.rank, r);
        }
        break;
      EW_U(EW_CONST, I.imm.u)
      EW_U(EW_IOTA, coord[I.a] + (I.a == P.rank - 1 ? e : 0))
      EW_U(EW_ACC, PRE ? 0u : acc[I.a])  // (a runtime index into acc would keep PRE's words out of registers)
      EW_F(EW_NEG, -EW_FA)
      EW_F(EW_ABS, fabsf(EW_FA))
      EW_F(EW_EXP, expf(EW_FA))
      EW_HEAVY(EW_LOG)
      EW_F(EW_RSQRT, 1.0f / sqrtf(EW_FA))
      EW_F(EW_SQRT, sqrtf(EW_FA))
      EW_HEAVY(EW_TANH)
      EW_F(EW_LOGISTIC, 1.0f / (1.0f + expf(-EW_FA)))
      EW_F(EW_FLOOR, floorf(EW_FA))
      EW_F(EW_CEIL, ceilf(EW_FA))
      EW_F(EW_SIGN, EW_FA != EW_FA ? EW_FA : (EW_FA > 0.f ? 1.f : (EW_FA < 0.f ? -1.f : EW_FA)))
      EW_HEAVY(EW_EXPM1)
      EW_HEAVY(EW_LOG1P)
      EW_HEAVY(EW_SIN)
      EW_HEAVY(EW_COS)
      EW_HEAVY(EW_TAN)
      EW_HEAVY(EW_CBRT)
      EW_F(EW_RINT, rintf(EW_FA))
      EW_F(EW_ROUND, roundf(EW_FA))
      EW_U(EW_ISFINITE, (EW_UA & 0x7f800000u) != 0x7f800000u)
      case EW_BITCAST:  // out of line, like the heavy ops
        if constexpr (!PRE) {
          _Pragma("unroll 1") for (int e = 0; e < V; ++e) r[e] = bitcast_reg(ra[e], I.imm.i >> 8, I.imm.i & 0xff);
        }
        break;
      case EW_REDPREC:
        if constexpr (!PRE) {
          _Pragma("unroll 1") for (int e = 0; e < V; ++e)
            r[e] = reduce_precision_reg(ra[e], I.imm.i >> 16, (I.imm.i >> 8) & 0xff, I.imm.i & 0xff);
        }
        break;
      EW_U(EW_INEG, -EW_IA)
      EW_U(EW_IABS, EW_IA < 0 ? -EW_IA : EW_IA)
      EW_U(EW_NOT, (I.round == DT_PRED) ? (uint32_t)(EW_IA == 0) : ~EW_UA)
      EW_U(EW_ISIGN, EW_IA > 0 ? 1 : (EW_IA < 0 ? -1 : 0))
      // bit counts over the element's own width (a narrow signed register holds its value sign-extended)
      EW_U(EW_POPCNT, __builtin_popcount(EW_UA & width_mask(I.imm.i)))
      EW_U(EW_CLZ, (EW_UA & width_mask(I.imm.i)) ? __builtin_clz(EW_UA & width_mask(I.imm.i)) - (32 - I.imm.i)
                                                  : I.imm.i)
      EW_F(EW_CVT_F2F, EW_FA)
      EW_HEAVY(EW_CVT_F2I)
      EW_F(EW_CVT_I2F, I.imm.i ? (float)EW_UA : (float)EW_IA)  // imm: source unsigned
      EW_U(EW_CVT_I2I, EW_UA)
      EW_U(EW_CVT_F2P, EW_FA != 0.0f)
      EW_U(EW_CVT_I2P, EW_IA != 0)
      EW_F(EW_ADD, EW_FA + EW_FB)
      EW_F(EW_SUB, EW_FA - EW_FB)
      EW_F(EW_MUL, EW_FA * EW_FB)
      EW_F(EW_DIV, EW_FA / EW_FB)
      EW_F(EW_MAX, (EW_FA != EW_FA || EW_FB != EW_FB) ? __uint_as_float(0x7fc00000u) : fmaxf(EW_FA, EW_FB))
      EW_F(EW_MIN, (EW_FA != EW_FA || EW_FB != EW_FB) ? __uint_as_float(0x7fc00000u) : fminf(EW_FA, EW_FB))
      EW_HEAVY(EW_POW)
      EW_HEAVY(EW_REM)
      EW_HEAVY(EW_ATAN2)
      EW_U(EW_IADD, EW_IA + EW_IB)
      EW_U(EW_ISUB, EW_IA - EW_IB)
      EW_U(EW_IMUL, EW_IA * EW_IB)
      EW_HEAVY(EW_IDIV)
      EW_HEAVY(EW_IREM)
      EW_HEAVY(EW_UDIV)
      EW_HEAVY(EW_UREM)
      EW_U(EW_IMAX, EW_IA > EW_IB ? EW_IA : EW_IB)
      EW_U(EW_IMIN, EW_IA < EW_IB ? EW_IA : EW_IB)
      EW_U(EW_UMAX, EW_UA > EW_UB ? EW_UA : EW_UB)
      EW_U(EW_UMIN, EW_UA < EW_UB ? EW_UA : EW_UB)
      EW_U(EW_AND, EW_UA & EW_UB)
      EW_U(EW_OR, EW_UA | EW_UB)
      EW_U(EW_XOR, EW_UA ^ EW_UB)
      EW_U(EW_SHL, EW_UB < (uint32_t)I.imm.i ? EW_UA << EW_UB : 0u)
      EW_U(EW_SRL, EW_UB < (uint32_t)I.imm.i ? (EW_UA & width_mask(I.imm.i)) >> EW_UB : 0u)
      EW_U(EW_SRA, sign_extend(EW_UA, I.imm.i) >> (EW_UB < (uint32_t)I.imm.i ? EW_UB : 31u))
      EW_U(EW_FCMP, cmp_f(EW_FA, EW_FB, I.imm.i))
      EW_U(EW_ICMP, cmp_i<int32_t>(EW_IA, EW_IB, I.imm.i))
      EW_U(EW_UCMP, cmp_i<uint32_t>(EW_UA, EW_UB, I.imm.i))
      EW_U(EW_SELECT, EW_UA ? EW_UB : rc[e])
      // clamp(min, x, max) = minimum(maximum(x, min), max), both NaN-propagating
      EW_F(EW_FCLAMP, (EW_FA != EW_FA || EW_FB != EW_FB || __uint_as_float(rc[e]) != __uint_as_float(rc[e]))
                          ? __uint_as_float(0x7fc00000u)
                          : fminf(fmaxf(EW_FB, EW_FA), __uint_as_float(rc[e])))
      EW_U(EW_ICLAMP, EW_IB < EW_IA ? EW_IA : (EW_IB > (int32_t)rc[e] ? (int32_t)rc[e] : EW_IB))
      default: EW_FOR r[e] = 0; break;
    }
    // per-op rounding to the StableHLO result element type
    // (one switch on the type, then straight-line code over the V elements)
    switch (I.round) {
      case 0: case DT_F32: case DT_S32: case DT_U32: break;
      case DT_BF16:
        if constexpr (V % 2 == 0) {
#pragma unroll
          for (int e = 0; e < V; e += 2) {
            const uint32_t pk = f32x2_to_bf16x2_bits(__uint_as_float(r[e]), __uint_as_float(r[e + 1]));
            r[e] = pk << 16, r[e + 1] = pk & 0xffff0000u;
          }
        } else {
          EW_FOR r[e] = (uint32_t)f32_to_bf16_bits(__uint_as_float(r[e])) << 16;
        }
        break;
      case DT_F16: EW_FOR r[e] = __float_as_uint((float)(_Float16)__uint_as_float(r[e])); break;
      case DT_F8E4M3FN: EW_FOR r[e] = __float_as_uint(e4m3fn_bits_to_f32(f32_to_e4m3fn_bits(__uint_as_float(r[e])))); break;
      case DT_F8E5M2: EW_FOR r[e] = __float_as_uint(e5m2_bits_to_f32(f32_to_e5m2_bits(__uint_as_float(r[e])))); break;
      case DT_S8: EW_FOR r[e] = (uint32_t)(int32_t)(int8_t)r[e]; break;
      case DT_S16: EW_FOR r[e] = (uint32_t)(int32_t)(int16_t)r[e]; break;
      case DT_U8: EW_FOR r[e] = r[e] & 0xffu; break;
      case DT_U16: EW_FOR r[e] = r[e] & 0xffffu; break;
      case DT_PRED: EW_FOR r[e] = r[e] != 0u; break;
      default: break;
    }
    R.store(I.dst, r);
  }
#undef EW_FOR
#undef EW_FA
#undef EW_FB
#undef EW_IA
#undef EW_IB
#undef EW_UA
#undef EW_UB
#undef EW_F
#undef EW_U
#undef EW_HEAVY
}

// Scalar form (one element): used by the generic GEMM epilogue and the unvectorised kernels.
__device__ __forceinline__ void ew_run(const EwProgram& P, int64_t lin, const int32_t* coord, const uint32_t* acc,
                                       RegFile1& R) {
  ew_run_v<1>(P, lin, coord, acc, R);
}

}  // namespace ryft
