// Device-side helpers: typed loads/stores with StableHLO rounding rules, and the elementwise program interpreter
// shared by the elementwise, reduction-prologue and GEMM-epilogue kernels.
#pragma once

#include <hip/hip_runtime.h>

#include "../kernel_abi.h"

namespace ryft {

// DType values (PJRT_Buffer_Type numbering; kept literal so kernels do not include the C API header).
enum : int {
  DT_PRED = 1, DT_S8 = 2, DT_S16 = 3, DT_S32 = 4, DT_S64 = 5, DT_U8 = 6, DT_U16 = 7, DT_U32 = 8, DT_U64 = 9,
  DT_F16 = 10, DT_F32 = 11, DT_F64 = 12, DT_BF16 = 13, DT_F8E5M2 = 16, DT_F8E4M3FN = 17,
};

__device__ __forceinline__ bool dt_is_float(int t) {
  return t == DT_F32 || t == DT_BF16 || t == DT_F16 || t == DT_F8E4M3FN || t == DT_F8E5M2 || t == DT_F64;
}

// ---- bit-exact conversions (round to nearest even; f8E4M3FN overflow → NaN, f8E5M2 overflow → inf)
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ uint8_t f32_to_e4m3fn_bits(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) return (uint8_t)(sign | 0x7fu);
  uint32_t code;
  if (a < 0x3c800000u) {  // |x| < 2^-6: subnormal grid of 2^-9
    code = (uint32_t)rintf(__uint_as_float(a) * 512.0f);
  } else {
    uint32_t r = (a + 0x7ffffu + ((a >> 20) & 1u)) >> 20;
    code = r - ((127u - 7u) << 3);
    if (code > 0x7eu) code = 0x7fu;
  }
  return (uint8_t)(sign | code);
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
  for (int d = 0; d < rank; ++d) off += (int64_t)coord[d] * L.strides[d];
  return off;
}

__device__ __forceinline__ void decompose(int64_t lin, const EwProgram& P, int32_t* coord) {
  for (int d = P.rank - 1; d >= 0; --d) {
    int64_t s = P.shape[d];
    coord[d] = (int32_t)(lin % s);
    lin /= s;
  }
}

// Runs the program; `acc` holds the GEMM accumulators (bits) for EW_ACC. Results land in regs[].
__device__ __forceinline__ void ew_run(const EwProgram& P, int64_t lin, const int32_t* coord, const uint32_t* acc,
                                       uint32_t* regs) {
  for (int pc = 0; pc < P.n_instr; ++pc) {
    const EwInstr I = P.instr[pc];
    uint32_t r = 0;
    float fa = __uint_as_float(regs[I.a]), fb = __uint_as_float(regs[I.b]);
    int32_t ia = (int32_t)regs[I.a], ib = (int32_t)regs[I.b];
    switch (I.op) {
      case EW_LOAD: {
        const EwLeaf& L = P.leaves[I.a];
        r = load_bits(L.ptr, leaf_offset(L, lin, coord, P.rank), L.dtype);
        break;
      }
      case EW_CONST: r = I.imm.u; break;
      case EW_IOTA: r = (uint32_t)coord[I.a]; break;
      case EW_ACC: r = acc[I.a]; break;
      case EW_NEG: r = __float_as_uint(-fa); break;
      case EW_ABS: r = __float_as_uint(fabsf(fa)); break;
      case EW_EXP: r = __float_as_uint(expf(fa)); break;
      case EW_LOG: r = __float_as_uint(logf(fa)); break;
      case EW_RSQRT: r = __float_as_uint(1.0f / sqrtf(fa)); break;
      case EW_SQRT: r = __float_as_uint(sqrtf(fa)); break;
      case EW_TANH: r = __float_as_uint(tanhf(fa)); break;
      case EW_LOGISTIC: r = __float_as_uint(1.0f / (1.0f + expf(-fa))); break;
      case EW_FLOOR: r = __float_as_uint(floorf(fa)); break;
      case EW_CEIL: r = __float_as_uint(ceilf(fa)); break;
      case EW_SIGN: r = __float_as_uint(fa != fa ? fa : (fa > 0.f ? 1.f : (fa < 0.f ? -1.f : fa))); break;
      case EW_EXPM1: r = __float_as_uint(expm1f(fa)); break;
      case EW_LOG1P: r = __float_as_uint(log1pf(fa)); break;
      case EW_INEG: r = (uint32_t)(-ia); break;
      case EW_IABS: r = (uint32_t)(ia < 0 ? -ia : ia); break;
      case EW_NOT: r = (I.round == DT_PRED) ? (uint32_t)(ia == 0) : ~regs[I.a]; break;
      case EW_ISIGN: r = (uint32_t)(ia > 0 ? 1 : (ia < 0 ? -1 : 0)); break;
      case EW_CVT_F2F: r = __float_as_uint(fa); break;
      case EW_CVT_F2I: r = (uint32_t)f2i_sat(fa, I.round); break;
      case EW_CVT_I2F: r = __float_as_uint(I.imm.i ? (float)regs[I.a] : (float)ia); break;  // imm: source unsigned
      case EW_CVT_I2I: r = regs[I.a]; break;
      case EW_CVT_F2P: r = (uint32_t)(fa != 0.0f); break;
      case EW_CVT_I2P: r = (uint32_t)(ia != 0); break;
      case EW_ADD: r = __float_as_uint(fa + fb); break;
      case EW_SUB: r = __float_as_uint(fa - fb); break;
      case EW_MUL: r = __float_as_uint(fa * fb); break;
      case EW_DIV: r = __float_as_uint(fa / fb); break;
      case EW_MAX: r = __float_as_uint((fa != fa || fb != fb) ? __uint_as_float(0x7fc00000u) : fmaxf(fa, fb)); break;
      case EW_MIN: r = __float_as_uint((fa != fa || fb != fb) ? __uint_as_float(0x7fc00000u) : fminf(fa, fb)); break;
      case EW_POW: r = __float_as_uint(powf(fa, fb)); break;
      case EW_REM: r = __float_as_uint(fmodf(fa, fb)); break;
      case EW_IADD: r = (uint32_t)(ia + ib); break;
      case EW_ISUB: r = (uint32_t)(ia - ib); break;
      case EW_IMUL: r = (uint32_t)(ia * ib); break;
      case EW_IDIV: r = (uint32_t)(ib == 0 ? -1 : (ia == (int32_t)0x80000000 && ib == -1) ? ia : ia / ib); break;
      case EW_IREM: r = (uint32_t)(ib == 0 ? ia : (ib == -1 ? 0 : ia % ib)); break;
      case EW_UDIV: r = regs[I.b] == 0 ? 0xffffffffu : regs[I.a] / regs[I.b]; break;
      case EW_UREM: r = regs[I.b] == 0 ? regs[I.a] : regs[I.a] % regs[I.b]; break;
      case EW_IMAX: r = (uint32_t)(ia > ib ? ia : ib); break;
      case EW_IMIN: r = (uint32_t)(ia < ib ? ia : ib); break;
      case EW_UMAX: r = regs[I.a] > regs[I.b] ? regs[I.a] : regs[I.b]; break;
      case EW_UMIN: r = regs[I.a] < regs[I.b] ? regs[I.a] : regs[I.b]; break;
      case EW_AND: r = regs[I.a] & regs[I.b]; break;
      case EW_OR: r = regs[I.a] | regs[I.b]; break;
      case EW_XOR: r = regs[I.a] ^ regs[I.b]; break;
      case EW_FCMP: r = cmp_f(fa, fb, I.imm.i); break;
      case EW_ICMP: r = cmp_i<int32_t>(ia, ib, I.imm.i); break;
      case EW_UCMP: r = cmp_i<uint32_t>(regs[I.a], regs[I.b], I.imm.i); break;
      case EW_SELECT: r = regs[I.a] ? regs[I.b] : regs[I.c]; break;
      case EW_FCLAMP: {
        float x = fb, lo = fa, hi = __uint_as_float(regs[I.c]);
        r = __float_as_uint(fminf(fmaxf(x, lo), hi));
        break;
      }
      case EW_ICLAMP: {
        int32_t x = ib, lo = ia, hi = (int32_t)regs[I.c];
        r = (uint32_t)(x < lo ? lo : (x > hi ? hi : x));
        break;
      }
      default: break;
    }
    // per-op rounding to the StableHLO result element type
    if (I.round) {
      if (dt_is_float(I.round)) r = __float_as_uint(round_float(__uint_as_float(r), I.round));
      else if (I.op != EW_CVT_F2I) r = (uint32_t)wrap_int((int32_t)r, I.round);
      else r = (uint32_t)wrap_int((int32_t)r, I.round);
    }
    regs[I.dst] = r;
  }
}

}  // namespace ryft
