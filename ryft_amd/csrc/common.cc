// Element-type names and bit-exact host conversions (IEEE-754 round-to-nearest-even).
#include "common.h"

#include <cmath>
#include <sstream>

namespace ryft {

const char* dtype_name(DType t) {
  switch (t) {
    case DType::PRED: return "i1";
    case DType::S8: return "i8";
    case DType::S16: return "i16";
    case DType::S32: return "i32";
    case DType::S64: return "i64";
    case DType::U8: return "ui8";
    case DType::U16: return "ui16";
    case DType::U32: return "ui32";
    case DType::U64: return "ui64";
    case DType::F16: return "f16";
    case DType::F32: return "f32";
    case DType::F64: return "f64";
    case DType::BF16: return "bf16";
    case DType::F8E5M2: return "f8E5M2";
    case DType::F8E4M3FN: return "f8E4M3FN";
    default: return "invalid";
  }
}

bool dtype_from_pjrt(PJRT_Buffer_Type t, DType* out) {
  switch (t) {
    case PJRT_Buffer_Type_PRED: case PJRT_Buffer_Type_S8: case PJRT_Buffer_Type_S16: case PJRT_Buffer_Type_S32:
    case PJRT_Buffer_Type_S64: case PJRT_Buffer_Type_U8: case PJRT_Buffer_Type_U16: case PJRT_Buffer_Type_U32:
    case PJRT_Buffer_Type_U64: case PJRT_Buffer_Type_F16: case PJRT_Buffer_Type_F32: case PJRT_Buffer_Type_F64:
    case PJRT_Buffer_Type_BF16: case PJRT_Buffer_Type_F8E5M2: case PJRT_Buffer_Type_F8E4M3FN:
      *out = (DType)t;
      return true;
    default:
      return false;
  }
}

std::string shape_str(const std::vector<int64_t>& shape) {
  std::ostringstream os;
  os << "[";
  for (size_t i = 0; i < shape.size(); ++i) os << (i ? "," : "") << shape[i];
  os << "]";
  return os.str();
}

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);  // quiet NaN, sign kept
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

// Rounds |a| (finite, non-negative) to a binary format with `mbits` stored mantissa bits and minimum normal
// exponent `emin`, returning (exponent field, mantissa field) before any overflow check. Round-to-nearest-even via
// nearbyint on an exactly scaled value.
static void round_small_float(float a, int mbits, int emin, int bias, int* efield, int* mfield) {
  if (a == 0.0f) { *efield = 0; *mfield = 0; return; }
  int e;
  std::frexp(a, &e);  // a = f * 2^e, f in [0.5, 1)
  int exp = e - 1;    // a in [2^exp, 2^(exp+1))
  if (exp < emin) {
    double quantum = std::ldexp(1.0, emin - mbits);
    double q = std::nearbyint((double)a / quantum);
    if (q >= (double)(1 << mbits)) { *efield = 1; *mfield = 0; }
    else { *efield = 0; *mfield = (int)q; }
    return;
  }
  double quantum = std::ldexp(1.0, exp - mbits);
  double q = std::nearbyint((double)a / quantum);
  if (q >= (double)(2 << mbits)) { exp += 1; q = (double)(1 << mbits); }
  *efield = exp + bias;
  *mfield = (int)q - (1 << mbits);
}

uint16_t f32_to_f16_rne(float f) {
  uint32_t u = f2u(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  float a = std::fabs(f);
  if (std::isnan(f)) return sign | 0x7e00;
  if (std::isinf(f)) return sign | 0x7c00;
  int ef, mf;
  round_small_float(a, 10, -14, 15, &ef, &mf);
  if (ef >= 31) return sign | 0x7c00;
  return (uint16_t)(sign | (ef << 10) | mf);
}
float f16_to_f32(uint16_t h) {
  int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
  float v;
  if (e == 0) v = std::ldexp((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = std::ldexp((float)(m | 1024), e - 25);
  return s ? -v : v;
}

// f8E4M3FN: 4 exponent bits (bias 7), 3 mantissa bits, no infinities, 0x7f/0xff are NaN, max finite 448.
// Values that round above 448 become NaN (non-saturating conversion, as ml_dtypes / XLA convert).
uint8_t f32_to_f8e4m3fn_rne(float f) {
  uint8_t sign = (f2u(f) >> 24) & 0x80;
  if (std::isnan(f) || std::isinf(f)) return sign | 0x7f;
  int ef, mf;
  round_small_float(std::fabs(f), 3, -6, 7, &ef, &mf);
  if (ef > 15 || (ef == 15 && mf == 7)) return sign | 0x7f;
  return (uint8_t)(sign | (ef << 3) | mf);
}
float f8e4m3fn_to_f32(uint8_t v) {
  int s = v >> 7, e = (v >> 3) & 15, m = v & 7;
  float r;
  if (e == 15 && m == 7) r = NAN;
  else if (e == 0) r = std::ldexp((float)m, -9);
  else r = std::ldexp((float)(m | 8), e - 10);
  return s ? -r : r;
}

// f8E5M2: IEEE-like, 5 exponent bits (bias 15), 2 mantissa bits, with infinities.
uint8_t f32_to_f8e5m2_rne(float f) {
  uint8_t sign = (f2u(f) >> 24) & 0x80;
  if (std::isnan(f)) return sign | 0x7f;
  if (std::isinf(f)) return sign | 0x7c;
  int ef, mf;
  round_small_float(std::fabs(f), 2, -14, 15, &ef, &mf);
  if (ef >= 31) return sign | 0x7c;
  return (uint8_t)(sign | (ef << 2) | mf);
}
float f8e5m2_to_f32(uint8_t v) {
  int s = v >> 7, e = (v >> 2) & 31, m = v & 3;
  float r;
  if (e == 31) r = m ? NAN : INFINITY;
  else if (e == 0) r = std::ldexp((float)m, -16);
  else r = std::ldexp((float)(m | 4), e - 17);
  return s ? -r : r;
}

}  // namespace ryft
