// Shared definitions for the MI355X PJRT plugin: element types, status, small utilities.
#pragma once

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "pjrt_c_api.h"

namespace ryft {

// Element types use the PJRT_Buffer_Type numbering (crates/ryft-pjrt/src/buffers.rs:2568-2600) so that a
// buffer's type crosses the ABI without translation.
enum class DType : uint32_t {
  INVALID = PJRT_Buffer_Type_INVALID,
  PRED = PJRT_Buffer_Type_PRED,
  S8 = PJRT_Buffer_Type_S8,
  S16 = PJRT_Buffer_Type_S16,
  S32 = PJRT_Buffer_Type_S32,
  S64 = PJRT_Buffer_Type_S64,
  U8 = PJRT_Buffer_Type_U8,
  U16 = PJRT_Buffer_Type_U16,
  U32 = PJRT_Buffer_Type_U32,
  U64 = PJRT_Buffer_Type_U64,
  F16 = PJRT_Buffer_Type_F16,
  F32 = PJRT_Buffer_Type_F32,
  F64 = PJRT_Buffer_Type_F64,
  BF16 = PJRT_Buffer_Type_BF16,
  F8E5M2 = PJRT_Buffer_Type_F8E5M2,
  F8E4M3FN = PJRT_Buffer_Type_F8E4M3FN,
};

inline size_t dtype_size(DType t) {
  switch (t) {
    case DType::PRED: case DType::S8: case DType::U8: case DType::F8E5M2: case DType::F8E4M3FN: return 1;
    case DType::S16: case DType::U16: case DType::F16: case DType::BF16: return 2;
    case DType::S32: case DType::U32: case DType::F32: return 4;
    case DType::S64: case DType::U64: case DType::F64: return 8;
    default: return 0;
  }
}
inline bool dtype_is_float(DType t) {
  return t == DType::F16 || t == DType::F32 || t == DType::F64 || t == DType::BF16 || t == DType::F8E5M2 ||
         t == DType::F8E4M3FN;
}
inline bool dtype_is_unsigned(DType t) {
  return t == DType::U8 || t == DType::U16 || t == DType::U32 || t == DType::U64 || t == DType::PRED;
}
inline bool dtype_is_int(DType t) { return !dtype_is_float(t) && t != DType::INVALID; }
const char* dtype_name(DType t);  // MLIR spelling, e.g. "bf16", "f8E4M3FN", "i1"
bool dtype_from_pjrt(PJRT_Buffer_Type t, DType* out);

// Errors inside the plugin are C++ exceptions carrying a PJRT error code; the C API boundary converts them to
// PJRT_Error objects (crates/ryft-pjrt/src/errors.rs:76-180 reads them back).
// An error may carry (name, value) payload strings, as PJRT_Error_ForEachPayload reports them.
using Payload = std::vector<std::pair<std::string, std::string>>;
struct Status : std::runtime_error {
  PJRT_Error_Code code;
  Payload payload;
  Status(PJRT_Error_Code c, const std::string& m, Payload p = {}) : std::runtime_error(m), code(c), payload(std::move(p)) {}
};
[[noreturn]] inline void fail(PJRT_Error_Code code, const std::string& msg) { throw Status(code, msg); }
[[noreturn]] inline void invalid(const std::string& msg) { fail(PJRT_Error_Code_INVALID_ARGUMENT, msg); }
[[noreturn]] inline void unimplemented(const std::string& msg) { fail(PJRT_Error_Code_UNIMPLEMENTED, msg); }

inline int64_t num_elements(const std::vector<int64_t>& shape) {
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  return n;
}
std::string shape_str(const std::vector<int64_t>& shape);

// Host-side bit-exact conversions used for constants and by the front-end.
uint16_t f32_to_bf16_rne(float f);
float bf16_to_f32(uint16_t h);
uint16_t f32_to_f16_rne(float f);
float f16_to_f32(uint16_t h);
uint8_t f32_to_f8e4m3fn_rne(float f);
float f8e4m3fn_to_f32(uint8_t v);
uint8_t f32_to_f8e5m2_rne(float f);
float f8e5m2_to_f32(uint8_t v);

}  // namespace ryft
