// Pieces shared by the kernels that run elementwise programs VEC elements at a time (k_elementwise.hip,
// k_reduce_body.hip): the vector width, the register file, host-side leaf preparation and coordinate decomposition.
#pragma once

#include <hip/hip_runtime.h>

#include "ew_device.h"

namespace ryft {

constexpr int VEC = 8;    // elements per thread in the vectorised kernels
constexpr int VNT = 256;  // threads per workgroup there
using VRegs = SwitchRegFile<VEC>;

// Element size in bytes of the types leaves and outputs use.
inline int elem_size(int dt) {
  switch (dt) {
    case DT_F64: case DT_S64: case DT_U64: return 8;
    case DT_F32: case DT_S32: case DT_U32: return 4;
    case DT_BF16: case DT_F16: case DT_S16: case DT_U16: return 2;
    default: return 1;
  }
}

// Chooses how each leaf is read when VEC consecutive innermost elements are evaluated together; false when the
// program cannot run VEC-wide (innermost extent not a multiple of VEC, misaligned outputs, huge strides).
inline bool prepare_vec(EwProgram& p, bool check_outputs) {
  if (p.rank < 1 || p.shape[p.rank - 1] % VEC != 0) return false;
  for (int i = 0; i < p.n_leaves; ++i) {
    EwLeaf& L = p.leaves[i];
    const int es = elem_size(L.dtype);
    const int64_t s = L.kind == EW_LEAF_SCALAR ? 0 : (L.kind == EW_LEAF_IDENTITY ? 1 : L.strides[p.rank - 1]);
    L.vstride = 0;
    if (s == 0) { L.vmode = EW_VEC_BCAST; continue; }
    bool contig = s == 1 && es <= 4 && ((uintptr_t)L.ptr % (uintptr_t)(VEC * es)) == 0 && L.offset % VEC == 0;
    if (contig && L.kind == EW_LEAF_GENERAL)
      for (int d = 0; d < p.rank - 1; ++d)
        if (L.strides[d] % VEC) contig = false;
    if (contig) { L.vmode = EW_VEC_CONTIG; continue; }
    if (s > INT32_MAX || s < INT32_MIN) return false;
    L.vmode = EW_VEC_GATHER;
    L.vstride = (int32_t)s;
  }
  if (check_outputs)
    for (int o = 0; o < p.n_out; ++o)
      if (((uintptr_t)p.out_ptr[o] % (uintptr_t)(VEC * elem_size(p.out_dtype[o]))) != 0) return false;
  return true;
}

// Coordinates of a linear index; 32-bit arithmetic when the iteration space allows it.
__device__ __forceinline__ void decompose_fast(int64_t lin, const EwProgram& P, int32_t* coord) {
  if (P.total <= 0x7fffffff) {
    uint32_t l = (uint32_t)lin;
    for (int d = P.rank - 1; d >= 0; --d) {
      const uint32_t sd = (uint32_t)P.shape[d];
      coord[d] = (int32_t)(l % sd);
      l /= sd;
    }
  } else {
    decompose(lin, P, coord);
  }
}

}  // namespace ryft
