// GEMM epilogues shared by the generic and MFMA GEMM kernels: one call per accumulator element at (b, m, n).
#pragma once

#include "ew_device.h"

namespace ryft {

template <bool INT_ACC>
__device__ __forceinline__ uint32_t acc_bits(float f, int32_t i) {
  return INT_ACC ? (uint32_t)i : __float_as_uint(f);
}

// acc0/acc1 hold float accumulators (or int32 in `iacc0` when INT_ACC).
template <bool INT_ACC>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& G, int b, int m, int n, float acc0, int32_t iacc0,
                                              float acc1) {
  const int64_t lin = ((int64_t)b * G.M + m) * (int64_t)G.N + n;
  const uint32_t raw = acc_bits<INT_ACC>(acc0, iacc0);
  switch (G.epilogue) {
    case EPI_STORE:
      store_bits(G.out_ptr[0], lin, G.out_dtype[0], raw, !INT_ACC);
      break;
    case EPI_SCALE: {
      float v = INT_ACC ? (float)iacc0 : acc0;
      v *= G.alpha;
      if (G.row) v *= G.row[(int64_t)b * G.row_sb + (int64_t)m * G.row_sm];
      if (G.col) v *= G.col[(int64_t)b * G.col_sb + (int64_t)n * G.col_sn];
      if (G.mid_round) v = round_float(v, G.mid_round);
      store_bits(G.out_ptr[0], lin, G.out_dtype[0], __float_as_uint(v), true);
      if (G.raw_out) store_bits(G.out_ptr[1], lin, G.out_dtype[1], raw, !INT_ACC);
      break;
    }
    case EPI_SWIGLU: {
      float a = acc0, u = acc1;
      if (G.col) a *= G.col[(int64_t)b * G.col_sb + (int64_t)n * G.col_sn];
      if (G.col2) u *= G.col2[(int64_t)b * G.col2_sb + (int64_t)n * G.col2_sn];
      float lg = 1.0f / (1.0f + expf(-a));
      float v = (a * lg) * u;
      if (G.mid_round) v = round_float(v, G.mid_round);
      store_bits(G.out_ptr[0], lin, G.out_dtype[0], __float_as_uint(v), true);
      break;
    }
    default: {  // EPI_PROGRAM
      const EwProgram& P = G.epi;
      int32_t coord[EW_MAX_RANK];
      if (P.needs_coords) {
        // split (b, m, n) over the dot result's (batch, lhs-free, rhs-free) dimension groups
        int64_t v3[3] = {b, m, n};
        int d = P.rank - 1;
        for (int g = 2; g >= 0; --g) {
          int64_t v = v3[g];
          for (int k = 0; k < G.epi_groups[g]; ++k, --d) {
            int64_t s = P.shape[d];
            coord[d] = (int32_t)(v % s);
            v /= s;
          }
        }
      }
      uint32_t acc[2] = {raw, __float_as_uint(acc1)};
      RegFile1 R;
      ew_run(P, lin, coord, acc, R);
      store_bits(G.out_ptr[0], lin, P.out_dtype[0], R.get(P.out_reg[0]), (P.out_float_mask & 1) != 0);
      if (G.n_out > 1) store_bits(G.out_ptr[1], lin, G.out_dtype[1], raw, !INT_ACC);
      break;
    }
  }
}

}  // namespace ryft
