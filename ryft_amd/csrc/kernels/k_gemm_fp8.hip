// MFMA GEMM instantiations: fp8.
#include "gemm_mfma.h"

namespace ryft {

bool pick_fp8(const GemmArgs& g, bool ar, bool br, Choice* c) {
  auto fits = [&](int bm, int bn, int bk) { return !ar && g.M % bm == 0 && g.N % bn == 0 && g.K % bk == 0; };
  if (g.splits > 1) {  // split-K runs the 128×128 tile over each K range
    if (g.dual || !fits(128, 128, 128 * g.splits)) return false;
    *c = br ? make_choice<MMA_FP8, 128, 128, 128, 2, 2, false, true, false>("gemm_fp8_mfma_128x128")
            : make_choice<MMA_FP8, 128, 128, 128, 2, 2, false, false, false>("gemm_fp8_mfma_128x128");
    return true;
  }
  if (g.dual) {
    if (!fits(128, 128, 128)) {
      *c = edge_choice<MMA_FP8, 128, 128, 128, 2, 2, true>(ar, br, "gemm_fp8_mfma_dual_edge_128x128");
      return true;
    }
    *c = br ? make_choice<MMA_FP8, 128, 128, 128, 2, 2, false, true, true>("gemm_fp8_mfma_dual_128x128")
            : make_choice<MMA_FP8, 128, 128, 128, 2, 2, false, false, true>("gemm_fp8_mfma_dual_128x128");
    return true;
  }
  if (fits(128, 128, 128) && (int64_t)(g.M / 128) * (g.N / 128) * g.batch >= 256) {
    *c = br ? make_choice<MMA_FP8, 128, 128, 128, 2, 2, false, true, false>("gemm_fp8_mfma_128x128")
            : make_choice<MMA_FP8, 128, 128, 128, 2, 2, false, false, false>("gemm_fp8_mfma_128x128");
    return true;
  }
  if (fits(64, 128, 128)) {
    *c = br ? make_choice<MMA_FP8, 64, 128, 128, 2, 2, false, true, false>("gemm_fp8_mfma_64x128")
            : make_choice<MMA_FP8, 64, 128, 128, 2, 2, false, false, false>("gemm_fp8_mfma_64x128");
    return true;
  }
  *c = edge_choice<MMA_FP8, 128, 128, 128, 2, 2, false>(ar, br, "gemm_fp8_mfma_edge_128x128");
  return true;
}

}  // namespace ryft
