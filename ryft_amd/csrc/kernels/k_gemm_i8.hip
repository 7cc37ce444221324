// MFMA GEMM instantiations: i8.
#include "gemm_mfma.h"

namespace ryft {

bool pick_i8(const GemmArgs& g, bool ar, bool br, Choice* c) {
  auto fits = [&](int bm, int bn, int bk) { return !ar && g.M % bm == 0 && g.N % bn == 0 && g.K % bk == 0; };
  if (g.dual) return false;
  if (g.splits > 1) {  // split-K runs the 128×128 tile over each K range
    if (!fits(128, 128, 128 * g.splits)) return false;
    *c = br ? make_choice<MMA_I8, 128, 128, 128, 2, 2, false, true, false>("gemm_i8_mfma_128x128")
            : make_choice<MMA_I8, 128, 128, 128, 2, 2, false, false, false>("gemm_i8_mfma_128x128");
    return true;
  }
  const int64_t tiles256 = (int64_t)(g.M / 256) * (g.N / 256) * g.batch;
  if (fits(256, 256, 128) && tiles256 >= 128) {
    // eight waves (two per SIMD, 128×64 each): one wave's LDS waits and barrier overlap the other's MFMAs
    *c = br ? make_choice<MMA_I8, 256, 256, 128, 2, 4, false, true, false>("gemm_i8_mfma_256x256")
            : make_choice<MMA_I8, 256, 256, 128, 2, 4, false, false, false>("gemm_i8_mfma_256x256");
    return true;
  }
  if (fits(128, 128, 128)) {
    *c = br ? make_choice<MMA_I8, 128, 128, 128, 2, 2, false, true, false>("gemm_i8_mfma_128x128")
            : make_choice<MMA_I8, 128, 128, 128, 2, 2, false, false, false>("gemm_i8_mfma_128x128");
    return true;
  }
  *c = edge_choice<MMA_I8, 128, 128, 128, 2, 2, false>(ar, br, "gemm_i8_mfma_edge_128x128");
  return true;
}

}  // namespace ryft
