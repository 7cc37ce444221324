// MFMA GEMM instantiations: f32.
#include "gemm_mfma.h"

namespace ryft {

bool pick_f32(const GemmArgs& g, bool ar, bool br, Choice* c) {
  auto fits = [&](int bm, int bn, int bk) { return !ar && g.M % bm == 0 && g.N % bn == 0 && g.K % bk == 0; };
  if (g.dual) return false;
  if (fits(64, 64, 16 * (g.splits > 1 ? g.splits : 1))) {
    *c = br ? make_choice<MMA_F32, 64, 64, 16, 2, 2, false, true, false>("gemm_f32_mfma_64x64")
            : make_choice<MMA_F32, 64, 64, 16, 2, 2, false, false, false>("gemm_f32_mfma_64x64");
    return true;
  }
  if (g.splits > 1) return false;
  *c = edge_choice<MMA_F32, 64, 64, 16, 2, 2, false>(ar, br, "gemm_f32_mfma_edge_64x64");
  return true;
}

}  // namespace ryft
