// MFMA GEMM instantiations: bf16, f16.
#include "gemm_mfma.h"

namespace ryft {

bool pick_bf16(const GemmArgs& g, bool ar, bool br, Choice* c) {
  auto fits = [&](int bm, int bn, int bk) { return !ar && g.M % bm == 0 && g.N % bn == 0 && g.K % bk == 0; };
  if (g.dual) return false;
  if (g.splits > 1) {  // split-K runs the 128×128 tile over each K range
    if (!fits(128, 128, 64 * g.splits)) return false;
    *c = br ? make_choice<MMA_BF16, 128, 128, 64, 2, 2, false, true, false>("gemm_bf16_mfma_128x128")
            : make_choice<MMA_BF16, 128, 128, 64, 2, 2, false, false, false>("gemm_bf16_mfma_128x128");
    return true;
  }
  const int64_t tiles256 = (int64_t)(g.M / 256) * (g.N / 256) * g.batch;
  if (fits(256, 256, 64) && tiles256 >= 128) {
    // eight waves (two per SIMD, 128×64 each): one wave's LDS waits and barrier overlap the other's MFMAs
    *c = br ? make_choice<MMA_BF16, 256, 256, 64, 2, 4, false, true, false>("gemm_bf16_mfma_256x256")
            : make_choice<MMA_BF16, 256, 256, 64, 2, 4, false, false, false>("gemm_bf16_mfma_256x256");
    return true;
  }
  if (fits(128, 128, 64)) {
    *c = br ? make_choice<MMA_BF16, 128, 128, 64, 2, 2, false, true, false>("gemm_bf16_mfma_128x128")
            : make_choice<MMA_BF16, 128, 128, 64, 2, 2, false, false, false>("gemm_bf16_mfma_128x128");
    return true;
  }
  *c = edge_choice<MMA_BF16, 128, 128, 64, 2, 2, false>(ar, br, "gemm_bf16_mfma_edge_128x128");
  return true;
}

bool pick_f16(const GemmArgs& g, bool ar, bool br, Choice* c) {
  auto fits = [&](int bm, int bn, int bk) { return !ar && g.M % bm == 0 && g.N % bn == 0 && g.K % bk == 0; };
  if (g.dual) return false;
  if (fits(128, 128, 64 * (g.splits > 1 ? g.splits : 1))) {
    *c = br ? make_choice<MMA_F16, 128, 128, 64, 2, 2, false, true, false>("gemm_f16_mfma_128x128")
            : make_choice<MMA_F16, 128, 128, 64, 2, 2, false, false, false>("gemm_f16_mfma_128x128");
    return true;
  }
  if (g.splits > 1) return false;
  *c = edge_choice<MMA_F16, 128, 128, 64, 2, 2, false>(ar, br, "gemm_f16_mfma_edge_128x128");
  return true;
}

}  // namespace ryft
