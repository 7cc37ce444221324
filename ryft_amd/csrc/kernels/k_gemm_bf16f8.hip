// MFMA GEMM instantiations: bf16 activations × f8E4M3FN weights (B widened to bf16 on its way into LDS).
#include "gemm_mfma.h"

namespace ryft {

bool pick_bf16f8(const GemmArgs& g, bool br, Choice* c) {
  auto fits = [&](int bm, int bn, int bk) { return g.M % bm == 0 && g.N % bn == 0 && g.K % bk == 0; };
  const int64_t tiles256 = (int64_t)(g.M / 256) * (g.N / 256) * g.batch;
  if (g.splits > 1) {  // split-K runs the 128×128 tile over each K range
    if (g.dual || !fits(128, 128, 64 * g.splits)) return false;
    *c = br ? make_choice<MMA_BF16_F8, 128, 128, 64, 2, 2, false, true, false>("gemm_bf16f8_mfma_128x128")
            : make_choice<MMA_BF16_F8, 128, 128, 64, 2, 2, false, false, false>("gemm_bf16f8_mfma_128x128");
    return true;
  }
  if (g.dual) {
    // gate and up tiles of 256 rows × 128 columns each, sharing the A tile: eight waves of 128×32 per B operand
    if (fits(256, 128, 64)) {
      *c = br ? make_choice<MMA_BF16_F8, 256, 128, 64, 2, 4, false, true, true>("gemm_bf16f8_mfma_dual_256x128")
              : make_choice<MMA_BF16_F8, 256, 128, 64, 2, 4, false, false, true>("gemm_bf16f8_mfma_dual_256x128");
      return true;
    }
    if (fits(128, 128, 64)) {
      *c = br ? make_choice<MMA_BF16_F8, 128, 128, 64, 2, 2, false, true, true>("gemm_bf16f8_mfma_dual_128x128")
              : make_choice<MMA_BF16_F8, 128, 128, 64, 2, 2, false, false, true>("gemm_bf16f8_mfma_dual_128x128");
      return true;
    }
    return false;
  }
  if (fits(256, 256, 64) && tiles256 >= 128) {
    *c = br ? make_choice<MMA_BF16_F8, 256, 256, 64, 2, 4, false, true, false>("gemm_bf16f8_mfma_256x256")
            : make_choice<MMA_BF16_F8, 256, 256, 64, 2, 4, false, false, false>("gemm_bf16f8_mfma_256x256");
    return true;
  }
  if (fits(128, 128, 64)) {
    *c = br ? make_choice<MMA_BF16_F8, 128, 128, 64, 2, 2, false, true, false>("gemm_bf16f8_mfma_128x128")
            : make_choice<MMA_BF16_F8, 128, 128, 64, 2, 2, false, false, false>("gemm_bf16f8_mfma_128x128");
    return true;
  }
  return false;
}

}  // namespace ryft
