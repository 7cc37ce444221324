// MFMA GEMM instantiations: bf16 activations × f8E4M3FN weights (an n-contiguous B stays f8 in LDS and is widened to
// bf16 in registers after its transposing read; a K-contiguous B is widened on its way into LDS).
#include "gemm_mfma.h"

namespace ryft {

bool pick_bf16f8(const GemmArgs& g, bool ar, bool br, Choice* c) {
  auto fits = [&](int bm, int bn, int bk) { return !ar && g.M % bm == 0 && g.N % bn == 0 && g.K % bk == 0; };
  if (g.splits > 1) {  // split-K: 128×256 tiles (eight waves of 64×64) over each K range, else 128×128
    if (g.dual) return false;
    if (fits(128, 256, 64 * g.splits)) {
      *c = br ? make_choice<MMA_BF16_F8, 128, 256, 64, 2, 4, false, true, false>("gemm_bf16f8_mfma_128x256")
              : make_choice<MMA_BF16_F8, 128, 256, 64, 2, 4, false, false, false>("gemm_bf16f8_mfma_128x256");
      return true;
    }
    if (!fits(128, 128, 64 * g.splits)) return false;
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
    *c = edge_choice<MMA_BF16_F8, 128, 128, 64, 2, 2, true>(ar, br, "gemm_bf16f8_mfma_dual_edge_128x128");
    return true;
  }
  const int64_t tiles256 = (int64_t)(g.M / 256) * (g.N / 256) * g.batch;
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
  *c = edge_choice<MMA_BF16_F8, 128, 128, 64, 2, 2, false>(ar, br, "gemm_bf16f8_mfma_edge_128x128");
  return true;
}

}  // namespace ryft
