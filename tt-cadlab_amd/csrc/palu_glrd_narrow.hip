// The grouped-latent scores kernel for K ranks up to 256 (palu_glrd_scores.h), in its own translation
// unit so that it is built with the MFMA results in VGPRs (-mllvm -amdgpu-mfma-vgpr-form, set for this
// file by the build). Same-box A/B of the r_k 128 launch: 55.5 -> 52.9 us tiled, 61.2 -> 57.5 us row-major.
#include "palu_glrd_scores.h"

namespace {

template <typename TabT, bool ROWS>
int narrow_kb(const DecodeArgs& a, float* scores, int n_wg, hipStream_t s) {
  switch ((a.rk_eff / 32 + 1) / 2) {              // the launch's rank blocks rounded up to even
    case 1: return launch_scores_full<2, TabT, ROWS>(a, scores, n_wg, s);
    case 2: return launch_scores_full<4, TabT, ROWS>(a, scores, n_wg, s);
    case 3: return launch_scores_full<6, TabT, ROWS>(a, scores, n_wg, s);
    case 4: return launch_scores_full<8, TabT, ROWS>(a, scores, n_wg, s);
  }
  return fail(PALU_EUNSUPPORTED, "grouped-latent r_k %d: not a narrow rank", a.rk_eff);
}

}  // namespace

namespace palu {

int glrd_scores_narrow(const DecodeArgs& a, float* scores, int n_wg, hipStream_t s, bool rows, bool tab_f32) {
  if (rows) return tab_f32 ? narrow_kb<float, true>(a, scores, n_wg, s) : narrow_kb<__bf16, true>(a, scores, n_wg, s);
  return tab_f32 ? narrow_kb<float, false>(a, scores, n_wg, s) : narrow_kb<__bf16, false>(a, scores, n_wg, s);
}

}  // namespace palu
