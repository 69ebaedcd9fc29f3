// Stock flash-decode kernels over full, already-rotated K (the non-fused decode path and the full-KV
// comparator): every V width (multiples of 32; of 16 for tiled caches), both cache layouts, contiguous or paged, fp32 or bf16 output.
#include "palu_kernel.h"

namespace {

template <bool TILED, bool PAGED>
int dispatch_full_dv(const palu::DecodeArgs& a, int dv, bool f32o, hipStream_t s) {
  using B16 = __bf16;
  switch (dv) {
    case 32: return f32o ? launch<HD, 32, true, TILED, PAGED, float, float>(a, s) : launch<HD, 32, true, TILED, PAGED, float, B16>(a, s);
    case 64: return f32o ? launch<HD, 64, true, TILED, PAGED, float, float>(a, s) : launch<HD, 64, true, TILED, PAGED, float, B16>(a, s);
    case 96: return f32o ? launch<HD, 96, true, TILED, PAGED, float, float>(a, s) : launch<HD, 96, true, TILED, PAGED, float, B16>(a, s);
    case 128: return f32o ? launch<HD, 128, true, TILED, PAGED, float, float>(a, s) : launch<HD, 128, true, TILED, PAGED, float, B16>(a, s);
  }
  if constexpr (TILED) {   // 16-wide V tiles: the widths in between as well
    switch (dv) {
      case 48: return f32o ? launch<HD, 48, true, TILED, PAGED, float, float>(a, s) : launch<HD, 48, true, TILED, PAGED, float, B16>(a, s);
      case 80: return f32o ? launch<HD, 80, true, TILED, PAGED, float, float>(a, s) : launch<HD, 80, true, TILED, PAGED, float, B16>(a, s);
      case 112: return f32o ? launch<HD, 112, true, TILED, PAGED, float, float>(a, s) : launch<HD, 112, true, TILED, PAGED, float, B16>(a, s);
    }
  }
  return fail(PALU_EUNSUPPORTED, "head_dim_v %d: this build supports V widths 32, 64, 96, 128 (and 48, 80, 112 for "
                                 "tiled caches)", dv);
}

}  // namespace

namespace palu {

int dispatch_full(const DecodeArgs& a, bool tiled, bool paged, int dv, bool f32_out, hipStream_t s) {
  if (paged) return tiled ? dispatch_full_dv<true, true>(a, dv, f32_out, s) : dispatch_full_dv<false, true>(a, dv, f32_out, s);
  return tiled ? dispatch_full_dv<true, false>(a, dv, f32_out, s) : dispatch_full_dv<false, false>(a, dv, f32_out, s);
}

}  // namespace palu
