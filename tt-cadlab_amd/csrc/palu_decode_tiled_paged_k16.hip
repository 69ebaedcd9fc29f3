// Fused latent decode kernels for paged tiled caches whose K latent width is an odd multiple of 16:
// every such width, V width and (table, output) dtype pair, in a translation unit of their own.
#include "palu_kernel.h"

namespace palu {

int dispatch_latent_tiled_paged_k16(const DecodeArgs& a, int rk, int rv, int cs_dtype, int out_dtype, hipStream_t s) {
  return dispatch_dtypes<true, true, true>(a, rk, rv, cs_dtype, out_dtype, s);
}

}  // namespace palu
