// Fused latent decode kernels for tiled caches whose K latent width is an odd multiple of 16 (the K rows
// end in a half tile): every such width, V width and (table, output) dtype pair, instantiated in a
// translation unit of their own to keep builds parallel.
#include "palu_kernel.h"

namespace palu {

int dispatch_latent_tiled_k16(const DecodeArgs& a, int rk, int rv, int cs_dtype, int out_dtype, hipStream_t s) {
  return dispatch_dtypes<true, false, true>(a, rk, rv, cs_dtype, out_dtype, s);
}

}  // namespace palu
