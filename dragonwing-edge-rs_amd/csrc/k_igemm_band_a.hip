// int8 band-tile implicit-GEMM instantiations: generic and plain-requantize
// epilogues.
#include "igemm_band.h"

namespace dw {

bool igemm_launch_band_i8_a(hipStream_t st, const IgemmArgs& a, const TileCfg& t, int epv) {
  if (epv == EPV_GENERIC) return ig::launch_band_tiles<1, EPV_GENERIC>(st, a, t);
  if (epv == EPV_QU8) return ig::launch_band_tiles<1, EPV_QU8>(st, a, t);
  return false;
}

}  // namespace dw
