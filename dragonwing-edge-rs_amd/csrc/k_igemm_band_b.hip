// int8 band-tile implicit-GEMM instantiations: requantize + activation
// table, with and without the fused residual QLinearAdd.
#include "igemm_band.h"

namespace dw {

bool igemm_launch_band_i8_b(hipStream_t st, const IgemmArgs& a, const TileCfg& t, int epv) {
  if (epv == EPV_QU8_LUT) return ig::launch_band_tiles<1, EPV_QU8_LUT>(st, a, t);
  if (epv == EPV_QU8_LUT_RES) return ig::launch_band_tiles<1, EPV_QU8_LUT_RES>(st, a, t);
  return false;
}

}  // namespace dw
