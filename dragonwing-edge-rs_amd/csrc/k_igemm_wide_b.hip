// int8 wide-tile implicit-GEMM instantiations: the activation-table
// epilogues (with and without the residual QLinearAdd).
#include "igemm_wide.h"

namespace dw {

bool igemm_launch_wide_i8_b(hipStream_t st, const IgemmArgs& a, const TileCfg& t, int epv) {
  if (epv == EPV_QU8_LUT) return ig::launch_wide_tiles<1, EPV_QU8_LUT>(st, a, t);
  if (epv == EPV_QU8_LUT_RES) return ig::launch_wide_tiles<1, EPV_QU8_LUT_RES>(st, a, t);
  return false;
}

}  // namespace dw
