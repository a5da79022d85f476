// int8 row-tile implicit-GEMM instantiations: requantize + activation table,
// with and without the fused residual QLinearAdd.
#include "igemm_rows.h"

namespace dw {

bool igemm_launch_rows_i8_b(hipStream_t st, const IgemmArgs& a, const TileCfg& t, int epv) {
  if (epv == EPV_QU8_LUT) return ig::launch_rows_tiles<1, EPV_QU8_LUT>(st, a, t);
  if (epv == EPV_QU8_LUT_RES) return ig::launch_rows_tiles<1, EPV_QU8_LUT_RES>(st, a, t);
  return false;
}

}  // namespace dw
