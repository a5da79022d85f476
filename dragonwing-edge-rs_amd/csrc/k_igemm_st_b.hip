// int8 streamed-weight implicit-GEMM instantiations: requantize + activation
// table, with and without the fused residual QLinearAdd.
#include "igemm_stream.h"

namespace dw {

bool igemm_launch_st_i8_b(hipStream_t st, const IgemmArgs& a, const TileCfg& t, int epv) {
  if (epv == EPV_QU8_LUT) return ig::launch_st_tiles<1, EPV_QU8_LUT>(st, a, t);
  if (epv == EPV_QU8_LUT_RES) return ig::launch_st_tiles<1, EPV_QU8_LUT_RES>(st, a, t);
  return false;
}

}  // namespace dw
