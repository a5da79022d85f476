// fp16 wide-tile implicit-GEMM instantiations (input rows of whole 128-byte
// units: c_in % 64 == 0), with the f16 epilogue chain.
#include "igemm_wide.h"

namespace dw {

bool igemm_launch_wide_f16(hipStream_t st, const IgemmArgs& a, const TileCfg& t) {
  return ig::launch_wide_tiles<2, EPV_GENERIC>(st, a, t);
}

}  // namespace dw
