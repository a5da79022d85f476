// fp16 row-tile implicit-GEMM instantiations (the generic f16 epilogue).
#include "igemm_rows.h"

namespace dw {

bool igemm_launch_rows_f16(hipStream_t st, const IgemmArgs& a, const TileCfg& t) {
  return ig::launch_rows_tiles<2, EPV_GENERIC>(st, a, t);
}

}  // namespace dw
