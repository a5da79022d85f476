// fp16 band-tile implicit-GEMM instantiations (the generic f16 epilogue).
#include "igemm_band.h"

namespace dw {

bool igemm_launch_band_f16(hipStream_t st, const IgemmArgs& a, const TileCfg& t) {
  return ig::launch_band_tiles<2, EPV_GENERIC>(st, a, t);
}

}  // namespace dw
