// fp16 implicit-GEMM instantiations.
#include "igemm_kernel.h"

namespace dw {

bool igemm_launch_f16(hipStream_t st, const IgemmArgs& a, const TileCfg& t) {
  return ig::launch_tiles<2, EPV_GENERIC>(st, a, t);
}

}  // namespace dw
