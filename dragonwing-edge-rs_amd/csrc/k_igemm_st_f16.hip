// fp16 streamed-weight implicit-GEMM instantiations.
#include "igemm_stream.h"

namespace dw {

bool igemm_launch_st_f16(hipStream_t st, const IgemmArgs& a, const TileCfg& t) {
  return ig::launch_st_tiles<2, EPV_GENERIC>(st, a, t);
}

}  // namespace dw
