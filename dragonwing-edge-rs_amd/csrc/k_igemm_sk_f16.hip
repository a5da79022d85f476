// Persistent small-K fp16 instantiations.
#include "igemm_sk.h"

namespace dw {

bool igemm_launch_sk_f16(hipStream_t st, const IgemmArgs& a, const TileCfg& t) {
  return ig::launch_sk_tiles<2, EPV_GENERIC>(st, a, t);
}

}  // namespace dw
