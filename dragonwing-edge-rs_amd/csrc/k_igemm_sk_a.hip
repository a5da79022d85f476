// Persistent small-K int8 instantiations: generic epilogue and plain
// requantization.
#include "igemm_sk.h"

namespace dw {

bool igemm_launch_sk_i8_a(hipStream_t st, const IgemmArgs& a, const TileCfg& t, int epv) {
  if (epv == EPV_GENERIC) return ig::launch_sk_tiles<1, EPV_GENERIC>(st, a, t);
  if (epv == EPV_QU8) return ig::launch_sk_tiles<1, EPV_QU8>(st, a, t);
  return false;
}

}  // namespace dw
