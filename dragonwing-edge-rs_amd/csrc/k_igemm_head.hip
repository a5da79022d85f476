// int8 implicit-GEMM instantiations with a detect head's u8 -> f16 1x1
// conv fused into the epilogue (EPV_QU8_LUT_HEAD): the staged kernel, the
// row-tile kernel and the band-tile kernel, tiles holding every channel of
// the 64- or 80-channel head convs.
#include "igemm_band.h"
#include "igemm_rows.h"

namespace dw {

bool igemm_launch_head_i8(hipStream_t st, const IgemmArgs& a, const TileCfg& t) {
  if (t.tpw == 0) {
    const int wgpix = 64 * t.pb;
    const dim3 grid((unsigned)(((a.m + wgpix - 1) / wgpix) * (a.cout_pad / t.bc)));
    if (t.bc == 64) return ig::launch_bc<1, 64, EPV_QU8_LUT_HEAD>(st, a, t, grid);
    if (t.bc == 80) return ig::launch_bc<1, 80, EPV_QU8_LUT_HEAD>(st, a, t, grid);
    return false;
  }
  if (t.tpw == -2) {
    const int r = ig::kRowsPix / a.w;
    const dim3 grid((unsigned)(a.n * (a.h / r) * (a.cout_pad / t.bc)));
    const size_t lds = ig::rows_lds_bytes(t.bc, a.ksteps, a.w, a.cin, 1);
    if (t.bc == 64) {
      hipLaunchKernelGGL((ig::igemm_rows_kernel<1, 64, EPV_QU8_LUT_HEAD>), grid, dim3(256), lds, st, a);
      return true;
    }
    if (t.bc == 80) {
      hipLaunchKernelGGL((ig::igemm_rows_kernel<1, 80, EPV_QU8_LUT_HEAD>), grid, dim3(256), lds, st, a);
      return true;
    }
  }
  if (t.tpw == -4) {
    if (t.bc == 64) {
      ig::launch_band_bc<1, 64, EPV_QU8_LUT_HEAD, 8>(st, a, t);
      return true;
    }
    if (t.bc == 80) {
      ig::launch_band_bc<1, 80, EPV_QU8_LUT_HEAD, 8>(st, a, t);
      return true;
    }
  }
  return false;
}

}  // namespace dw
