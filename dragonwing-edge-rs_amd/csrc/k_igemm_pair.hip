// The chained pair of int8 3x3 convolutions (a C2f bottleneck) in one
// launch: shape checks, band heights, launch geometry and the
// instantiations.
#include "igemm_pair.h"

namespace dw {
namespace {

// The pair's shapes and views, independent of the band height.
bool pair_shapes_ok(const IgemmArgs& a1, const IgemmArgs& a2) {
  const int c = a1.cin;
  if (!(c == 16 || c == 32 || c == 64)) return false;
  if (a1.cout != c || a2.cin != c || a2.cout != c) return false;
  if (a1.epi != EPI_QU8 || a2.epi != EPI_QU8 || !a1.lut || !a2.lut || !a1.bias_i || !a2.bias_i || a1.res)
    return false;
  for (const IgemmArgs* a : {&a1, &a2})
    if (a->kh != 3 || a->kw != 3 || a->sh != 1 || a->sw != 1 || a->pt != 1 || a->pl != 1 || a->ho != a->h ||
        a->wo != a->w || a->ksteps != (9 * c + 63) / 64 || a->cout_pad < c)
      return false;
  if (a2.n != a1.n || a2.h != a1.h || a2.w != a1.w || a1.w < 1 || a1.h < 1) return false;
  // the second conv reads exactly what the first writes
  if (a2.x != (const uint8_t*)a1.y || a2.x_pix_stride != a1.y_pix_stride || a2.x_c_off != a1.y_c_off) return false;
  // the residual, if any, is the block input
  if (a2.res && (a2.res != (const void*)a1.x || a2.r_pix_stride != a1.x_pix_stride || a2.r_c_off != a1.x_c_off))
    return false;
  if (a1.x_pix_stride % 16 != 0 || a1.x_c_off % 16 != 0 || a2.y_pix_stride % 4 != 0 || a2.y_c_off % 4 != 0)
    return false;
  if ((long long)a1.n * a1.h * a1.w * a1.x_pix_stride >= (1ll << 31)) return false;
  return (long long)a1.n * a1.h * a1.w < (1ll << 24);
}

}  // namespace

bool igemm_pair_ok(const IgemmArgs& a1, const IgemmArgs& a2, int rows) {
  if (!pair_shapes_ok(a1, a2) || rows < 1 || a1.h % rows != 0) return false;
  const int c = a1.cin, w = a1.w;
  if ((rows + 4) * (w + 2) * (c / 16) > ig::kPairFill * 256) return false;  // the input tile's start-up loads
  return ig::pair_lds_bytes(c, a1.ksteps, w, rows) <= 160 * 1024;
}

int igemm_pair_rows(const IgemmArgs& a1, const IgemmArgs& a2, int* rows, int max) {
  int n = 0;
  if (!pair_shapes_ok(a1, a2)) return 0;
  // band heights of at least 64 output pixels, tallest first (least
  // recomputed halo), at most `max` of them
  for (int r = a1.h; r >= 1 && n < max; --r)
    if (r * a1.w >= 64 && igemm_pair_ok(a1, a2, r)) rows[n++] = r;
  return n;
}

bool igemm_pair_lds_two_per_cu(const IgemmArgs& a1, int rows) {
  return ig::pair_lds_bytes(a1.cin, a1.ksteps, a1.w, rows) <= 80 * 1024;
}

void launch_igemm_pair(hipStream_t st, const IgemmArgs& a1_in, const IgemmArgs& a2_in, int rows, int waves) {
  if (!igemm_pair_ok(a1_in, a2_in, rows)) fail(-2, "igemm pair: unsupported shapes, views or band height");
  if (waves != 4 && waves != 16) fail(-2, "igemm pair: 4 or 16 waves");
  ig::PairArgs p;
  p.a1 = a1_in;
  p.a2 = a2_in;
  const int w = p.a1.w, h = p.a1.h, c = p.a1.cin;
  p.rows = rows;
  p.a1.x_bytes = (int)((long long)p.a1.n * h * w * p.a1.x_pix_stride);
  p.a1.r_wo = 1.0f / (float)w;
  const dim3 grid((unsigned)(p.a1.n * (h / rows)));
  const size_t lds = (size_t)ig::pair_lds_bytes(c, p.a1.ksteps, w, rows);
  const bool res = p.a2.res != nullptr;
#define DW_P(CB_)                                                                                       \
  if (c == 16 * (CB_)) {                                                                               \
    if (res && waves == 16)                                                                            \
      hipLaunchKernelGGL((ig::igemm_pair_kernel<CB_, true, 16>), grid, dim3(1024), lds, st, p);       \
    else if (res)                                                                                      \
      hipLaunchKernelGGL((ig::igemm_pair_kernel<CB_, true, 4>), grid, dim3(256), lds, st, p);         \
    else if (waves == 16)                                                                              \
      hipLaunchKernelGGL((ig::igemm_pair_kernel<CB_, false, 16>), grid, dim3(1024), lds, st, p);      \
    else                                                                                               \
      hipLaunchKernelGGL((ig::igemm_pair_kernel<CB_, false, 4>), grid, dim3(256), lds, st, p);        \
    DW_HIP(hipGetLastError());                                                                         \
    return;                                                                                            \
  }
  DW_P(1) DW_P(2) DW_P(4)
#undef DW_P
  fail(-2, "igemm pair: no kernel for the channel count");
}

}  // namespace dw
