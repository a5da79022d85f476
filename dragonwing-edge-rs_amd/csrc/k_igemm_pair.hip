// The chained pair of int8 3x3 convolutions (a C2f bottleneck) in one
// launch: shape checks, launch geometry and the instantiations.
#include "igemm_pair.h"

namespace dw {
namespace {

// 16-pixel blocks per wave in phase 1: (rows + 2) * w pixels over 4 waves
int pair_pb1(int w, int rows) { return ((rows + 2) * w + 63) / 64; }

}  // namespace

bool igemm_pair_ok(const IgemmArgs& a1, const IgemmArgs& a2) {
  const int c = a1.cin;
  if (!(c == 16 || c == 32 || c == 64)) return false;
  if (a1.cout != c || a2.cin != c || a2.cout != c) return false;
  if (a1.epi != EPI_QU8 || a2.epi != EPI_QU8 || !a1.lut || !a2.lut || !a1.bias_i || !a2.bias_i || a1.res)
    return false;
  for (const IgemmArgs* a : {&a1, &a2})
    if (a->kh != 3 || a->kw != 3 || a->sh != 1 || a->sw != 1 || a->pt != 1 || a->pl != 1 || a->ho != a->h ||
        a->wo != a->w || a->ksteps != (9 * c + 63) / 64 || a->cout_pad < c)
      return false;
  if (a2.n != a1.n || a2.h != a1.h || a2.w != a1.w) return false;
  // the second conv reads exactly what the first writes
  if (a2.x != (const uint8_t*)a1.y || a2.x_pix_stride != a1.y_pix_stride || a2.x_c_off != a1.y_c_off) return false;
  // the residual, if any, is the block input
  if (a2.res && (a2.res != (const void*)a1.x || a2.r_pix_stride != a1.x_pix_stride || a2.r_c_off != a1.x_c_off))
    return false;
  if (a1.x_pix_stride % 16 != 0 || a1.x_c_off % 16 != 0 || a2.y_pix_stride % 4 != 0 || a2.y_c_off % 4 != 0)
    return false;
  const int w = a1.w, h = a1.h;
  if (w <= 0 || ig::kPairPix % w != 0) return false;
  const int rows = ig::kPairPix / w;
  if (h % rows != 0) return false;
  if ((rows + 4) * (w + 2) * (c / 16) > ig::kPairFill * 256) return false;
  const int pb1 = pair_pb1(w, rows);
  if (!(pb1 == 6 || pb1 == 7 || pb1 == 8 || (pb1 == 10 && c <= 32))) return false;
  if ((long long)a1.n * h * w * a1.x_pix_stride >= (1ll << 31)) return false;
  if ((long long)a1.n * h * w >= (1ll << 24)) return false;
  return ig::pair_lds_bytes(c, a1.ksteps, w, rows) <= 160 * 1024;
}

void launch_igemm_pair(hipStream_t st, const IgemmArgs& a1_in, const IgemmArgs& a2_in) {
  if (!igemm_pair_ok(a1_in, a2_in)) fail(-2, "igemm pair: unsupported shapes or views");
  ig::PairArgs p;
  p.a1 = a1_in;
  p.a2 = a2_in;
  const int w = p.a1.w, h = p.a1.h, c = p.a1.cin;
  p.rows = ig::kPairPix / w;
  p.a1.x_bytes = (int)((long long)p.a1.n * h * w * p.a1.x_pix_stride);
  p.a1.r_wo = 1.0f / (float)w;
  const int pb1 = pair_pb1(w, p.rows);
  const dim3 grid((unsigned)(p.a1.n * (h / p.rows)));
  const size_t lds = (size_t)ig::pair_lds_bytes(c, p.a1.ksteps, w, p.rows);
  const bool res = p.a2.res != nullptr;
#define DW_P(CB_, PB_)                                                                                   \
  if (c == 16 * (CB_) && pb1 == (PB_)) {                                                                \
    if (res)                                                                                            \
      hipLaunchKernelGGL((ig::igemm_pair_kernel<CB_, PB_, true>), grid, dim3(256), lds, st, p);        \
    else                                                                                                \
      hipLaunchKernelGGL((ig::igemm_pair_kernel<CB_, PB_, false>), grid, dim3(256), lds, st, p);       \
    DW_HIP(hipGetLastError());                                                                          \
    return;                                                                                             \
  }
  DW_P(1, 6) DW_P(1, 7) DW_P(1, 8) DW_P(1, 10)
  DW_P(2, 6) DW_P(2, 7) DW_P(2, 8) DW_P(2, 10)
  DW_P(4, 6) DW_P(4, 7) DW_P(4, 8)
#undef DW_P
  fail(-2, "igemm pair: no kernel for the shape");
}

}  // namespace dw
