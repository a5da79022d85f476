// A whole int8 C2f block with one bottleneck in one launch (igemm_c2f.h):
// shape and view checks, band heights, launch geometry, instantiations.
#include "igemm_c2f.h"

namespace dw {
namespace {

bool conv_is(const IgemmArgs& a, int k, int pad) {
  return a.kh == k && a.kw == k && a.sh == 1 && a.sw == 1 && a.pt == pad && a.pl == pad && a.ho == a.h && a.wo == a.w;
}

bool table_epilogue(const IgemmArgs& a) {
  return a.epi == EPI_QU8 && a.lut && a.bias_i && !a.h_wfrag && a.cout % 4 == 0;
}

}  // namespace

bool igemm_c2f_shapes_ok(const IgemmArgs& a0, const IgemmArgs& a1, const IgemmArgs& a2, const IgemmArgs& a3) {
  const int c = a1.cin;
  if (!(c == 16 || c == 32)) return false;
  // cv1: 1x1, c1 -> 2c, at most 2 k-steps (c = 16) or 3 (c = 32)
  if (!conv_is(a0, 1, 0) || !table_epilogue(a0) || a0.res || a0.cout != 2 * c || a0.cout_pad != 2 * c) return false;
  if (a0.cin % 16 != 0 || a0.x_pix_stride % 16 != 0 || a0.x_c_off % 16 != 0) return false;
  if (a0.ksteps != (a0.cin + 63) / 64 || a0.ksteps > (c == 16 ? 2 : 3)) return false;
  // the bottleneck: two 3x3 convs, c -> c
  for (const IgemmArgs* a : {&a1, &a2})
    if (!conv_is(*a, 3, 1) || !table_epilogue(*a) || a->cin != c || a->cout != c || a->cout_pad < c ||
        a->ksteps != (9 * c + 63) / 64)
      return false;
  if (a1.res) return false;
  // cv2: 1x1, 3c -> 2c (the YOLOv8 C2f widths), no shortcut of its own
  if (!conv_is(a3, 1, 0) || !table_epilogue(a3) || a3.res || a3.cin != 3 * c || a3.cout != 2 * c ||
      a3.cout_pad != a3.cout || a3.ksteps != (3 * c + 63) / 64)
    return false;
  if (a3.y_pix_stride % 4 != 0 || a3.y_c_off % 4 != 0) return false;
  // views: y at channels [o, o + 2c) of the block's concat, y1 = its second
  // half, t read by m.cv2 only, z at [o + 2c, o + 3c), cv2 reading [o, o + 3c)
  const uint8_t* cat = (const uint8_t*)a0.y;
  const int o = a0.y_c_off, ps = a0.y_pix_stride;
  if (a1.x != cat || a1.x_pix_stride != ps || a1.x_c_off != o + c) return false;
  if (a2.x != (const uint8_t*)a1.y || a2.x_pix_stride != a1.y_pix_stride || a2.x_c_off != a1.y_c_off) return false;
  if (a2.res && (a2.res != (const void*)cat || a2.r_pix_stride != ps || a2.r_c_off != o + c)) return false;
  if ((const uint8_t*)a2.y != cat || a2.y_pix_stride != ps || a2.y_c_off != o + 2 * c) return false;
  if (a3.x != cat || a3.x_pix_stride != ps || a3.x_c_off != o) return false;
  // operands: u8 everywhere after the first conv
  if (a1.xxor != 0x80808080u || a3.xxor != 0x80808080u || a2.xxor != 0x80808080u) return false;
  for (const IgemmArgs* a : {&a1, &a2, &a3})
    if (a->n != a0.n || a->h != a0.h || a->w != a0.w) return false;
  if ((long long)a0.n * a0.h * a0.w >= (1ll << 24)) return false;
  return (long long)a0.n * a0.h * a0.w * a0.x_pix_stride < (1ll << 31);
}

bool igemm_c2f_ok(const IgemmArgs& a0, const IgemmArgs& a1, const IgemmArgs& a2, const IgemmArgs& a3, int rows) {
  if (!igemm_c2f_shapes_ok(a0, a1, a2, a3) || rows < 1 || a1.h % rows != 0) return false;
  const int c = a1.cin;
  return ig::c2f_layout(c, a3.cout, a0.ksteps, a1.ksteps, a3.ksteps, a1.w, rows).total <= 160 * 1024;
}

int igemm_c2f_rows(const IgemmArgs& a0, const IgemmArgs& a1, const IgemmArgs& a2, const IgemmArgs& a3, int* rows,
                   int max) {
  int n = 0;
  if (!igemm_c2f_shapes_ok(a0, a1, a2, a3)) return 0;
  // band heights giving at most 1024 workgroups, tallest first (least
  // halo); those giving fewer than 128 only when no height gives more
  bool many = false;
  for (int r = a1.h; r >= 1; --r)
    many |= a1.h % r == 0 && (long)a1.n * (a1.h / r) >= 128 && (long)a1.n * (a1.h / r) <= 1024 &&
            igemm_c2f_ok(a0, a1, a2, a3, r);
  for (int r = a1.h; r >= 1 && n < max; --r) {
    const long wgs = (long)a1.n * (a1.h / r);
    if (a1.h % r == 0 && wgs <= 1024 && (!many || wgs >= 128) && igemm_c2f_ok(a0, a1, a2, a3, r)) rows[n++] = r;
  }
  return n;
}

void launch_igemm_c2f(hipStream_t st, const IgemmArgs& a0, const IgemmArgs& a1, const IgemmArgs& a2,
                      const IgemmArgs& a3, int rows) {
  if (!igemm_c2f_ok(a0, a1, a2, a3, rows)) fail(-2, "igemm c2f: unsupported shapes, views or band height");
  ig::C2fArgs p;
  p.a0 = a0;
  p.a1 = a1;
  p.a2 = a2;
  p.a3 = a3;
  p.rows = rows;
  p.a0.x_bytes = (int)((long long)a0.n * a0.h * a0.w * a0.x_pix_stride);
  p.a1.r_wo = 1.0f / (float)a1.w;
  const int c = a1.cin;
  const dim3 grid((unsigned)(a1.n * (a1.h / rows)));
  const size_t lds = (size_t)ig::c2f_layout(c, a3.cout, a0.ksteps, a1.ksteps, a3.ksteps, a1.w, rows).total;
  const bool res = a2.res != nullptr;
  const int ks0 = a0.ksteps;
#define DW_C(CB_, KS0_)                                                                                   \
  if (c == 16 * (CB_) && ks0 == (KS0_)) {                                                                \
    if (res)                                                                                             \
      hipLaunchKernelGGL((ig::igemm_c2f_kernel<CB_, 2 * (CB_), KS0_, true>), grid, dim3(ig::kC2fThreads), lds, st, p); \
    else                                                                                                 \
      hipLaunchKernelGGL((ig::igemm_c2f_kernel<CB_, 2 * (CB_), KS0_, false>), grid, dim3(ig::kC2fThreads), lds, st, p); \
    DW_HIP(hipGetLastError());                                                                           \
    return;                                                                                              \
  }
  DW_C(1, 1) DW_C(1, 2) DW_C(2, 1) DW_C(2, 2) DW_C(2, 3)
#undef DW_C
  fail(-2, "igemm c2f: no kernel for the channel counts");
}

}  // namespace dw
