// Depthwise 3x3 convolution, stride 1, padding 1, fp16 NHWC, with bias and
// activation, held to the fp16 tolerance: the bandwidth-bound path of the
// fp16 graphs.  (dwconv3_f16_kernel in k_direct.hip is the reference-order
// alternative, bit-exact before the activation.)
//
// A workgroup owns one image, a band of RB output rows, every column and a
// channel slice of 32 or 64 channels (4 or 8 16-byte units of 8 channels);
// one thread per (column, unit).  Each thread loads its column of the RB + 2
// input rows (all loads in flight at once; consecutive threads read one
// pixel's 64 or 128 contiguous bytes) into LDS, with zeros for the padding
// rows and the two padding columns, then computes its column and unit down
// the band from a 3 x 3 window of units held in registers (one new row of
// three units read from LDS per output row).  Tiles stay under 64 KB of LDS
// so several workgroups share a CU and their load and compute phases
// overlap; the runtime's tuner picks the slice width and band height.  Global traffic is the input once plus the band
// halo ((RB + 2) / RB) and the output once, with dense 16-byte stores.
//
// Arithmetic: the nine taps as packed f16 FMAs in the reference's kh, kw
// order, then the f16 bias add and the activation on packed f16 (SiLU with
// the hardware's f16 exp2 and rcp), two channels per instruction.  Rounding to f16
// after every tap instead of once after an f32 chain moves a result by a
// few f16 ulps of the partial sums, far inside the 1e-2 bar.
#include "dw_common.h"
#include "dw_device.h"

#include <algorithm>

namespace dw {
namespace {

__device__ __forceinline__ h16x2 as_h2(uint32_t v) { return __builtin_bit_cast(h16x2, v); }
__device__ __forceinline__ uint32_t as_u(h16x2 v) { return __builtin_bit_cast(uint32_t, v); }

__device__ __forceinline__ uint4 fma_unit(uint4 x, uint4 w, uint4 acc) {
  acc.x = as_u(__builtin_elementwise_fma(as_h2(x.x), as_h2(w.x), as_h2(acc.x)));
  acc.y = as_u(__builtin_elementwise_fma(as_h2(x.y), as_h2(w.y), as_h2(acc.y)));
  acc.z = as_u(__builtin_elementwise_fma(as_h2(x.z), as_h2(w.z), as_h2(acc.z)));
  acc.w = as_u(__builtin_elementwise_fma(as_h2(x.w), as_h2(w.w), as_h2(acc.w)));
  return acc;
}

// SiLU of two f16 values entirely in f16: x * rcp(1 + 2^(-x log2 e)) with
// the hardware's f16 exp2 and rcp (each within an f16 ulp), no conversions
// to f32; the sigmoid then carries a few f16 ulps, inside the fp16 bar.
__device__ __forceinline__ h16x2 silu_h16(h16x2 x) {
  const h16x2 t = x * h16x2{(_Float16)-1.44269504f, (_Float16)-1.44269504f};
  h16x2 e;
  e[0] = __builtin_exp2f16(t[0]);
  e[1] = __builtin_exp2f16(t[1]);
  const h16x2 d = e + h16x2{(_Float16)1.0f, (_Float16)1.0f};
  h16x2 r;
  r[0] = __builtin_amdgcn_rcph(d[0]);
  r[1] = __builtin_amdgcn_rcph(d[1]);
  return x * r;
}

template <int ACT>
__device__ __forceinline__ uint32_t finish2(uint32_t acc, uint32_t b) {
  h16x2 v = as_h2(acc) + as_h2(b);
  if constexpr (ACT == ACT_SILU) v = silu_h16(v);
  if constexpr (ACT == ACT_RELU) v = __builtin_elementwise_max(v, h16x2{0, 0});
  return as_u(v);
}

// UNITS: 16-byte units (8 channels) of the workgroup's channel slice; one
// thread per (column, unit), blockDim = W * UNITS.  RB: output rows per band.
template <int UNITS, int RB, int ACT>
__global__ __launch_bounds__(1024) void dwconv3_tile_kernel(const DwArgs a, int bands, int slices) {
  constexpr int kMaxBand = RB;
  const int rb = RB;
  extern __shared__ __attribute__((aligned(16))) uint4 tile[];  // [(rb + 2)][(w + 2)][UNITS]
  const int W = a.w, H = a.h, TW = W + 2;
  const int tid = threadIdx.x;
  const int u = tid % UNITS;
  const int col = tid / UNITS;
  int b = blockIdx.x;
  const int slice = b % slices;
  b /= slices;
  const int band = b % bands;
  const int n = b / bands;
  const int r0 = band * rb;
  const int rows = min(rb, H - r0);  // output rows of this band
  const int c0 = slice * (UNITS * 8);  // first channel of the slice

  // ---- this thread's column of the input rows r0 - 1 .. r0 + rows, all
  // loads in flight before the first LDS store (zeros outside the image)
  const uint8_t* xcol = (const uint8_t*)a.x + ((size_t)((size_t)n * H * W + col) * a.x_pix_stride + a.x_c_off +
                                               c0 + u * 8) * 2;
  const size_t row_bytes = (size_t)W * a.x_pix_stride * 2;
  uint4 v[kMaxBand + 2];
#pragma unroll
  for (int tr = 0; tr < kMaxBand + 2; ++tr) {
    const int row = r0 - 1 + tr;
    v[tr] = make_uint4(0, 0, 0, 0);
    if (tr < rows + 2 && row >= 0 && row < H) v[tr] = *reinterpret_cast<const uint4*>(xcol + row * row_bytes);
  }
#pragma unroll
  for (int tr = 0; tr < kMaxBand + 2; ++tr)
    if (tr < rows + 2) tile[(tr * TW + col + 1) * UNITS + u] = v[tr];
  if (col < 2)  // the padding columns
    for (int tr = 0; tr < rows + 2; ++tr) tile[(tr * TW + (col ? W + 1 : 0)) * UNITS + u] = make_uint4(0, 0, 0, 0);
  __syncthreads();

  // ---- one column and one unit per thread, down the band
  const uint16_t* wt = (const uint16_t*)a.wt;
  uint4 wk[9];
#pragma unroll
  for (int k = 0; k < 9; ++k) wk[k] = *reinterpret_cast<const uint4*>(wt + (size_t)k * a.c + c0 + u * 8);
  const uint4 bias = a.bias ? *reinterpret_cast<const uint4*>((const uint16_t*)a.bias + c0 + u * 8)
                            : make_uint4(0, 0, 0, 0);
  auto ld = [&](int tr, int dc) { return tile[(tr * TW + col + dc) * UNITS + u]; };
  uint4 x0[3], x1[3], x2[3];
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    x0[d] = ld(0, d);
    x1[d] = ld(1, d);
  }
  uint8_t* ycol = (uint8_t*)a.y + ((size_t)((size_t)n * H * W + (size_t)r0 * W + col) * a.y_pix_stride + a.y_c_off +
                                   c0 + u * 8) * 2;
  const size_t yrow_bytes = (size_t)W * a.y_pix_stride * 2;
  for (int r = 0; r < rows; ++r) {
#pragma unroll
    for (int d = 0; d < 3; ++d) x2[d] = ld(r + 2, d);
    uint4 acc = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int d = 0; d < 3; ++d) acc = fma_unit(x0[d], wk[d], acc);
#pragma unroll
    for (int d = 0; d < 3; ++d) acc = fma_unit(x1[d], wk[3 + d], acc);
#pragma unroll
    for (int d = 0; d < 3; ++d) acc = fma_unit(x2[d], wk[6 + d], acc);
    uint4 o;
    o.x = finish2<ACT>(acc.x, bias.x);
    o.y = finish2<ACT>(acc.y, bias.y);
    o.z = finish2<ACT>(acc.z, bias.z);
    o.w = finish2<ACT>(acc.w, bias.w);
    *reinterpret_cast<uint4*>(ycol + r * yrow_bytes) = o;
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      x0[d] = x1[d];
      x1[d] = x2[d];
    }
  }
}

}  // namespace

bool dwconv3_tile_ok(const DwArgs& a) {
  const bool al16 = (uintptr_t)a.x % 16 == 0 && (uintptr_t)a.y % 16 == 0 && (uintptr_t)a.wt % 16 == 0 &&
                    (uintptr_t)a.bias % 16 == 0 && (a.x_pix_stride * 2) % 16 == 0 && (a.x_c_off * 2) % 16 == 0 &&
                    (a.y_pix_stride * 2) % 16 == 0 && (a.y_c_off * 2) % 16 == 0;
  return a.kh == 3 && a.kw == 3 && a.sh == 1 && a.sw == 1 && a.pt == 1 && a.pl == 1 && a.ho == a.h &&
         a.wo == a.w && a.c % 32 == 0 && a.w >= 2 && a.w * 4 <= 1024 && al16 &&
         (long long)a.n * a.h * a.w * a.x_pix_stride < (1ll << 31) &&
         (long long)a.n * a.h * a.w * a.y_pix_stride < (1ll << 31);
}

bool dwconv3_tile_cfg_ok(const DwArgs& a, int units, int band_rows) {
  return dwconv3_tile_ok(a) && (units == 4 || units == 8) && a.c % (units * 8) == 0 && a.w * units <= 1024 &&
         (band_rows == 4 || band_rows == 8 || band_rows == 10 || band_rows == 20) && band_rows <= a.h &&
         (size_t)(band_rows + 2) * (a.w + 2) * units * 16 <= 64 * 1024;
}

void launch_dwconv3_tile(hipStream_t st, const DwArgs& a, int units, int band_rows) {
  if (!dwconv3_tile_cfg_ok(a, units, band_rows)) fail(-2, "depthwise tile: unsupported shape, alignment or tile");
  const int rb = band_rows;
  const int bands = (a.h + rb - 1) / rb;
  const int slices = a.c / (units * 8);
  const int threads = a.w * units;
  const size_t lds = (size_t)(rb + 2) * (a.w + 2) * units * 16;
  const dim3 grid((unsigned)((long long)a.n * bands * slices));
#define DW_DWT(U_, RB_, ACT_) \
  hipLaunchKernelGGL((dwconv3_tile_kernel<U_, RB_, ACT_>), grid, dim3(threads), lds, st, a, bands, slices)
#define DW_DWT_ACT(U_, RB_)                   \
  if (a.act == ACT_SILU) DW_DWT(U_, RB_, ACT_SILU); \
  else if (a.act == ACT_RELU) DW_DWT(U_, RB_, ACT_RELU); \
  else DW_DWT(U_, RB_, ACT_NONE);
#define DW_DWT_RB(U_)                     \
  if (rb == 4) { DW_DWT_ACT(U_, 4) }      \
  else if (rb == 8) { DW_DWT_ACT(U_, 8) } \
  else if (rb == 10) { DW_DWT_ACT(U_, 10) } \
  else { DW_DWT_ACT(U_, 20) }
  if (units == 8) {
    DW_DWT_RB(8)
  } else {
    DW_DWT_RB(4)
  }
#undef DW_DWT_RB
#undef DW_DWT_ACT
#undef DW_DWT
  DW_HIP(hipGetLastError());
}

}  // namespace dw
