// Layout and broadcasting kernels for the ops an exported model's tail uses
// (Transpose, Slice, Concat / Split along a non-channel axis, the layout
// changes around Reshape, Add / Sub / Mul / Div with broadcasting) and
// AveragePool.  All are HBM-bound byte movers with no matrix work.
//
// Every tensor is addressed as a rank-4 index space (lower ranks padded with
// leading 1s) with an element stride per axis, so one kernel covers any
// permutation, slice, or concat placement:
//   y[off_y + sum i_k ys_k] = x[off_x + sum i_k xs_k],  0 <= i_k < d_k.
// The reference runs Transpose and Slice of f16 tensors through f32
// (runtime.rs:2073-2084, :2130-2140): F16::from_f32(to_f32(v)), which is the
// identity except that subnormals come back at half their value (the
// decode's one-binade-low exponent) and NaN payloads are re-encoded; with
// F16RT set the copy applies the same round trip.
#include "dw_common.h"
#include "dw_device.h"

namespace dw {
namespace {

// index i (row-major over d) -> the four coordinates
__device__ __forceinline__ void coords(long long i, const long long (&d)[4], long long (&c)[4]) {
  c[3] = i % d[3];
  i /= d[3];
  c[2] = i % d[2];
  i /= d[2];
  c[1] = i % d[1];
  c[0] = i / d[1];
}

template <int ES, bool F16RT>
__global__ __launch_bounds__(256) void strided_copy_kernel(const StridedCopyArgs a, long long total) {
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long long)gridDim.x * 256) {
    long long c[4];
    coords(i, a.dims, c);
    const long long xo = a.x_off + c[0] * a.xs[0] + c[1] * a.xs[1] + c[2] * a.xs[2] + c[3] * a.xs[3];
    const long long yo = a.y_off + c[0] * a.ys[0] + c[1] * a.ys[1] + c[2] * a.ys[2] + c[3] * a.ys[3];
    if constexpr (ES == 1) {
      ((uint8_t*)a.y)[yo] = ((const uint8_t*)a.x)[xo];
    } else if constexpr (ES == 2) {
      uint16_t v = ((const uint16_t*)a.x)[xo];
      if constexpr (F16RT) v = f2h(h2f(v));
      ((uint16_t*)a.y)[yo] = v;
    } else {
      ((uint32_t*)a.y)[yo] = ((const uint32_t*)a.x)[xo];
    }
  }
}

// Add / Sub / Mul / Div with broadcasting: y over dims from a and b, each
// addressed by its own strides (0 along a broadcast axis).
// f32: one IEEE operation (add_f32 / sub_f32 / mul_f32 / div_f32,
// ops.rs:363-384, :1899-1919, :1978-2003, :2057-2082; division correctly
// rounded).  f16: F16::from_f32(to_f32(a) op to_f32(b)) (add_fp16,
// mul_fp16, sub_fp16, div_fp16, ops.rs:434-442, :1959-1967, :2038-2046,
// :2117-2125, and the broadcast loops of runtime.rs:1045-1860).
template <int OP, bool F16>
__global__ __launch_bounds__(256) void broadcast_binary_kernel(const BinaryArgs a, long long total) {
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long long)gridDim.x * 256) {
    long long c[4];
    coords(i, a.dims, c);
    const long long ao = a.a_off + c[0] * a.as[0] + c[1] * a.as[1] + c[2] * a.as[2] + c[3] * a.as[3];
    const long long bo = a.b_off + c[0] * a.bs[0] + c[1] * a.bs[1] + c[2] * a.bs[2] + c[3] * a.bs[3];
    const long long yo = a.y_off + c[0] * a.ys[0] + c[1] * a.ys[1] + c[2] * a.ys[2] + c[3] * a.ys[3];
    float x, y;
    if constexpr (F16) {
      x = h2f(((const uint16_t*)a.a)[ao]);
      y = h2f(((const uint16_t*)a.b)[bo]);
    } else {
      x = ((const float*)a.a)[ao];
      y = ((const float*)a.b)[bo];
    }
    float r;
    if constexpr (OP == BIN_ADD) r = x + y;
    else if constexpr (OP == BIN_SUB) r = x - y;
    else if constexpr (OP == BIN_MUL) r = x * y;
    else r = x / y;
    if constexpr (F16)
      ((uint16_t*)a.y)[yo] = f2h(r);
    else
      ((float*)a.y)[yo] = r;
  }
}

// avgpool2d_f32_nhwc (ops.rs:1556-1595): unpadded window; the sum runs over
// ph then pw in f32, then one division by kh * kw.  f16 tensors widen every
// value with to_f32 and store F16::from_f32 of the average
// (runtime.rs:1571-1630).
template <bool F16>
__global__ __launch_bounds__(256) void avgpool_kernel(const AvgPoolArgs a, long long total) {
  const float area = (float)(a.kh * a.kw);
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long long)gridDim.x * 256) {
    const int ch = (int)(i % a.c);
    long long p = i / a.c;
    const int ow = (int)(p % a.wo);
    p /= a.wo;
    const int oh = (int)(p % a.ho);
    const long long n = p / a.ho;
    float s = 0.0f;
    for (int ph = 0; ph < a.kh; ++ph)
      for (int pw = 0; pw < a.kw; ++pw) {
        const long long idx = ((n * a.h + oh * a.sh + ph) * a.w + ow * a.sw + pw) * a.c + ch;
        s += F16 ? h2f(((const uint16_t*)a.x)[idx]) : ((const float*)a.x)[idx];
      }
    const float r = s / area;
    if constexpr (F16)
      ((uint16_t*)a.y)[i] = f2h(r);
    else
      ((float*)a.y)[i] = r;
  }
}

unsigned grid_for(long long total) {
  const long long g = (total + 255) / 256;
  return (unsigned)(g < 8192 ? (g > 0 ? g : 1) : 8192);
}

}  // namespace

void launch_strided_copy(hipStream_t st, const StridedCopyArgs& a) {
  const long long total = a.dims[0] * a.dims[1] * a.dims[2] * a.dims[3];
  if (total <= 0) return;
  const dim3 grid(grid_for(total));
  if (a.esize == 1)
    hipLaunchKernelGGL((strided_copy_kernel<1, false>), grid, dim3(256), 0, st, a, total);
  else if (a.esize == 2 && a.f16_round_trip)
    hipLaunchKernelGGL((strided_copy_kernel<2, true>), grid, dim3(256), 0, st, a, total);
  else if (a.esize == 2)
    hipLaunchKernelGGL((strided_copy_kernel<2, false>), grid, dim3(256), 0, st, a, total);
  else if (a.esize == 4)
    hipLaunchKernelGGL((strided_copy_kernel<4, false>), grid, dim3(256), 0, st, a, total);
  else
    fail(-2, "strided copy: element size");
  DW_HIP(hipGetLastError());
}

void launch_broadcast_binary(hipStream_t st, const BinaryArgs& a) {
  const long long total = a.dims[0] * a.dims[1] * a.dims[2] * a.dims[3];
  if (total <= 0) return;
  const dim3 grid(grid_for(total));
#define DW_BIN(OP_)                                                                                   \
  if (a.f16)                                                                                          \
    hipLaunchKernelGGL((broadcast_binary_kernel<OP_, true>), grid, dim3(256), 0, st, a, total);       \
  else                                                                                                \
    hipLaunchKernelGGL((broadcast_binary_kernel<OP_, false>), grid, dim3(256), 0, st, a, total);
  switch (a.op) {
    case BIN_ADD: DW_BIN(BIN_ADD) break;
    case BIN_SUB: DW_BIN(BIN_SUB) break;
    case BIN_MUL: DW_BIN(BIN_MUL) break;
    case BIN_DIV: DW_BIN(BIN_DIV) break;
    default: fail(-2, "broadcast binary: op");
  }
#undef DW_BIN
  DW_HIP(hipGetLastError());
}

void launch_avgpool(hipStream_t st, const AvgPoolArgs& a) {
  const long long total = (long long)a.n * a.ho * a.wo * a.c;
  if (total <= 0) return;
  const dim3 grid(grid_for(total));
  if (a.f16)
    hipLaunchKernelGGL((avgpool_kernel<true>), grid, dim3(256), 0, st, a, total);
  else
    hipLaunchKernelGGL((avgpool_kernel<false>), grid, dim3(256), 0, st, a, total);
  DW_HIP(hipGetLastError());
}

}  // namespace dw
