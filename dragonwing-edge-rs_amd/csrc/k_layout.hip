// Layout and graph-boundary kernels.
//
// transpose_tile_kernel: per batch entry, dst[col][row] = src[row][col] for
// a rows x cols matrix, through 32 x 32 LDS tiles so that both the loads and
// the stores are coalesced.  NCHW -> NHWC is rows = C, cols = H*W
// (transpose_nchw_to_nhwc, onnx graph.rs:339-356); NHWC -> NCHW is
// rows = H*W, cols = C (transpose_nhwc_to_nchw, graph.rs:358-379).  The f32
// -> f16 form rounds each value as F16::from_f32 does (dtype.rs:164-222), so
// an NCHW f32 input lands in an f16 NHWC graph input exactly as the host
// conversion would put it there; the destination may be a channel-strided
// view (dst_stride elements per pixel).
//
// fold_bn_kernel: fold_batchnorm (graph.rs:521-690) on device-resident
// weights, in f64 as the reference computes it: per output channel
// s = gamma / sqrt(var + eps), w' = (f32)(w * s), b' = (f32)((b - mean) * s +
// beta).  sqrt and the division are IEEE double operations, so the result is
// the reference's to the bit.
#include <algorithm>

#include "dw_common.h"
#include "dw_device.h"

namespace dw {
namespace {

template <typename TI, typename TO>
__device__ __forceinline__ TO convert_elem(TI v) {
  if constexpr (sizeof(TO) == 2 && sizeof(TI) == 4)
    return (TO)f2h(v);
  else
    return (TO)v;
}

template <typename TI, typename TO>
__global__ __launch_bounds__(256) void transpose_tile_kernel(const TI* src, TO* dst, int rows, int cols,
                                                             long long src_batch, long long dst_batch,
                                                             int dst_row_stride, int dst_off) {
  __shared__ TI t[32][33];
  const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
  const long long b = blockIdx.z;
  const TI* s = src + b * src_batch;
  TO* d = dst + b * dst_batch;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int k = ty; k < 32; k += 8) {
    const int r = r0 + k, c = c0 + tx;
    if (r < rows && c < cols) t[k][tx] = s[(size_t)r * cols + c];
  }
  __syncthreads();
  // dst is [cols][rows] with dst_row_stride elements between its rows
  for (int k = ty; k < 32; k += 8) {
    const int c = c0 + k, r = r0 + tx;
    if (r < rows && c < cols) d[(size_t)c * dst_row_stride + dst_off + r] = convert_elem<TI, TO>(t[tx][k]);
  }
}

__global__ __launch_bounds__(256) void fold_bn_kernel(const float* w, const float* bias_in, const float* gamma,
                                                      const float* beta, const float* mean, const float* var,
                                                      float eps, int c_out, int per, float* w_out,
                                                      float* b_out) {
  const int c = blockIdx.y;
  const double sf = (double)gamma[c] * (1.0 / sqrt((double)var[c] + (double)eps));
  for (int k = blockIdx.x * 256 + threadIdx.x; k < per; k += gridDim.x * 256)
    w_out[(size_t)c * per + k] = (float)((double)w[(size_t)c * per + k] * sf);
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    const double ob = bias_in ? (double)bias_in[c] : 0.0;
    b_out[c] = (float)((ob - (double)mean[c]) * sf + (double)beta[c]);
  }
}

template <typename TI, typename TO>
void launch_tt(hipStream_t st, const void* src, void* dst, int batch, int rows, int cols, int dst_row_stride,
               int dst_off, long long dst_batch) {
  const dim3 g((unsigned)((cols + 31) / 32), (unsigned)((rows + 31) / 32), (unsigned)batch);
  hipLaunchKernelGGL((transpose_tile_kernel<TI, TO>), g, dim3(256), 0, st, (const TI*)src, (TO*)dst, rows, cols,
                     (long long)rows * cols, dst_batch, dst_row_stride, dst_off);
  DW_HIP(hipGetLastError());
}

}  // namespace

void launch_transpose(hipStream_t st, const void* src, void* dst, int batch, int rows, int cols, int esize) {
  const long long db = (long long)rows * cols;
  if (esize == 4)
    launch_tt<uint32_t, uint32_t>(st, src, dst, batch, rows, cols, rows, 0, db);
  else if (esize == 2)
    launch_tt<uint16_t, uint16_t>(st, src, dst, batch, rows, cols, rows, 0, db);
  else if (esize == 1)
    launch_tt<uint8_t, uint8_t>(st, src, dst, batch, rows, cols, rows, 0, db);
  else
    fail(-2, "transpose: element size");
}

void launch_nchw_f32_to_nhwc(hipStream_t st, const float* src, void* dst, int n, int c, int hw, int out_dtype,
                             int pix_stride, int c_off) {
  const long long db = (long long)hw * pix_stride;
  if (out_dtype == F32)
    launch_tt<float, float>(st, src, dst, n, c, hw, pix_stride, c_off, db);
  else if (out_dtype == F16)
    launch_tt<float, uint16_t>(st, src, dst, n, c, hw, pix_stride, c_off, db);
  else
    fail(-2, "NCHW input: f32 or f16 destination");
}

void launch_fold_batchnorm(hipStream_t st, const float* w, const float* bias_in, const float* gamma,
                           const float* beta, const float* mean, const float* var, float eps, int c_out, int per,
                           float* w_out, float* b_out) {
  const dim3 g((unsigned)std::min(64, (per + 255) / 256), (unsigned)c_out);
  hipLaunchKernelGGL(fold_bn_kernel, g, dim3(256), 0, st, w, bias_in, gamma, beta, mean, var, eps, c_out, per,
                     w_out, b_out);
  DW_HIP(hipGetLastError());
}

}  // namespace dw
