// Classifier-head ops: Gemm (f32, f16, int8) with the reference's
// accumulation order, GlobalAveragePool and Softmax over rows.  These are
// small ops (a classifier's last layers: batch x 1280 -> 1000, a 7 x 7
// pool), so every output is one thread walking its sum in the reference
// order; the loads of each step are coalesced across the threads of a row
// of outputs.
#include "dw_common.h"
#include "dw_device.h"

namespace dw {
namespace {

// C[i][j] = sum over p of A[i][p] * B[p][j]: thread (i, j), j across the
// lanes (B rows coalesced, A[i][p] the same in every lane).  f32: fma chain
// from +0 in p order (gemm_f32_naive, ops.rs:273-290).  F16: operands
// widened with the reference decode (h2f), the same chain, f2h of the sum
// (gemm_fp16, ops.rs:461-479).  TB (the graph runtime's transposed path,
// onnx runtime.rs:1220-1233, :1256-1266): B is [n][k] and each step is a
// multiply then an add, each rounded.  bias (blen values): the stored sum
// plus bias[j % blen] (f32 add; f16: F16 of the widened sum).
template <bool F16, bool TB>
__global__ __launch_bounds__(256) void gemm_exact_kernel(const void* A, const void* B, void* Cm, int m, int n,
                                                         int k, const void* bias, int blen) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  const int i = blockIdx.y;
  if (j >= n || i >= m) return;
  float acc = 0.0f;
  const size_t bs = TB ? 1 : (size_t)n;  // B step along p
  const size_t b0 = TB ? (size_t)j * k : (size_t)j;
  if constexpr (F16) {
    const uint16_t* a = (const uint16_t*)A + (size_t)i * k;
    const uint16_t* b = (const uint16_t*)B + b0;
    for (int p = 0; p < k; ++p) {
      if constexpr (TB) {
        float prod = h2f(a[p]) * h2f(b[p * bs]);
        asm("" : "+v"(prod));  // rounded product, then the add
        acc = acc + prod;
      } else {
        acc = fmaf(h2f(a[p]), h2f(b[p * bs]), acc);
      }
    }
    uint16_t hb = f2h(acc);
    if (bias) hb = f16_add_bits(hb, ((const uint16_t*)bias)[j % blen]);
    ((uint16_t*)Cm)[(size_t)i * n + j] = hb;
  } else {
    const float* a = (const float*)A + (size_t)i * k;
    const float* b = (const float*)B + b0;
    for (int p = 0; p < k; ++p) {
      if constexpr (TB) {
        float prod = a[p] * b[p * bs];
        asm("" : "+v"(prod));
        acc = acc + prod;
      } else {
        acc = fmaf(a[p], b[p * bs], acc);
      }
    }
    if (bias) acc = acc + ((const float*)bias)[j % blen];
    ((float*)Cm)[(size_t)i * n + j] = acc;
  }
}

// int32 sum of i8 products (gemm_i8_scalar, ops.rs:2981-2995); integer
// addition wraps like the reference's release build, in any order.
__global__ __launch_bounds__(256) void gemm_i8_kernel(const int8_t* A, const int8_t* B, int32_t* Cm, int m, int n,
                                                      int k) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  const int i = blockIdx.y;
  if (j >= n || i >= m) return;
  const int8_t* a = A + (size_t)i * k;
  const int8_t* b = B + j;
  uint32_t acc = 0;
  for (int p = 0; p < k; ++p) acc += (uint32_t)((int32_t)a[p] * (int32_t)b[(size_t)p * n]);
  Cm[(size_t)i * n + j] = (int32_t)acc;
}

// NHWC global average pool (CpuGraphRuntime::dispatch_global_avg_pool,
// onnx runtime.rs:1109-1175): thread (batch, channel) sums its h x w values
// in row-major order in f32 and divides by h * w (correctly rounded); f16
// widens with the reference decode and rounds the mean to f16.
template <bool F16>
__global__ __launch_bounds__(256) void global_avg_pool_kernel(const void* X, void* Y, int n, int hw, int c) {
  const int ch = blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (ch >= c || b >= n) return;
  float sum = 0.0f;
  const size_t base = (size_t)b * hw * c + ch;
  if constexpr (F16) {
    const uint16_t* x = (const uint16_t*)X + base;
    for (int s = 0; s < hw; ++s) sum += h2f(x[(size_t)s * c]);
    ((uint16_t*)Y)[(size_t)b * c + ch] = f2h(__fdiv_rn(sum, (float)hw));
  } else {
    const float* x = (const float*)X + base;
    for (int s = 0; s < hw; ++s) sum += x[(size_t)s * c];
    ((float*)Y)[(size_t)b * c + ch] = __fdiv_rn(sum, (float)hw);
  }
}

// Softmax over rows of n (softmax_f32, ops.rs:1609-1638), one thread per
// row: the max from -inf (fmaxf: a NaN operand loses, as f32::max), e =
// exp(x - max), the sum in order, out = e * (1 / sum).  exp is the device
// expf, so outputs agree with the host's to within a few ulps.  The f16 form
// (CpuGraphRuntime::dispatch_softmax, runtime.rs:1311-1322) widens every
// input with the reference decode, runs the f32 softmax and rounds each
// output once to f16.
template <bool H>
__global__ __launch_bounds__(256) void softmax_rows_kernel(const void* X, void* Y, int rows, int n) {
  const int r = blockIdx.x * 256 + threadIdx.x;
  if (r >= rows) return;
  auto ld = [&](int i) -> float {
    if (H) return h2f(((const uint16_t*)X)[(size_t)r * n + i]);
    return ((const float*)X)[(size_t)r * n + i];
  };
  float mx = -INFINITY;
  for (int i = 0; i < n; ++i) mx = fmaxf(mx, ld(i));
  float sum = 0.0f;
  for (int i = 0; i < n; ++i) sum += expf(ld(i) - mx);
  const float inv = __fdiv_rn(1.0f, sum);
  for (int i = 0; i < n; ++i) {
    const float v = expf(ld(i) - mx) * inv;
    if (H)
      ((uint16_t*)Y)[(size_t)r * n + i] = f2h(v);
    else
      ((float*)Y)[(size_t)r * n + i] = v;
  }
}

// QLinearGlobalAveragePool over NHWC u8: thread (batch, channel) sums its
// h x w values minus the input zero point as an int32, then
// y = clamp(rint((float)sum * M) + y_zp, 0, 255) with M = (x_scale / y_scale)
// / (h * w) in f32 (rint: round half to even).
__global__ __launch_bounds__(256) void qlinear_gap_kernel(const uint8_t* X, uint8_t* Y, int n, int hw, int c,
                                                          int x_zp, float m, int y_zp) {
  const int ch = blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (ch >= c || b >= n) return;
  const uint8_t* x = X + (size_t)b * hw * c + ch;
  int acc = 0;
  for (int s = 0; s < hw; ++s) acc += (int)x[(size_t)s * c] - x_zp;
  float q = rintf((float)acc * m) + (float)y_zp;
  q = fminf(fmaxf(q, 0.0f), 255.0f);
  Y[(size_t)b * c + ch] = (uint8_t)q;
}

// dst[c][r] = src[r][c] for a rows x cols byte matrix (32 x 32 tiles through LDS).
__global__ __launch_bounds__(256) void transpose_u8_kernel(const uint8_t* src, uint8_t* dst, int rows, int cols) {
  __shared__ uint8_t t[32][33];
  const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int k = ty; k < 32; k += 8) {
    const int r = r0 + k, c = c0 + tx;
    if (r < rows && c < cols) t[k][tx] = src[(size_t)r * cols + c];
  }
  __syncthreads();
  for (int k = ty; k < 32; k += 8) {
    const int c = c0 + k, r = r0 + tx;
    if (r < rows && c < cols) dst[(size_t)c * rows + r] = t[tx][k];
  }
}

}  // namespace

void launch_gemm_ex(hipStream_t st, int dtype, const void* a, const void* b, void* c, int m, int n, int k,
                    bool trans_b, const void* bias, int blen) {
  if (m > 65535) fail(-2, "gemm: more than 65535 rows");
  const dim3 g((unsigned)((n + 255) / 256), (unsigned)m);
  if (dtype == F32 && !trans_b)
    hipLaunchKernelGGL((gemm_exact_kernel<false, false>), g, dim3(256), 0, st, a, b, c, m, n, k, bias, blen);
  else if (dtype == F32)
    hipLaunchKernelGGL((gemm_exact_kernel<false, true>), g, dim3(256), 0, st, a, b, c, m, n, k, bias, blen);
  else if (dtype == F16 && !trans_b)
    hipLaunchKernelGGL((gemm_exact_kernel<true, false>), g, dim3(256), 0, st, a, b, c, m, n, k, bias, blen);
  else if (dtype == F16)
    hipLaunchKernelGGL((gemm_exact_kernel<true, true>), g, dim3(256), 0, st, a, b, c, m, n, k, bias, blen);
  else
    fail(-2, "gemm: dtype");
  DW_HIP(hipGetLastError());
}

void launch_gemm(hipStream_t st, int dtype, const void* a, const void* b, void* c, int m, int n, int k) {
  const dim3 g((unsigned)((n + 255) / 256), (unsigned)m);
  if (dtype == F32 || dtype == F16)
    return launch_gemm_ex(st, dtype, a, b, c, m, n, k, false, nullptr, 1);
  if (dtype == I8)
    hipLaunchKernelGGL(gemm_i8_kernel, g, dim3(256), 0, st, (const int8_t*)a, (const int8_t*)b, (int32_t*)c, m, n,
                       k);
  else
    fail(-2, "gemm: dtype");
  DW_HIP(hipGetLastError());
}

void launch_global_avg_pool(hipStream_t st, int dtype, const void* x, void* y, int n, int hw, int c) {
  const dim3 g((unsigned)((c + 255) / 256), (unsigned)n);
  if (dtype == F32)
    hipLaunchKernelGGL((global_avg_pool_kernel<false>), g, dim3(256), 0, st, x, y, n, hw, c);
  else if (dtype == F16)
    hipLaunchKernelGGL((global_avg_pool_kernel<true>), g, dim3(256), 0, st, x, y, n, hw, c);
  else
    fail(-2, "global average pool: dtype");
  DW_HIP(hipGetLastError());
}

void launch_softmax_rows(hipStream_t st, const float* x, float* y, int rows, int n) {
  launch_softmax_rows_t(st, F32, x, y, rows, n);
}

void launch_softmax_rows_t(hipStream_t st, int dtype, const void* x, void* y, int rows, int n) {
  const dim3 g((unsigned)((rows + 255) / 256));
  if (dtype == F32)
    hipLaunchKernelGGL(softmax_rows_kernel<false>, g, dim3(256), 0, st, x, y, rows, n);
  else if (dtype == F16)
    hipLaunchKernelGGL(softmax_rows_kernel<true>, g, dim3(256), 0, st, x, y, rows, n);
  else
    fail(-2, "softmax: dtype");
  DW_HIP(hipGetLastError());
}

}  // namespace dw

namespace dw {

void launch_qlinear_gap(hipStream_t st, const uint8_t* x, uint8_t* y, int n, int hw, int c, int x_zp, float m,
                        int y_zp) {
  const dim3 g((unsigned)((c + 255) / 256), (unsigned)n);
  hipLaunchKernelGGL(qlinear_gap_kernel, g, dim3(256), 0, st, x, y, n, hw, c, x_zp, m, y_zp);
  DW_HIP(hipGetLastError());
}

void launch_transpose_u8(hipStream_t st, const void* src, void* dst, int rows, int cols) {
  const dim3 g((unsigned)((cols + 31) / 32), (unsigned)((rows + 31) / 32));
  hipLaunchKernelGGL(transpose_u8_kernel, g, dim3(256), 0, st, (const uint8_t*)src, (uint8_t*)dst, rows, cols);
  DW_HIP(hipGetLastError());
}

}  // namespace dw
