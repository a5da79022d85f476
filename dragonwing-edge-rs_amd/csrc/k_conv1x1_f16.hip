// 1x1 convolution (stride 1, no padding) with u8 input dequantized to f16,
// f16 weights and f16 output, on the fp16 matrix cores: the dequantized
// fp16 layers of a quantized graph (DequantizeLinear -> Conv, e.g. the last
// 1x1 convs of a YOLOv8 detect head).  Results are held to the fp16
// tolerance (the MFMA sums accumulate in f32 in another order than the
// CPU's fma chain); the reference-order kernel (k_direct1x1.hip) is the
// exact alternative.
//
// The GEMM is Y[c][p] = sum_k W[k][c] * X[p][k] with K = c_in.  Each MFMA
// (v_mfma_f32_16x16x32_f16) takes 16 output channels (operand A, rows) by
// 32 values of K, and 32 values of K by 16 pixels (operand B): lane l
// supplies row (l % 16) and K-slice 8 (l / 16) .. +7 of both.  A lane's 8
// input values are 8 consecutive u8 channels of one pixel (one 8-byte
// load), dequantized in registers as DequantizeLinear u8 -> f16 does:
// f16((q - zp) * scale), rounded to nearest even.
//
// A workgroup (4 waves) owns 256 consecutive pixels, a wave 64 of them (four
// 16-pixel blocks) and every output channel.  The weights, packed on the
// host in fragment order ([channel block][k-step][lane][8 f16]), are staged
// once per workgroup in LDS; all of a lane's input loads are issued before
// the workgroup waits for them, so the staging overlaps the input latency.
// The accumulator of block (cb, pb) holds channels cb*16 + 4 (l / 16) .. +3
// of pixel pb*16 + l % 16; the epilogue rounds them to f16, adds the f16
// bias, applies the activation (packed f16, as the other fp16 epilogues)
// and stores 8 bytes per lane and block.
#include "dw_common.h"
#include "dw_device.h"

namespace dw {
namespace {

typedef f16x8 v8h;
typedef f32x4 v4f;

template <int CB, int KS>
__global__ __launch_bounds__(256) void conv1x1_u8_f16_mfma_kernel(const Conv1x1F16Args a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint4* const s_w = reinterpret_cast<uint4*>(smem);                       // CB * KS * 64 fragments slices
  uint16_t* const s_bias = reinterpret_cast<uint16_t*>(smem + CB * KS * 1024);  // CB * 16 values

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int p0 = blockIdx.x * 256 + wave * 64;
  const int kq = (lane >> 4) * 8;  // this lane's K-slice within a k-step

  // input loads first: four pixel blocks x KS k-steps of 8 bytes
  uint2 raw[4][KS];
#pragma unroll
  for (int pb = 0; pb < 4; ++pb) {
    const int p = p0 + pb * 16 + (lane & 15);
    const uint8_t* row = a.x + (size_t)p * a.x_pix_stride + a.x_c_off;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int k = ks * 32 + kq;
      raw[pb][ks] = (p < a.m && k < a.cin) ? *reinterpret_cast<const uint2*>(row + k)
                                           : make_uint2(a.zp_bytes, a.zp_bytes);
    }
  }
  // weights and bias to LDS
  const uint4* wsrc = reinterpret_cast<const uint4*>(a.wfrag);
  for (int i = tid; i < CB * KS * 64; i += 256) s_w[i] = wsrc[i];
  if (tid < CB * 16) s_bias[tid] = (a.bias && tid < a.cout) ? a.bias[tid] : (uint16_t)0;
  __syncthreads();

  const float zp = (float)a.in_zp, scale = a.in_scale;
  v8h xf[4][KS];
#pragma unroll
  for (int pb = 0; pb < 4; ++pb)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) xf[pb][ks] = dequant_u8x8_f16(raw[pb][ks], zp, scale);
  // each weight fragment is read from LDS once and used for the four blocks
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    v8h wf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) wf[ks] = __builtin_bit_cast(v8h, s_w[(cb * KS + ks) * 64 + lane]);
    const int ch = cb * 16 + 4 * (lane >> 4);
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
      v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[ks], xf[pb][ks], acc, 0, 0, 0);
      const int p = p0 + pb * 16 + (lane & 15);
      if (p >= a.m || ch >= a.cout) continue;
      uint16_t* yrow = a.y + (size_t)p * a.y_pix_stride + a.y_c_off;
      *reinterpret_cast<uint2*>(yrow + ch) = conv1x1_f16_finish(acc, a.bias ? s_bias + ch : nullptr, a.act);
    }
  }
}

}  // namespace

bool conv1x1_u8_f16_supported(int cin, int cout) {
  const int cb = (cout + 15) / 16, ks = (cin + 31) / 32;
  return cin % 8 == 0 && cout % 4 == 0 && cb >= 1 && cb <= 8 && ks >= 1 && ks <= 4;
}

void launch_conv1x1_u8_f16(hipStream_t st, const Conv1x1F16Args& a) {
  if (!conv1x1_u8_f16_supported(a.cin, a.cout)) fail(-2, "conv1x1 u8->f16: unsupported channel counts");
  if (a.m <= 0) return;
  const int cb = (a.cout + 15) / 16, ks = (a.cin + 31) / 32;
  const size_t lds = (size_t)cb * ks * 1024 + cb * 32;
  const dim3 grid((a.m + 255) / 256);
#define DW_C1(CB_, KS_)                                                                          \
  case CB_ * 8 + KS_:                                                                            \
    hipLaunchKernelGGL((conv1x1_u8_f16_mfma_kernel<CB_, KS_>), grid, dim3(256), lds, st, a); \
    break;
#define DW_C1_KS(CB_) DW_C1(CB_, 1) DW_C1(CB_, 2) DW_C1(CB_, 3) DW_C1(CB_, 4)
  switch (cb * 8 + ks) {
    DW_C1_KS(1) DW_C1_KS(2) DW_C1_KS(3) DW_C1_KS(4) DW_C1_KS(5) DW_C1_KS(6) DW_C1_KS(7) DW_C1_KS(8)
    default: fail(-2, "conv1x1 u8->f16: no kernel for the shape");
  }
#undef DW_C1_KS
#undef DW_C1
  DW_HIP(hipGetLastError());
}

}  // namespace dw
