// Convolutions that keep dragonwing-cpu's accumulation order, so their
// results are bit-identical to the CPU implementation:
//   acc = 0; for kh, for kw (skip taps outside the image), for ic:
//       acc = fma(x, w, acc)                       (f32, single rounding)
// (crates/dragonwing-cpu/src/ops.rs:1356-1436, :2572-2651, :2819-2933).
//
// direct_conv: one thread = one output pixel x 8 output channels.  A
// wavefront covers 64 pixels of one 8-channel group, so the weight row for
// (tap, ic) is wave-uniform and is fetched with scalar loads; inputs stream
// per lane.  Used for fp32 convolutions, for convolutions whose c_in is not
// a multiple of 8 (the 3-channel stem), and for the fp16 layers of the int8
// graph that must match the CPU bit for bit.
//
// dwconv: depthwise 3x3 (any k), channel multiplier 1.  One thread = one
// pixel x 8 channels, so every load/store is a 16-byte (f16) or 32-byte
// (f32) vector and consecutive threads walk consecutive channels (coalesced
// NHWC).  No matrix cores: the op is HBM-bound.
#include "dw_common.h"
#include "dw_device.h"

namespace dw {
namespace {


// relu_f32_scalar (ops.rs:208-220): x > 0 -> x, NaN -> NaN, else +0.
__device__ __forceinline__ float relu_ref(float v) { return v > 0.0f ? v : (v != v ? v : 0.0f); }

constexpr int OCG = 8;

__global__ __launch_bounds__(256) void direct_conv_kernel(const DirectArgs a) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  const int oc0 = blockIdx.y * OCG;
  if (p >= a.m) return;
  const int hw = a.ho * a.wo;
  const int nn = p / hw;
  const int rem = p - nn * hw;
  const int oh = rem / a.wo;
  const int ow = rem - oh * a.wo;
  const int nv = min(OCG, a.cout - oc0);

  float acc[OCG];
#pragma unroll
  for (int j = 0; j < OCG; ++j) acc[j] = 0.0f;

  for (int kh = 0; kh < a.kh; ++kh) {
    const int ih = oh * a.sh + kh - a.pt;
    if (ih < 0 || ih >= a.h) continue;
    for (int kw = 0; kw < a.kw; ++kw) {
      const int iw = ow * a.sw + kw - a.pl;
      if (iw < 0 || iw >= a.w) continue;
      const size_t xo = ((size_t)(nn * a.h + ih) * a.w + iw) * a.x_pix_stride + a.x_c_off;
      const float* wrow = a.wf + ((size_t)(kh * a.kw + kw) * a.cin) * a.cout + oc0;
      for (int ic = 0; ic < a.cin; ++ic) {
        float xv;
        if (a.in_kind == 0) {
          xv = ((const float*)a.x)[xo + ic];
        } else if (a.in_kind == 1) {
          xv = h2f(((const uint16_t*)a.x)[xo + ic]);
        } else {
          const int q = ((const uint8_t*)a.x)[xo + ic];
          xv = round_f16(((float)(q - a.in_zp) * a.in_scale));
        }
        const float* wr = wrow + (size_t)ic * a.cout;
        if (nv == OCG) {
#pragma unroll
          for (int j = 0; j < OCG; ++j) acc[j] = fmaf(xv, wr[j], acc[j]);
        } else {
          for (int j = 0; j < nv; ++j) acc[j] = fmaf(xv, wr[j], acc[j]);
        }
      }
    }
  }

  const size_t yo = (size_t)p * a.y_pix_stride + a.y_c_off + oc0;
  for (int j = 0; j < nv; ++j) {
    const int oc = oc0 + j;
    if (a.out_kind == 0) {
      float v = acc[j];
      if (a.bias_f) v = v + a.bias_f[oc];
      if (a.act == ACT_RELU) {
        v = relu_ref(v);
      } else if (a.act == ACT_SILU) {
        const float s = 1.0f / (1.0f + expf(-v));
        v = v * s;
      }
      ((float*)a.y)[yo + j] = v;
    } else {
      uint16_t hb = f2h(acc[j]);
      if (a.bias_h) hb = f16_add_bits(hb, a.bias_h[oc]);
      if (a.out_kind == 1) {
        ((uint16_t*)a.y)[yo + j] = f16_act_bits(hb, a.act);
      } else {
        // QuantizeLinear of the stored f16 value.
        float q = rintf(__fdiv_rn(h2f(hb), a.out_scale)) + (float)a.out_zp;
        q = fminf(fmaxf(q, 0.0f), 255.0f);
        int qi = (int)q;
        if (a.lut) qi = a.lut[qi];
        ((uint8_t*)a.y)[yo + j] = (uint8_t)qi;
      }
    }
  }
}

template <int ESZ>
__global__ __launch_bounds__(256) void dwconv_kernel(const DwArgs a) {
  constexpr int V = 8;
  const int groups = a.c / V;
  const size_t total = (size_t)a.n * a.ho * a.wo * groups;
  for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < total;
       t += (size_t)gridDim.x * blockDim.x) {
    const int g = (int)(t % groups);
    const size_t p = t / groups;
    const int hw = a.ho * a.wo;
    const int nn = (int)(p / hw);
    const int rem = (int)(p - (size_t)nn * hw);
    const int oh = rem / a.wo;
    const int ow = rem - oh * a.wo;
    const int c0 = g * V;
    float acc[V];
#pragma unroll
    for (int j = 0; j < V; ++j) acc[j] = 0.0f;
    for (int kh = 0; kh < a.kh; ++kh) {
      const int ih = oh * a.sh + kh - a.pt;
      if (ih < 0 || ih >= a.h) continue;
      for (int kw = 0; kw < a.kw; ++kw) {
        const int iw = ow * a.sw + kw - a.pl;
        if (iw < 0 || iw >= a.w) continue;
        const size_t xo = ((size_t)(nn * a.h + ih) * a.w + iw) * a.x_pix_stride + a.x_c_off + c0;
        const size_t wo_ = (size_t)(kh * a.kw + kw) * a.c + c0;
        float xv[V], wv[V];
        if (ESZ == 2) {
          const uint4 xr = *reinterpret_cast<const uint4*>((const uint16_t*)a.x + xo);
          const uint4 wr = *reinterpret_cast<const uint4*>((const uint16_t*)a.wt + wo_);
          const uint32_t xs[4] = {xr.x, xr.y, xr.z, xr.w};
          const uint32_t ws[4] = {wr.x, wr.y, wr.z, wr.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            xv[2 * q] = h2f(xs[q] & 0xffff);
            xv[2 * q + 1] = h2f(xs[q] >> 16);
            wv[2 * q] = h2f(ws[q] & 0xffff);
            wv[2 * q + 1] = h2f(ws[q] >> 16);
          }
        } else {
          const float4* xp = reinterpret_cast<const float4*>((const float*)a.x + xo);
          const float4* wp = reinterpret_cast<const float4*>((const float*)a.wt + wo_);
          const float4 x0 = xp[0], x1 = xp[1], w0 = wp[0], w1 = wp[1];
          xv[0] = x0.x; xv[1] = x0.y; xv[2] = x0.z; xv[3] = x0.w;
          xv[4] = x1.x; xv[5] = x1.y; xv[6] = x1.z; xv[7] = x1.w;
          wv[0] = w0.x; wv[1] = w0.y; wv[2] = w0.z; wv[3] = w0.w;
          wv[4] = w1.x; wv[5] = w1.y; wv[6] = w1.z; wv[7] = w1.w;
        }
#pragma unroll
        for (int j = 0; j < V; ++j) acc[j] = fmaf(xv[j], wv[j], acc[j]);
      }
    }
    const size_t yo = p * a.y_pix_stride + a.y_c_off + c0;
    if (ESZ == 2) {
      uint32_t outw[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint16_t hv[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int j = 2 * q + e;
          uint16_t hb = f2h(acc[j]);
          if (a.bias) hb = f16_add_bits(hb, ((const uint16_t*)a.bias)[c0 + j]);
          hv[e] = f16_act_bits(hb, a.act);
        }
        outw[q] = (uint32_t)hv[0] | ((uint32_t)hv[1] << 16);
      }
      *reinterpret_cast<uint4*>((uint16_t*)a.y + yo) = make_uint4(outw[0], outw[1], outw[2], outw[3]);
    } else {
      float ov[V];
#pragma unroll
      for (int j = 0; j < V; ++j) {
        float v = acc[j];
        if (a.bias) v = v + ((const float*)a.bias)[c0 + j];
        if (a.act == ACT_RELU) {
          v = relu_ref(v);
        } else if (a.act == ACT_SILU) {
          const float s = 1.0f / (1.0f + expf(-v));
          v = v * s;
        }
        ov[j] = v;
      }
      float4* yp = reinterpret_cast<float4*>((float*)a.y + yo);
      yp[0] = make_float4(ov[0], ov[1], ov[2], ov[3]);
      yp[1] = make_float4(ov[4], ov[5], ov[6], ov[7]);
    }
  }
}

}  // namespace

void launch_direct_conv(hipStream_t st, const DirectArgs& a) {
  dim3 grid((a.m + 255) / 256, (a.cout + OCG - 1) / OCG);
  hipLaunchKernelGGL(direct_conv_kernel, grid, dim3(256), 0, st, a);
  DW_HIP(hipGetLastError());
}

void launch_dwconv(hipStream_t st, const DwArgs& a, int dtype) {
  const size_t total = (size_t)a.n * a.ho * a.wo * (a.c / 8);
  size_t blocks = (total + 255) / 256;
  if (blocks > 65535 * 8) blocks = 65535 * 8;
  if (dtype == F16)
    hipLaunchKernelGGL(dwconv_kernel<2>, dim3((unsigned)blocks), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(dwconv_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, st, a);
  DW_HIP(hipGetLastError());
}

}  // namespace dw
