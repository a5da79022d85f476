// Convolutions that keep dragonwing-cpu's accumulation order, so their
// results are bit-identical to the CPU implementation:
//   acc = 0; for kh, for kw (skip taps outside the image), for ic:
//       acc = fma(x, w, acc)                       (f32, single rounding)
// (crates/dragonwing-cpu/src/ops.rs:1356-1436, :2572-2651, :2819-2933).
//
// direct_conv: one thread = one output pixel x a chunk of output channels
// (up to 80).  A wavefront covers 64 pixels of one chunk, so the weight row
// for (tap, ic) is wave-uniform and is fetched with scalar loads, and each
// input value is read and decoded once for the whole chunk.  Used for fp32
// convolutions, for convolutions whose c_in is not a multiple of 8 (the
// 3-channel stem), and for the fp16 layers of the int8 graph that must match
// the CPU bit for bit.
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

template <int IN_KIND>
__device__ __forceinline__ float load1(const DirectArgs& a, size_t i) {
  if (IN_KIND == 0) return ((const float*)a.x)[i];
  if (IN_KIND == 1) return h2f(((const uint16_t*)a.x)[i]);
  const int q = ((const uint8_t*)a.x)[i];
  return round_f16((float)(q - a.in_zp) * a.in_scale);  // DequantizeLinear to f16, then read
}

// Four consecutive channels; the caller guarantees 4-element alignment.
template <int IN_KIND>
__device__ __forceinline__ void load4(const DirectArgs& a, size_t i, float v[4]) {
  if (IN_KIND == 0) {
    const float4 f = *reinterpret_cast<const float4*>((const float*)a.x + i);
    v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
  } else if (IN_KIND == 1) {
    const uint2 u = *reinterpret_cast<const uint2*>((const uint16_t*)a.x + i);
    v[0] = h2f(u.x & 0xffff); v[1] = h2f(u.x >> 16); v[2] = h2f(u.y & 0xffff); v[3] = h2f(u.y >> 16);
  } else {
    const uint32_t u = *reinterpret_cast<const uint32_t*>((const uint8_t*)a.x + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = round_f16((float)((int)((u >> (8 * e)) & 0xff) - a.in_zp) * a.in_scale);
  }
}

// One thread = one output pixel x OC output channels (OC | c_out).  The
// workgroup first copies its weight slice [K][OC] (K = kh*kw*c_in) into
// LDS; every lane of a wavefront then reads the same weight row (a
// broadcast, free of bank conflicts), and each decoded input value feeds
// OC accumulators.  Per output the FMA sequence is the reference's.
template <int IN_KIND, int OC>
__global__ __launch_bounds__(256) void direct_conv_kernel(const DirectArgs a) {
  extern __shared__ float wl[];
  const int K = a.kh * a.kw * a.cin;
  const int oc0 = blockIdx.y * OC;
  for (int i = threadIdx.x; i < K * OC; i += blockDim.x) {
    const int k = i / OC, j = i - (i / OC) * OC;
    wl[i] = a.wf[(size_t)k * a.cout + oc0 + j];
  }
  __syncthreads();
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= a.m) return;
  const int hw = a.ho * a.wo;
  const int nn = p / hw;
  const int rem = p - nn * hw;
  const int oh = rem / a.wo;
  const int ow = rem - oh * a.wo;
  const bool vec4 = (a.cin & 3) == 0 && (a.x_pix_stride & 3) == 0 && (a.x_c_off & 3) == 0;

  float acc[OC];
#pragma unroll
  for (int j = 0; j < OC; ++j) acc[j] = 0.0f;

  auto fma_row = [&](float xv, const float* wr) {
    if constexpr (OC % 4 == 0) {
#pragma unroll
      for (int j = 0; j < OC; j += 4) {
        const float4 w4 = *reinterpret_cast<const float4*>(wr + j);
        acc[j] = fmaf(xv, w4.x, acc[j]);
        acc[j + 1] = fmaf(xv, w4.y, acc[j + 1]);
        acc[j + 2] = fmaf(xv, w4.z, acc[j + 2]);
        acc[j + 3] = fmaf(xv, w4.w, acc[j + 3]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < OC; ++j) acc[j] = fmaf(xv, wr[j], acc[j]);
    }
  };

  for (int kh = 0; kh < a.kh; ++kh) {
    const int ih = oh * a.sh + kh - a.pt;
    if (ih < 0 || ih >= a.h) continue;
    for (int kw = 0; kw < a.kw; ++kw) {
      const int iw = ow * a.sw + kw - a.pl;
      if (iw < 0 || iw >= a.w) continue;
      const size_t xo = ((size_t)(nn * a.h + ih) * a.w + iw) * a.x_pix_stride + a.x_c_off;
      const float* wrow = wl + (size_t)(kh * a.kw + kw) * a.cin * OC;
      if (vec4) {
        for (int ic = 0; ic < a.cin; ic += 4) {
          float xv[4];
          load4<IN_KIND>(a, xo + ic, xv);
#pragma unroll
          for (int e = 0; e < 4; ++e) fma_row(xv[e], wrow + (ic + e) * OC);
        }
      } else {
        for (int ic = 0; ic < a.cin; ++ic) fma_row(load1<IN_KIND>(a, xo + ic), wrow + ic * OC);
      }
    }
  }

  const size_t yo = (size_t)p * a.y_pix_stride + a.y_c_off + oc0;
#pragma unroll
  for (int j = 0; j < OC; ++j) {
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
  // Output-channel chunk: as wide as c_out and the 64 KB LDS weight slice
  // allow (each decoded input feeds more FMAs), narrowed when there are too
  // few pixels to fill the GPU.
  const long K = (long)a.kh * a.kw * a.cin;
  int oc = 0;
  for (int c : {32, 16, 8, 4, 1})
    if (a.cout % c == 0 && K * c * 4 <= 65536) { oc = c; break; }
  if (!oc) fail(-2, "direct conv: kernel too large for the LDS weight slice");
  const long waves = ((long)a.m + 63) / 64;
  if (oc == 32 && waves * (a.cout / oc) < 2048 && a.cout % 16 == 0) oc = 16;
  dim3 grid((a.m + 255) / 256, a.cout / oc);
  const size_t lds = (size_t)K * oc * 4;
#define DW_DC(KIND, O)                                                                         \
  if (a.in_kind == KIND && oc == O) {                                                          \
    hipLaunchKernelGGL((direct_conv_kernel<KIND, O>), grid, dim3(256), lds, st, a);            \
    DW_HIP(hipGetLastError());                                                                 \
    return;                                                                                    \
  }
#define DW_DC_ALL(O) DW_DC(0, O) DW_DC(1, O) DW_DC(2, O)
  DW_DC_ALL(32)
  DW_DC_ALL(16)
  DW_DC_ALL(8)
  DW_DC_ALL(4)
  DW_DC_ALL(1)
#undef DW_DC_ALL
#undef DW_DC
  fail(-2, "direct conv: no kernel for this channel count");
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
