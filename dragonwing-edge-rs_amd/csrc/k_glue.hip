// Bandwidth-bound glue: elementwise math, (re)quantization, max pooling,
// nearest resize, channel copies and the calibration min/max reduction.
// No matrix cores.  Each thread handles a short contiguous run of elements
// so loads and stores are issued as wide vectors where alignment allows,
// and NHWC views keep channels (the fastest axis) on consecutive lanes.
#include "dw_common.h"
#include "dw_device.h"

#include <algorithm>
#include <type_traits>

namespace dw {
namespace {


// --- scalar semantics, one element -----------------------------------------
// Each case cites the dragonwing-cpu function it reproduces.
__device__ __forceinline__ void ew_one(const EwArgs& a, size_t i) {
  switch (a.op) {
    case EW_RELU:
      if (a.dtype == F32) {  // relu_f32_scalar ops.rs:208-220
        const float v = ((const float*)a.a)[i];
        ((float*)a.y)[i] = v > 0.0f ? v : (v != v ? v : 0.0f);
      } else {  // relu_fp16 ops.rs:345-352
        const float v = h2f(((const uint16_t*)a.a)[i]);
        ((uint16_t*)a.y)[i] = f2h(v > 0.0f ? v : 0.0f);
      }
      break;
    case EW_ADD:
      if (a.dtype == F32)  // add_f32_scalar ops.rs:378-384
        ((float*)a.y)[i] = ((const float*)a.a)[i] + ((const float*)a.b)[i];
      else  // add_fp16 ops.rs:434-442
        ((uint16_t*)a.y)[i] =
            f2h(h2f(((const uint16_t*)a.a)[i]) + h2f(((const uint16_t*)a.b)[i]));
      break;
    case EW_MUL:
      if (a.dtype == F32)  // mul_f32_scalar ops.rs:1913-1919
        ((float*)a.y)[i] = ((const float*)a.a)[i] * ((const float*)a.b)[i];
      else  // mul_fp16 ops.rs:1959-1967
        ((uint16_t*)a.y)[i] =
            f2h(h2f(((const uint16_t*)a.a)[i]) * h2f(((const uint16_t*)a.b)[i]));
      break;
    case EW_SIGMOID:
      if (a.dtype == F32) {  // sigmoid_f32_scalar ops.rs:1865-1870
        const float v = ((const float*)a.a)[i];
        ((float*)a.y)[i] = 1.0f / (1.0f + expf(-v));
      } else {  // sigmoid_fp16 ops.rs:1881-1888
        const float v = h2f(((const uint16_t*)a.a)[i]);
        ((uint16_t*)a.y)[i] = f2h(1.0f / (1.0f + expf(-v)));
      }
      break;
    case EW_SILU:
      if (a.dtype == F32) {  // sigmoid then mul in f32
        const float v = ((const float*)a.a)[i];
        const float s = 1.0f / (1.0f + expf(-v));
        ((float*)a.y)[i] = v * s;
      } else {  // sigmoid_fp16 then mul_fp16
        const float v = h2f(((const uint16_t*)a.a)[i]);
        const float s = round_f16((1.0f / (1.0f + expf(-v))));
        ((uint16_t*)a.y)[i] = f2h(v * s);
      }
      break;
    case EW_BIAS_ADD:  // bias_add_f32_nhwc: y[i] += b[i % c]
      ((float*)a.y)[i] = ((const float*)a.a)[i] + ((const float*)a.b)[i % a.c];
      break;
    case EW_REQUANT_I32_I8: {  // requantize_i32_to_i8_scalar ops.rs:3380-3386
      float f = (float)((const int*)a.a)[i] * a.s0;
      f = fminf(fmaxf(f, -128.0f), 127.0f);
      ((int8_t*)a.y)[i] = (int8_t)(int)roundf(f);
      break;
    }
    case EW_QUANT_F32_I8: {  // quantize_f32_to_i8_scalar ops.rs:3519-3525 (s0 = 1/scale)
      float f = ((const float*)a.a)[i] * a.s0;
      f = fminf(fmaxf(f, -128.0f), 127.0f);
      ((int8_t*)a.y)[i] = (int8_t)(int)roundf(f);
      break;
    }
    case EW_DEQUANT_I8_F32:  // dequantize_i8_to_f32_scalar ops.rs:3453-3457
      ((float*)a.y)[i] = (float)((const int8_t*)a.a)[i] * a.s0;
      break;
    case EW_ADD_I8: {  // add_i8_scalar ops.rs:3197-3209
      const float r = (float)((const int8_t*)a.a)[i] * a.s0 + (float)((const int8_t*)a.b)[i] * a.s1;
      const float c = fminf(fmaxf(r, -128.0f), 127.0f);
      ((int8_t*)a.y)[i] = (int8_t)(int)roundf(c);
      break;
    }
    case EW_RELU_I8: {  // relu_i8_scalar ops.rs:3315-3320
      const int8_t v = ((const int8_t*)a.a)[i];
      ((int8_t*)a.y)[i] = v > 0 ? v : 0;
      break;
    }
    case EW_QUANT_LINEAR_F16_U8: {  // ONNX QuantizeLinear, RNE
      const float v = h2f(((const uint16_t*)a.a)[i]);
      float q = rintf(__fdiv_rn(v, a.s0)) + (float)a.z0;
      q = fminf(fmaxf(q, 0.0f), 255.0f);
      ((uint8_t*)a.y)[i] = (uint8_t)(int)q;
      break;
    }
    case EW_DEQUANT_LINEAR_U8_F16: {  // ONNX DequantizeLinear into f16
      const int q = ((const uint8_t*)a.a)[i];
      ((uint16_t*)a.y)[i] = f2h((float)(q - a.z0) * a.s0);
      break;
    }
    case EW_QADD_U8: {  // QLinearAdd, RNE: s0 = sa/sy, s1 = sb/sy
      const int qa = ((const uint8_t*)a.a)[i];
      const int qb = ((const uint8_t*)a.b)[i];
      const float f = (float)(qa - a.z0) * a.s0 + (float)(qb - a.z1) * a.s1;
      float g = rintf(f) + (float)a.z2;
      g = fminf(fmaxf(g, 0.0f), 255.0f);
      ((uint8_t*)a.y)[i] = (uint8_t)(int)g;
      break;
    }
    case EW_LUT_U8:
      ((uint8_t*)a.y)[i] = a.lut[((const uint8_t*)a.a)[i]];
      break;
    case EW_F32_TO_F16:
      ((uint16_t*)a.y)[i] = f2h(((const float*)a.a)[i]);
      break;
    case EW_F16_TO_F32:
      ((float*)a.y)[i] = h2f(((const uint16_t*)a.a)[i]);
      break;
    case EW_CLIP:  // dispatch_clip (onnx runtime.rs:1004-1042): f32::clamp(min = s0, max = s1)
      if (a.dtype == F32) {
        const float v = ((const float*)a.a)[i];
        ((float*)a.y)[i] = v < a.s0 ? a.s0 : (v > a.s1 ? a.s1 : v);
      } else {  // F16::from_f32(to_f32().clamp(min, max))
        const float v = h2f(((const uint16_t*)a.a)[i]);
        ((uint16_t*)a.y)[i] = f2h(v < a.s0 ? a.s0 : (v > a.s1 ? a.s1 : v));
      }
      break;
  }
}

// Element sizes of an op's first operand and its result.
__device__ __forceinline__ void ew_sizes(int op, int dtype, int& in, int& out) {
  switch (op) {
    case EW_QADD_U8: case EW_LUT_U8: case EW_ADD_I8: case EW_RELU_I8: in = 1; out = 1; return;
    case EW_DEQUANT_LINEAR_U8_F16: in = 1; out = 2; return;
    case EW_QUANT_LINEAR_F16_U8: in = 2; out = 1; return;
    case EW_REQUANT_I32_I8: case EW_QUANT_F32_I8: in = 4; out = 1; return;
    case EW_DEQUANT_I8_F32: in = 1; out = 4; return;
    default: in = out = dtype_size(dtype); return;
  }
}

__global__ __launch_bounds__(256) void elementwise_kernel(const EwArgs a) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < a.count;
       i += (size_t)gridDim.x * blockDim.x)
    ew_one(a, i);
}

// 2-D (pixel x channel) version over channel-strided views: element (p, c)
// of a, b and y are located through their own views.  Used by the graph
// runtime for ops whose operands are slices of concat buffers.
__global__ __launch_bounds__(256) void elementwise2d_kernel(const Ew2Args e) {
  const size_t total = (size_t)e.pixels * e.channels;
  int esz_in, esz_out;
  ew_sizes(e.op, e.dtype, esz_in, esz_out);
  for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < total;
       t += (size_t)gridDim.x * blockDim.x) {
    const size_t p = t / e.channels;
    const int c = (int)(t - p * e.channels);
    EwArgs a;
    a.op = e.op;
    a.dtype = e.dtype;
    a.a = (const uint8_t*)e.a.base + (p * e.a.pix_stride + e.a.c_off + c) * esz_in;
    a.b = e.b.base ? (const uint8_t*)e.b.base + (p * e.b.pix_stride + e.b.c_off + c) * esz_in
                   : nullptr;
    a.y = (uint8_t*)e.y.base + (p * e.y.pix_stride + e.y.c_off + c) * esz_out;
    a.count = 1;
    a.c = 1;
    a.s0 = e.s0; a.s1 = e.s1; a.s2 = e.s2;
    a.z0 = e.z0; a.z1 = e.z1; a.z2 = e.z2;
    a.lut = e.lut;
    ew_one(a, 0);
  }
}

// Padded max pool over one element type.  Padded taps never win (ONNX
// MaxPool); a window with no valid tap cannot occur for pad < kernel.
template <typename T>
__device__ __forceinline__ T tmax(T a, T b);
template <>
__device__ __forceinline__ float tmax<float>(float a, float b) {
  return b > a ? b : a;  // f32::max ignoring NaN second operand order as in ops.rs:1540
}
template <>
__device__ __forceinline__ uint8_t tmax<uint8_t>(uint8_t a, uint8_t b) { return b > a ? b : a; }
template <>
__device__ __forceinline__ int8_t tmax<int8_t>(int8_t a, int8_t b) { return b > a ? b : a; }

template <typename T>
__device__ __forceinline__ T tlow();
template <>
__device__ __forceinline__ float tlow<float>() { return -__builtin_inff(); }
template <>
__device__ __forceinline__ uint8_t tlow<uint8_t>() { return 0; }
template <>
__device__ __forceinline__ int8_t tlow<int8_t>() { return -128; }

// f16 values are compared as f32 (exact); storage stays f16 bits.
struct H16 {
  uint16_t b;
};

template <typename T>
__global__ __launch_bounds__(256) void maxpool_kernel(const PoolArgs a) {
  const size_t total = (size_t)a.n * a.ho * a.wo * a.c;
  for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < total;
       t += (size_t)gridDim.x * blockDim.x) {
    const int ch = (int)(t % a.c);
    const size_t p = t / a.c;
    const int hw = a.ho * a.wo;
    const int nn = (int)(p / hw);
    const int rem = (int)(p - (size_t)nn * hw);
    const int oh = rem / a.wo, ow = rem - (rem / a.wo) * a.wo;
    T best = tlow<T>();
    for (int kh = 0; kh < a.kh; ++kh) {
      const int ih = oh * a.sh + kh - a.pt;
      if (ih < 0 || ih >= a.h) continue;
      for (int kw = 0; kw < a.kw; ++kw) {
        const int iw = ow * a.sw + kw - a.pl;
        if (iw < 0 || iw >= a.w) continue;
        const size_t xi = ((size_t)(nn * a.h + ih) * a.w + iw) * a.x.pix_stride + a.x.c_off + ch;
        best = tmax<T>(best, ((const T*)a.x.base)[xi]);
      }
    }
    ((T*)a.y.base)[p * a.y.pix_stride + a.y.c_off + ch] = best;
  }
}

__global__ __launch_bounds__(256) void maxpool_f16_kernel(const PoolArgs a) {
  const size_t total = (size_t)a.n * a.ho * a.wo * a.c;
  for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < total;
       t += (size_t)gridDim.x * blockDim.x) {
    const int ch = (int)(t % a.c);
    const size_t p = t / a.c;
    const int hw = a.ho * a.wo;
    const int nn = (int)(p / hw);
    const int rem = (int)(p - (size_t)nn * hw);
    const int oh = rem / a.wo, ow = rem - (rem / a.wo) * a.wo;
    float best = -__builtin_inff();
    uint16_t bestb = 0xfc00;
    for (int kh = 0; kh < a.kh; ++kh) {
      const int ih = oh * a.sh + kh - a.pt;
      if (ih < 0 || ih >= a.h) continue;
      for (int kw = 0; kw < a.kw; ++kw) {
        const int iw = ow * a.sw + kw - a.pl;
        if (iw < 0 || iw >= a.w) continue;
        const size_t xi = ((size_t)(nn * a.h + ih) * a.w + iw) * a.x.pix_stride + a.x.c_off + ch;
        const uint16_t b = ((const uint16_t*)a.x.base)[xi];
        const float v = h2f(b);
        if (v > best) { best = v; bestb = b; }
      }
    }
    ((uint16_t*)a.y.base)[p * a.y.pix_stride + a.y.c_off + ch] = bestb;
  }
}

// SPPF: three cascaded k x k / stride 1 / pad k/2 pools.  Cascading such
// pools equals single pools of size k, 2k-1 and 3k-2 (max is associative
// and the padded taps never win), so all three outputs come from one read
// of the input neighbourhood.
template <typename T>
__global__ __launch_bounds__(256) void maxpool_cascade3_kernel(const PoolArgs a, View y2, View y3) {
  const size_t total = (size_t)a.n * a.h * a.w * a.c;
  const int r1 = a.kh / 2, r2 = 2 * r1, r3 = 3 * r1;
  for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < total;
       t += (size_t)gridDim.x * blockDim.x) {
    const int ch = (int)(t % a.c);
    const size_t p = t / a.c;
    const int hw = a.h * a.w;
    const int nn = (int)(p / hw);
    const int rem = (int)(p - (size_t)nn * hw);
    const int oh = rem / a.w, ow = rem - (rem / a.w) * a.w;
    float b1 = -__builtin_inff(), b2 = b1, b3 = b1;
    uint32_t v1 = 0, v2 = 0, v3 = 0;
    for (int dy = -r3; dy <= r3; ++dy) {
      const int ih = oh + dy;
      if (ih < 0 || ih >= a.h) continue;
      const int ady = dy < 0 ? -dy : dy;
      for (int dx = -r3; dx <= r3; ++dx) {
        const int iw = ow + dx;
        if (iw < 0 || iw >= a.w) continue;
        const int adx = dx < 0 ? -dx : dx;
        const int d = ady > adx ? ady : adx;
        const size_t xi = ((size_t)(nn * a.h + ih) * a.w + iw) * a.x.pix_stride + a.x.c_off + ch;
        float v;
        uint32_t raw;
        if constexpr (sizeof(T) == 2) {
          raw = ((const uint16_t*)a.x.base)[xi];
          v = h2f((uint16_t)raw);
        } else if constexpr (sizeof(T) == 4) {
          v = ((const float*)a.x.base)[xi];
          raw = __builtin_bit_cast(uint32_t, v);
        } else {
          raw = ((const uint8_t*)a.x.base)[xi];
          v = (float)raw;
        }
        if (v > b3) { b3 = v; v3 = raw; }
        if (d <= r2 && v > b2) { b2 = v; v2 = raw; }
        if (d <= r1 && v > b1) { b1 = v; v1 = raw; }
      }
    }
    const size_t o1 = p * a.y.pix_stride + a.y.c_off + ch;
    const size_t o2 = p * y2.pix_stride + y2.c_off + ch;
    const size_t o3 = p * y3.pix_stride + y3.c_off + ch;
    if constexpr (sizeof(T) == 2) {
      ((uint16_t*)a.y.base)[o1] = (uint16_t)v1;
      ((uint16_t*)y2.base)[o2] = (uint16_t)v2;
      ((uint16_t*)y3.base)[o3] = (uint16_t)v3;
    } else if constexpr (sizeof(T) == 4) {
      ((uint32_t*)a.y.base)[o1] = v1;
      ((uint32_t*)y2.base)[o2] = v2;
      ((uint32_t*)y3.base)[o3] = v3;
    } else {
      ((uint8_t*)a.y.base)[o1] = (uint8_t)v1;
      ((uint8_t*)y2.base)[o2] = (uint8_t)v2;
      ((uint8_t*)y3.base)[o3] = (uint8_t)v3;
    }
  }
}

// SPPF cascade for planes that fit in LDS: one workgroup owns one image and
// one 16-byte channel slice (16 u8 / 8 f16 / 4 f32 channels) and keeps the
// whole H x W plane in LDS.  The cascade of three k x k pools (stride 1,
// pad k/2) equals single pools of sizes k, 2k - 1 and 3k - 2, each the
// separable row-then-column maximum, so one pass computes the three row
// maxima of every pixel from one read of its 3k - 2 row neighbours, and a
// second pass the three column maxima, which are the three outputs: two
// barriers for the whole cascade.  Max is exact, so the order of the
// comparisons does not change any value.
typedef unsigned char u8x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

template <int ES>
__device__ __forceinline__ uint4 vmax16(uint4 a, uint4 b) {
  if constexpr (ES == 1) {
    return __builtin_bit_cast(uint4, __builtin_elementwise_max(__builtin_bit_cast(u8x16, a),
                                                               __builtin_bit_cast(u8x16, b)));
  } else if constexpr (ES == 2) {
    return __builtin_bit_cast(uint4, __builtin_elementwise_max(__builtin_bit_cast(f16x8, a),
                                                               __builtin_bit_cast(f16x8, b)));
  } else {
    const float4 x = __builtin_bit_cast(float4, a), y = __builtin_bit_cast(float4, b);
    return __builtin_bit_cast(uint4, make_float4(fmaxf(x.x, y.x), fmaxf(x.y, y.y), fmaxf(x.z, y.z),
                                                 fmaxf(x.w, y.w)));
  }
}

// plane: hw pixels of the input, then three planes of row maxima (radius
// r, 2r, 3r); 4 * hw * 16 bytes of LDS
// RAD > 0: the radius fixed at compile time (the SPPF's 5x5 pools: 2), the
// loops unrolled, and neighbours outside the image clamped to the edge
// pixel instead of skipped (that pixel is in the window already, and max
// is idempotent, so the results are the same); RAD = 0: any radius.
template <int ES, int RAD>
__global__ __launch_bounds__(512) void sppf_lds_kernel(const PoolArgs a, View y2, View y3) {
  extern __shared__ uint4 plane[];
  const int hw = a.h * a.w;
  uint4* const X = plane;
  uint4* const R1 = plane + hw;
  uint4* const R2 = plane + 2 * hw;
  uint4* const R3 = plane + 3 * hw;
  const int nn = blockIdx.x;
  const int c0 = blockIdx.y * (16 / ES);
  const int r = a.kh / 2;
  auto gaddr = [&](const View& v, int pix) {
    return (uint8_t*)v.base + ((size_t)(nn * hw + pix) * v.pix_stride + v.c_off + c0) * ES;
  };
  for (int i = threadIdx.x; i < hw; i += blockDim.x) X[i] = *reinterpret_cast<const uint4*>(gaddr(a.x, i));
  __syncthreads();
  // row maxima over |dx| <= r, 2r, 3r (columns outside the image never win)
  for (int i = threadIdx.x; i < hw; i += blockDim.x) {
    const int y = i / a.w, x = i - (i / a.w) * a.w;
    const uint4* row = X + y * a.w;
    uint4 m = row[x];
    if constexpr (RAD > 0) {
#pragma unroll
      for (int d = 1; d <= 3 * RAD; ++d) {
        m = vmax16<ES>(m, row[max(x - d, 0)]);
        m = vmax16<ES>(m, row[min(x + d, a.w - 1)]);
        if (d == RAD) R1[i] = m;
        if (d == 2 * RAD) R2[i] = m;
      }
    } else {
      R1[i] = m;  // r = 0 (a 1x1 pool): the loops below add nothing
      R2[i] = m;
      for (int d = 1; d <= 3 * r; ++d) {
        if (x - d >= 0) m = vmax16<ES>(m, row[x - d]);
        if (x + d < a.w) m = vmax16<ES>(m, row[x + d]);
        if (d == r) R1[i] = m;
        if (d == 2 * r) R2[i] = m;
      }
    }
    R3[i] = m;
  }
  __syncthreads();
  // column maxima of the three row-maximum planes: the three outputs
  for (int i = threadIdx.x; i < hw; i += blockDim.x) {
    const int y = i / a.w;
    uint4 m1 = R1[i], m2 = R2[i], m3 = R3[i];
    if constexpr (RAD > 0) {
#pragma unroll
      for (int d = 1; d <= 3 * RAD; ++d) {
        const int up = i - min(d, y) * a.w, dn = i + min(d, a.h - 1 - y) * a.w;
        if (d <= RAD) m1 = vmax16<ES>(vmax16<ES>(m1, R1[up]), R1[dn]);
        if (d <= 2 * RAD) m2 = vmax16<ES>(vmax16<ES>(m2, R2[up]), R2[dn]);
        m3 = vmax16<ES>(vmax16<ES>(m3, R3[up]), R3[dn]);
      }
    } else {
      for (int d = 1; d <= 3 * r; ++d) {
        const bool up = y - d >= 0, dn = y + d < a.h;
        if (d <= r) {
          if (up) m1 = vmax16<ES>(m1, R1[i - d * a.w]);
          if (dn) m1 = vmax16<ES>(m1, R1[i + d * a.w]);
        }
        if (d <= 2 * r) {
          if (up) m2 = vmax16<ES>(m2, R2[i - d * a.w]);
          if (dn) m2 = vmax16<ES>(m2, R2[i + d * a.w]);
        }
        if (up) m3 = vmax16<ES>(m3, R3[i - d * a.w]);
        if (dn) m3 = vmax16<ES>(m3, R3[i + d * a.w]);
      }
    }
    *reinterpret_cast<uint4*>(gaddr(a.y, i)) = m1;
    *reinterpret_cast<uint4*>(gaddr(y2, i)) = m2;
    *reinterpret_cast<uint4*>(gaddr(y3, i)) = m3;
  }
}

// Nearest resize (resize_f32 Nearest, ops.rs:2320-2351):
//   ih = clamp(round((oh + 0.5) * (h_in / h_out) - 0.5), 0, h_in - 1)
// computed in f32 like the reference; `round` is half away from zero.
__device__ __forceinline__ int nearest_index(int o, float scale, int n_in) {
  float f = roundf(((float)o + 0.5f) * scale - 0.5f);
  f = fmaxf(f, 0.0f);
  f = fminf(f, (float)(n_in - 1));
  return (int)f;
}

// Workgroups take strips of one output row (row = n * ho + oh, so the
// source row is uniform); threads over (output column, VB-byte word of the
// channels).  VB = 16 when both views' rows are 16-byte aligned, else 4.
template <int VB>
__global__ __launch_bounds__(256) void resize_nearest_kernel(const ResizeArgs a, int esz, int strips) {
  using V = typename std::conditional<VB == 16, uint4, uint32_t>::type;
  const int words = a.c * esz / VB;
  const int row = blockIdx.x / strips;
  const int t = (blockIdx.x - row * strips) * 256 + threadIdx.x;
  if (t >= a.wo * words) return;
  const int nn = row / a.ho, oh = row - nn * a.ho;
  const int ow = t / words, wd = t - ow * words;
  const int ih = nearest_index(oh, (float)a.h / (float)a.ho, a.h);
  const int iw = nearest_index(ow, (float)a.w / (float)a.wo, a.w);
  const size_t src = ((size_t)(nn * a.h + ih) * a.w + iw) * a.x.pix_stride + a.x.c_off;
  const size_t dst = ((size_t)row * a.wo + ow) * a.y.pix_stride + a.y.c_off;
  const V v = *reinterpret_cast<const V*>((const uint8_t*)a.x.base + src * esz + (size_t)wd * VB);
  *reinterpret_cast<V*>((uint8_t*)a.y.base + dst * esz + (size_t)wd * VB) = v;
}

__global__ __launch_bounds__(256) void copy_channels_kernel(View s, View d, int pixels, int bytes_row,
                                                           int esz) {
  const size_t total = (size_t)pixels * bytes_row;
  for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < total;
       t += (size_t)gridDim.x * blockDim.x) {
    const size_t p = t / bytes_row;
    const int b = (int)(t - p * bytes_row);
    ((uint8_t*)d.base)[(p * d.pix_stride + d.c_off) * esz + b] =
        ((const uint8_t*)s.base)[(p * s.pix_stride + s.c_off) * esz + b];
  }
}

__global__ void minmax_init_kernel(float* out) {
  out[0] = __builtin_inff();
  out[1] = -__builtin_inff();
}

// Ordered-int trick: for finite floats, atomic min/max on the int bits of
// non-negative values and on the reversed bits of negative values.
__device__ __forceinline__ void atomic_min_f(float* addr, float v) {
  if (v >= 0.0f)
    atomicMin((int*)addr, __float_as_int(v));
  else
    atomicMax((unsigned*)addr, __float_as_uint(v));
}
__device__ __forceinline__ void atomic_max_f(float* addr, float v) {
  if (v >= 0.0f)
    atomicMax((int*)addr, __float_as_int(v));
  else
    atomicMin((unsigned*)addr, __float_as_uint(v));
}

__global__ __launch_bounds__(256) void minmax_kernel(View x, int pixels, int channels, float* out) {
  const size_t total = (size_t)pixels * channels;
  float lo = __builtin_inff(), hi = -__builtin_inff();
  for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < total;
       t += (size_t)gridDim.x * blockDim.x) {
    const size_t p = t / channels;
    const int c = (int)(t - p * channels);
    const float v = ((const float*)x.base)[p * x.pix_stride + x.c_off + c];
    if (__builtin_isfinite(v)) {  // TensorStats::update skips non-finite values (calibration.rs:56-63)
      lo = fminf(lo, v);
      hi = fmaxf(hi, v);
    }
  }
  for (int off = 32; off > 0; off >>= 1) {
    lo = fminf(lo, __shfl_xor(lo, off));
    hi = fmaxf(hi, __shfl_xor(hi, off));
  }
  __shared__ float slo[4], shi[4];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { slo[wave] = lo; shi[wave] = hi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) {
      lo = fminf(lo, slo[w]);
      hi = fmaxf(hi, shi[w]);
    }
    if (lo <= hi) {
      // -0 and +0 are equal as range ends; +0's bit pattern keeps the
      // integer orderings of atomic_min_f / atomic_max_f valid
      if (lo == 0.0f) lo = 0.0f;
      if (hi == 0.0f) hi = 0.0f;
      atomic_min_f(out, lo);
      atomic_max_f(out + 1, hi);
    }
  }
}

unsigned grid_for(size_t total) {
  size_t b = (total + 255) / 256;
  if (b > 65535u * 16u) b = 65535u * 16u;
  if (b == 0) b = 1;
  return (unsigned)b;
}

}  // namespace

void launch_elementwise(hipStream_t st, const EwArgs& a) {
  if (a.count == 0) return;
  hipLaunchKernelGGL(elementwise_kernel, dim3(grid_for(a.count)), dim3(256), 0, st, a);
  DW_HIP(hipGetLastError());
}

void launch_elementwise2d(hipStream_t st, const Ew2Args& a) {
  const size_t total = (size_t)a.pixels * a.channels;
  if (total == 0) return;
  hipLaunchKernelGGL(elementwise2d_kernel, dim3(grid_for(total)), dim3(256), 0, st, a);
  DW_HIP(hipGetLastError());
}

void launch_maxpool(hipStream_t st, const PoolArgs& a, int dtype) {
  const size_t total = (size_t)a.n * a.ho * a.wo * a.c;
  if (total == 0) return;
  const dim3 g(grid_for(total)), b(256);
  switch (dtype) {
    case F32: hipLaunchKernelGGL(maxpool_kernel<float>, g, b, 0, st, a); break;
    case F16: hipLaunchKernelGGL(maxpool_f16_kernel, g, b, 0, st, a); break;
    case U8: hipLaunchKernelGGL(maxpool_kernel<uint8_t>, g, b, 0, st, a); break;
    case I8: hipLaunchKernelGGL(maxpool_kernel<int8_t>, g, b, 0, st, a); break;
    default: fail(-2, "maxpool: unsupported dtype");
  }
  DW_HIP(hipGetLastError());
}

void launch_maxpool_cascade3(hipStream_t st, const PoolArgs& a, View y2, View y3, int dtype) {
  const size_t total = (size_t)a.n * a.h * a.w * a.c;
  if (total == 0) return;
  const int es = dtype_size(dtype);
  const size_t lds = (size_t)4 * a.h * a.w * 16;
  auto al16 = [&](const View& v) { return (v.pix_stride * es) % 16 == 0 && (v.c_off * es) % 16 == 0; };
  if ((a.c * es) % 16 == 0 && lds <= 65536 && al16(a.x) && al16(a.y) && al16(y2) && al16(y3) &&
      (dtype == U8 || dtype == F16 || dtype == F32)) {
    // one thread per pixel up to 512 pixels
    const int threads = std::min(512, ((a.h * a.w + 63) / 64) * 64);
    const dim3 g(a.n, a.c * es / 16), b(threads);
    const bool k5 = a.kh == 5;  // the SPPF's pools: the unrolled form
#define DW_SPPF(ES_)                                                                   \
  if (k5)                                                                              \
    hipLaunchKernelGGL((sppf_lds_kernel<ES_, 2>), g, b, lds, st, a, y2, y3);          \
  else                                                                                 \
    hipLaunchKernelGGL((sppf_lds_kernel<ES_, 0>), g, b, lds, st, a, y2, y3);
    if (es == 1) {
      DW_SPPF(1)
    } else if (es == 2) {
      DW_SPPF(2)
    } else {
      DW_SPPF(4)
    }
#undef DW_SPPF
    DW_HIP(hipGetLastError());
    return;
  }
  const dim3 g(grid_for(total)), b(256);
  switch (dtype) {
    case F32: hipLaunchKernelGGL(maxpool_cascade3_kernel<float>, g, b, 0, st, a, y2, y3); break;
    case F16: hipLaunchKernelGGL(maxpool_cascade3_kernel<H16>, g, b, 0, st, a, y2, y3); break;
    case U8: hipLaunchKernelGGL(maxpool_cascade3_kernel<uint8_t>, g, b, 0, st, a, y2, y3); break;
    default: fail(-2, "maxpool cascade: unsupported dtype");
  }
  DW_HIP(hipGetLastError());
}

void launch_resize_nearest(hipStream_t st, const ResizeArgs& a, int dtype) {
  const int esz = dtype_size(dtype);
  if ((a.c * esz) % 4 != 0) fail(-2, "resize: channel bytes must be a multiple of 4");
  if ((size_t)a.n * a.ho * a.wo * a.c == 0) return;
  auto aligned16 = [&](const View& v, const void* base) {
    return ((uintptr_t)base % 16 == 0) && (v.pix_stride * esz) % 16 == 0 && (v.c_off * esz) % 16 == 0;
  };
  const bool v16 = (a.c * esz) % 16 == 0 && aligned16(a.x, a.x.base) && aligned16(a.y, a.y.base);
  const int vb = v16 ? 16 : 4;
  const int strips = (a.wo * (a.c * esz / vb) + 255) / 256;
  const long long blocks = (long long)a.n * a.ho * strips;
  if (blocks >= (1ll << 31)) fail(-2, "resize: output too large");
  const dim3 g((unsigned)blocks), b(256);
  if (v16)
    hipLaunchKernelGGL(resize_nearest_kernel<16>, g, b, 0, st, a, esz, strips);
  else
    hipLaunchKernelGGL(resize_nearest_kernel<4>, g, b, 0, st, a, esz, strips);
  DW_HIP(hipGetLastError());
}

void launch_copy_channels(hipStream_t st, View src, View dst, int pixels, int channels, int esize) {
  const size_t total = (size_t)pixels * channels * esize;
  if (total == 0) return;
  hipLaunchKernelGGL(copy_channels_kernel, dim3(grid_for(total)), dim3(256), 0, st, src, dst, pixels,
                     channels * esize, esize);
  DW_HIP(hipGetLastError());
}

void launch_minmax_init(hipStream_t st, float* out) {
  hipLaunchKernelGGL(minmax_init_kernel, dim3(1), dim3(1), 0, st, out);
  DW_HIP(hipGetLastError());
}

void launch_minmax(hipStream_t st, View x, int pixels, int channels, float* out) {
  const size_t total = (size_t)pixels * channels;
  if (total == 0) return;
  unsigned g = grid_for(total);
  if (g > 4096) g = 4096;
  hipLaunchKernelGGL(minmax_kernel, dim3(g), dim3(256), 0, st, x, pixels, channels, out);
  DW_HIP(hipGetLastError());
}

}  // namespace dw
