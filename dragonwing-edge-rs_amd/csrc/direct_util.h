// Device helpers shared by the exact-order convolution kernels (k_direct.hip,
// k_direct1x1.hip): input decoding and the fused output stage, each as
// dragonwing-cpu computes it.
#pragma once

#include "dw_common.h"
#include "dw_device.h"

namespace dw {
namespace dx {

// relu_f32_scalar (ops.rs:208-220): x > 0 -> x, NaN -> NaN, else +0.
__device__ __forceinline__ float relu_ref(float v) { return v > 0.0f ? v : (v != v ? v : 0.0f); }

// u8 -> the f32 value a conv reads after DequantizeLinear to f16:
// F16((q - zp) * scale), widened with the reference decode.
__device__ __forceinline__ float dequant_f16(int q, int zp, float scale) {
  return round_f16((float)(q - zp) * scale);
}

// One input element as the reference conv reads it.
template <int IN_KIND>
__device__ __forceinline__ float load1(const DirectArgs& a, const uint8_t* p) {
  if (IN_KIND == 0) return *reinterpret_cast<const float*>(p);
  if (IN_KIND == 1) return h2f(*reinterpret_cast<const uint16_t*>(p));
  return dequant_f16((int)*p, a.in_zp, a.in_scale);
}

// Elements per 16-byte input vector.
template <int IN_KIND>
__host__ __device__ constexpr int vec_elems() {
  return IN_KIND == 0 ? 4 : (IN_KIND == 1 ? 8 : 16);
}

// Element e of a raw 16-byte vector of consecutive input channels, decoded.
template <int IN_KIND>
__device__ __forceinline__ float decode_elem(const DirectArgs& a, const uint4& u, int e) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
  if (IN_KIND == 0) return __builtin_bit_cast(float, w[e]);
  if (IN_KIND == 1) return h2f((w[e >> 1] >> (16 * (e & 1))) & 0xffff);
  return dequant_f16((int)((w[e >> 2] >> (8 * (e & 3))) & 0xff), a.in_zp, a.in_scale);
}

// A 16-byte vector of consecutive input channels, decoded.
template <int IN_KIND>
__device__ __forceinline__ void load_vec(const DirectArgs& a, const uint8_t* p, float* v) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
#pragma unroll
  for (int e = 0; e < vec_elems<IN_KIND>(); ++e) v[e] = decode_elem<IN_KIND>(a, u, e);
}

// The rest of the fused group for OC accumulators of one pixel (output
// channels oc0..oc0+OC-1), stored at yb, for one output type OUT: 0 = f32
// (bias pass, ReLU or SiLU), 1 = f16 (conv result rounded, bias pass and
// activation on stored f16), 2 = u8 (QuantizeLinear of the stored f16
// value, optional table).  Values are packed into 32-bit words and stored
// 16 or 4 bytes at a time when the view allows (a.vec_out), else element by
// element.  One instantiation per output type keeps each unrolled loop
// small, so acc and words stay in registers.
// FE (a.fast_epi set by the host): the f16 values are widened as IEEE f16
// (one instruction) and the quantization rounds by adding 1.5 * 2^23 and
// clamps with one med3 on the float (as requant_bits in igemm_kernel.h).
// lut: the activation table (LDS or global); a.lut when null.
//
// u8 quantization of the IEEE value xv of a stored f16 (FE): the integer
// rint(xv / out_scale) + zp clamped to 0..255, as its low byte.  PLAIN: the
// host checked that xv * (1 / out_scale) rounds to the same integer for
// every finite f16 xv, so the correction FMAs are left out.
template <bool PLAIN>
__device__ __forceinline__ int quant_u8_fe(const DirectArgs& a, float xv) {
  const float q0 = xv * a.out_rcp;
  float d = q0;
  if constexpr (!PLAIN) {
    const float dc = fmaf(fmaf(-q0, a.out_scale, xv), a.out_rcp, q0);
    d = fabsf(xv) <= 65504.0f ? dc : q0;  // inf * rcp is the quotient too
  }
  const float lo = 12582912.0f - (float)a.out_zp;
  const int qb = __builtin_bit_cast(int, __builtin_amdgcn_fmed3f(d + 12582912.0f, lo, lo + 255.0f));
  return (qb - (0x4B400000 - a.out_zp)) & 0xff;  // the clamp makes it 0..255 (the mask keeps table reads in range)
}

// The u8 epilogue when a.epi_pk is set: the conv results are rounded to
// f16 two at a time and the bias pass F16(f32(y) + f32(b)) is one packed
// f16 add (f32 holds the sum of two f16 values to 2 * 11 + 2 bits, so
// rounding it to f16 is the correctly rounded f16 sum).  Exact when neither
// y nor b is an f16 subnormal (the reference decodes those at half value):
// the host checked the biases, and the caller checks the results.  The sum
// is then quantized as an IEEE value: a subnormal sum quantizes to the zero
// point either way, since the host also checked out_scale >= 2^-13.
template <int OC, bool PLAIN>
__device__ __forceinline__ void quant_pairs_fe(const DirectArgs& a, const float* acc, int oc0, const uint8_t* lut,
                                               uint32_t* words) {
#pragma unroll
  for (int j = 0; j < OC; j += 2) {
    h16x2 p = pk_f2h(acc[j], acc[j + 1]);
    if (a.bias_h) p = p + *reinterpret_cast<const h16x2*>(a.bias_h + oc0 + j);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      int qi = quant_u8_fe<PLAIN>(a, (float)p[i]);
      if (a.lut) qi = lut[qi];
      words[(j + i) >> 2] |= (uint32_t)qi << (8 * ((j + i) & 3));
    }
  }
}

template <int OUT, int OC, bool FE = false>
__device__ __forceinline__ void store_outputs_t(const DirectArgs& a, const float* acc, int oc0, uint8_t* yb,
                                                const uint8_t* lut = nullptr) {
  constexpr int OES = OUT == 0 ? 4 : (OUT == 1 ? 2 : 1);
  constexpr int NW = (OC * OES + 3) / 4;
  uint32_t words[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) words[i] = 0;
  if constexpr (OUT == 1 && OC % 2 == 0) {
    // f16 out, no activation or SiLU: the same packed rounding and bias
    // pass; SiLU (held to the fp16 tolerance, as every expf-based output)
    // two values at a time
    float amin = fabsf(acc[0]);
#pragma unroll
    for (int j = 1; j < OC; ++j) amin = fminf(amin, fabsf(acc[j]));
    if (a.epi_pk && (a.act == ACT_NONE || a.act == ACT_SILU) && a.vec_out != 1 &&
        !__any(amin < 6.103515625e-05f)) {
#pragma unroll
      for (int j = 0; j < OC; j += 2) {
        h16x2 p = pk_f2h(acc[j], acc[j + 1]);
        if (a.bias_h) p = p + *reinterpret_cast<const h16x2*>(a.bias_h + oc0 + j);
        if (a.act == ACT_SILU) p = silu_f16_pk(p);
        words[j >> 1] = __builtin_bit_cast(uint32_t, p);
      }
      if (a.vec_out == 16) {
#pragma unroll
        for (int i = 0; i < NW / 4; ++i)
          *reinterpret_cast<uint4*>(yb + 16 * i) =
              make_uint4(words[4 * i], words[4 * i + 1], words[4 * i + 2], words[4 * i + 3]);
      } else {
#pragma unroll
        for (int i = 0; i < NW; ++i) *reinterpret_cast<uint32_t*>(yb + 4 * i) = words[i];
      }
      return;
    }
  }
  if constexpr (OUT == 2 && OC % 4 == 0) {
    // no result that rounds to an f16 subnormal (|acc| < 2^-14) anywhere
    // in the wave: else the wave takes the per-channel path below
    float amin = fabsf(acc[0]);
#pragma unroll
    for (int j = 1; j < OC; ++j) amin = fminf(amin, fabsf(acc[j]));
    if (a.epi_pk && a.vec_out != 1 && !__any(amin < 6.103515625e-05f)) {
      const uint8_t* lt = lut ? lut : a.lut;
      if (a.out_plain)
        quant_pairs_fe<OC, true>(a, acc, oc0, lt, words);
      else
        quant_pairs_fe<OC, false>(a, acc, oc0, lt, words);
      if (a.vec_out == 16) {
#pragma unroll
        for (int i = 0; i < NW / 4; ++i)
          *reinterpret_cast<uint4*>(yb + 16 * i) =
              make_uint4(words[4 * i], words[4 * i + 1], words[4 * i + 2], words[4 * i + 3]);
      } else {
#pragma unroll
        for (int i = 0; i < NW; ++i) *reinterpret_cast<uint32_t*>(yb + 4 * i) = words[i];
      }
      return;
    }
  }
#pragma unroll
  for (int j = 0; j < OC; ++j) {
    if constexpr (OUT == 0) {
      float v = acc[j];
      if (a.bias_f) v = v + a.bias_f[oc0 + j];
      if (a.act == ACT_RELU) {
        v = relu_ref(v);
      } else if (a.act == ACT_SILU) {
        const float s = 1.0f / (1.0f + expf(-v));
        v = v * s;
      }
      words[j] = __builtin_bit_cast(uint32_t, v);
      if (a.vec_out == 1) reinterpret_cast<float*>(yb)[j] = v;
    } else if constexpr (OUT == 1) {
      uint16_t hb = f2h(acc[j]);
      if (a.bias_hf)
        hb = f2h((FE ? h2f_ieee(hb) : h2f(hb)) + a.bias_hf[oc0 + j]);
      else if (a.bias_h)
        hb = f16_add_bits(hb, a.bias_h[oc0 + j]);
      const uint16_t ob = f16_act_bits(hb, a.act);
      words[j >> 1] |= (uint32_t)ob << (16 * (j & 1));
      if (a.vec_out == 1) reinterpret_cast<uint16_t*>(yb)[j] = ob;
    } else {
      uint16_t hb = f2h(acc[j]);
      if (a.bias_hf)
        hb = f2h((FE ? h2f_ieee(hb) : h2f(hb)) + a.bias_hf[oc0 + j]);
      else if (a.bias_h)
        hb = f16_add_bits(hb, a.bias_h[oc0 + j]);
      // QuantizeLinear of the stored f16 value: x / scale, correctly rounded
      // (reciprocal + one FMA correction where the host proved that equal for
      // every finite f16 x; the division otherwise).
      int qi;
      if constexpr (FE) {
        const float xv = h2f_ieee(hb);
        const float q0 = xv * a.out_rcp;
        const float dc = fmaf(fmaf(-q0, a.out_scale, xv), a.out_rcp, q0);
        const float d = fabsf(xv) <= 65504.0f ? dc : q0;  // inf * rcp is the quotient too
        const float lo = 12582912.0f - (float)a.out_zp;
        const int qb = __builtin_bit_cast(int, __builtin_amdgcn_fmed3f(d + 12582912.0f, lo, lo + 255.0f));
        qi = (qb - (0x4B400000 - a.out_zp)) & 0xff;  // the clamp makes it 0..255 (the mask keeps table reads in range)
      } else {
        const float xv = h2f(hb);
        float d;
        if (a.out_fast && fabsf(xv) <= 65504.0f) {
          const float q0 = xv * a.out_rcp;
          d = fmaf(fmaf(-q0, a.out_scale, xv), a.out_rcp, q0);
        } else {
          d = __fdiv_rn(xv, a.out_scale);
        }
        float q = rintf(d) + (float)a.out_zp;
        q = __builtin_amdgcn_fmed3f(q, 0.0f, 255.0f);
        qi = (int)q;
      }
      if (a.lut) qi = (lut ? lut : a.lut)[qi];
      words[j >> 2] |= (uint32_t)qi << (8 * (j & 3));
      if (a.vec_out == 1) yb[j] = (uint8_t)qi;
    }
  }
  if (a.vec_out == 16) {
#pragma unroll
    for (int i = 0; i < NW / 4; ++i)
      *reinterpret_cast<uint4*>(yb + 16 * i) =
          make_uint4(words[4 * i], words[4 * i + 1], words[4 * i + 2], words[4 * i + 3]);
  } else if (a.vec_out == 4) {
#pragma unroll
    for (int i = 0; i < NW; ++i) *reinterpret_cast<uint32_t*>(yb + 4 * i) = words[i];
  }
}

// All output types (run-time choice) for a single accumulator set.
template <int OC>
__device__ __forceinline__ void store_outputs(const DirectArgs& a, const float* acc, int oc0, uint8_t* yb) {
  if (a.out_kind == 0)
    store_outputs_t<0, OC>(a, acc, oc0, yb);
  else if (a.out_kind == 1)
    store_outputs_t<1, OC>(a, acc, oc0, yb);
  else
    store_outputs_t<2, OC>(a, acc, oc0, yb);
}

}  // namespace dx

// The 1x1 exact-order kernel (k_direct1x1.hip); false if the problem is not
// one it handles.
bool launch_conv1x1_exact(hipStream_t st, const DirectArgs& a);

}  // namespace dw
