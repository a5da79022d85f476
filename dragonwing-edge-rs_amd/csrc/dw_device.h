// Device-side scalar helpers shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dw {

// IEEE binary16 <-> f32 (hardware conversions; f32 -> f16 rounds to nearest
// even with subnormals, as F16::from_f32_soft does, dtype.rs:164-222).
__device__ __forceinline__ float h2f_ieee(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
// f32 -> f16, round to nearest even, of an f32 value that has been rounded
// to f32.  The empty asm makes the value opaque: without it the compiler
// may fuse the conversion with the fmaf that produced the value into one
// v_fma_mixlo_f16, which rounds the exact sum to f16 once, not to f32 and
// then to f16 as the reference does (the two differ by an f16 ulp when the
// f32 rounding lands on an f16 rounding midpoint).
// A NaN is encoded as F16::from_f32_soft does (dtype.rs:173-178): its sign,
// the quiet bit and the top payload bits clamped below it, sign | 0x7E00 |
// min(mant >> 13, 0x1FF) (so a quiet f32 NaN gives 0x7FFF, where the
// hardware conversion gives 0x7E00).  The packed conversions (pk_f2h) and
// packed f16 arithmetic keep the hardware's NaN encoding.
__device__ __forceinline__ uint16_t f2h(float f) {
  asm("" : "+v"(f));
  const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)f);
  const uint32_t b = __builtin_bit_cast(uint32_t, f);
  const uint32_t nan_bits = ((b >> 16) & 0x8000u) | 0x7E00u | min((b & 0x7FFFFFu) >> 13, 0x1FFu);
  return __builtin_isnan(f) ? (uint16_t)nan_bits : h;
}

// F16::to_f32_soft (crates/dragonwing-core/src/dtype.rs:226-263).  It is the
// IEEE decode except for subnormals, which it returns at half their IEEE
// value (the normalising loop leaves the exponent one binade low).
// dragonwing-cpu widens every f16 operand through it, so kernels that must
// reproduce the CPU results bit for bit decode with this function.
__device__ __forceinline__ float h2f(uint16_t b) {
  // subnormal f16 <=> nonzero |v| < 2^-14; zeros give v * 0.5 = v, and NaN
  // fails the comparison
  const float v = h2f_ieee(b);
  return fabsf(v) < 6.103515625e-05f ? v * 0.5f : v;
}

// f32 -> f16 -> f32: the value the next CPU op sees after an f16 store.
__device__ __forceinline__ float round_f16(float f) { return h2f(f2h(f)); }

// The f16 ops CpuGraphRuntime runs after a conv, on stored f16 bits: each
// op widens its inputs with to_f32 and stores F16::from_f32 of its result.
// bias add (runtime.rs:1483-1498): F16(f32(y) + f32(b))
__device__ __forceinline__ uint16_t f16_add_bits(uint16_t a, uint16_t b) {
  return f2h(h2f(a) + h2f(b));
}
// relu_fp16 (ops.rs:345-352), or sigmoid_fp16 then mul_fp16 (ops.rs:1881,
// :1959) for SiLU.  act: 0 none, 1 relu, 2 silu.
__device__ __forceinline__ uint16_t f16_act_bits(uint16_t hb, int act) {
  if (act == 1) {
    const float v = h2f(hb);
    return f2h(v > 0.0f ? v : 0.0f);
  }
  if (act == 2) {
    const float v = h2f(hb);
    const uint16_t s = f2h(1.0f / (1.0f + expf(-v)));
    return f2h(v * h2f(s));
  }
  return hb;
}

// SiLU of an f16 value for the fp16 paths held to the fp16 tolerance: the
// reference's steps (sigmoid in f32, rounded to f16, times x, rounded to
// f16) with exp and the reciprocal from the hardware's exp2 and rcp, each
// refined to about an f32 ulp: exp(-x) = 2^hi * (1 + lo ln 2) with hi + lo
// = -x log2(e) split exactly by an fma, and one Newton step on 1 / (1 + e).
// Operands are widened as IEEE f16 (the reference halves subnormals; a
// subnormal x only changes an output below 2^-14 in magnitude).
__device__ __forceinline__ uint16_t silu_f16_fast(uint16_t hb) {
  const float x = h2f_ieee(hb);
  const float hi = x * -1.44269502f;
  const float lo = fmaf(x, -1.44269502f, -hi) + x * -1.92596299e-08f;
  float e = __builtin_amdgcn_exp2f(hi);
  e = fmaf(e, lo * 0.693147182f, e);
  const float d = 1.0f + e;
  float r = __builtin_amdgcn_rcpf(d);
  r = fmaf(r, fmaf(-d, r, 1.0f), r);
  const uint16_t s = f2h(r);
  return f2h(x * h2f_ieee(s));
}

// Two f16 values in one 32-bit register (element 0 in the low half); the
// arithmetic operators on it are the packed f16 instructions, correctly
// rounded with f16 subnormals kept.
typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint16_t pk_lo(h16x2 v) { return (uint16_t)__builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ uint16_t pk_hi(h16x2 v) { return (uint16_t)(__builtin_bit_cast(uint32_t, v) >> 16); }
__device__ __forceinline__ h16x2 pk_make(uint16_t lo, uint16_t hi) {
  return __builtin_bit_cast(h16x2, (uint32_t)lo | ((uint32_t)hi << 16));
}
// f2h of two values (each rounded to f32 first, as f2h requires)
__device__ __forceinline__ h16x2 pk_f2h(float a, float b) {
  asm("" : "+v"(a));
  asm("" : "+v"(b));
  return h16x2{(_Float16)a, (_Float16)b};
}

// SiLU of two f16 values for the fp16-tolerance paths, fewer instructions
// than silu_f16_fast: exp(-x) = 2^h * (1 + r) with h = -x log2(e) rounded to
// f32 and r = -x - h ln 2 its residual (ln 2 in two parts, Cody-Waite), then
// one rcp of 1 + exp(-x) (1 ulp); the sigmoid is rounded to f16 and the
// product x * s of two f16 values (exact in f32, so one rounding) is one
// packed f16 multiply.
__device__ __forceinline__ h16x2 silu_f16_pk(h16x2 x) {
  float r[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float v = (float)x[i];
    const float h = v * -1.44269502f;
    float res = fmaf(-h, 0.693145751953125f, -v);
    res = fmaf(-h, 1.42860677e-06f, res);
    float e = __builtin_amdgcn_exp2f(h);
    e = fmaf(e, res, e);
    r[i] = __builtin_amdgcn_rcpf(1.0f + e);
  }
  return x * pk_f2h(r[0], r[1]);
}

// The same SiLU without the residual correction: exp(-x) = 2^h with h =
// -x log2(e) rounded to f32, whose rounding error (|h| 2^-24 relative in
// the exponent) moves the sigmoid by under 2^-20 relative for |x| < 20,
// well inside the f16 rounding of the result (2^-12); used where the
// output is held to the fp16 tolerance and the vector ALUs bound the
// kernel (the depthwise conv).
__device__ __forceinline__ h16x2 silu_f16_pk_lite(h16x2 x) {
  float r[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float e = __builtin_amdgcn_exp2f((float)x[i] * -1.44269502f);
    r[i] = __builtin_amdgcn_rcpf(1.0f + e);
  }
  return x * pk_f2h(r[0], r[1]);
}

// The u8 -> f16 1x1 convolution's per-lane pieces (conv1x1_u8_f16_mfma_kernel
// and the igemm epilogue that runs the same conv on a tile's u8 results):
// DequantizeLinear of 8 bytes, f16((q - zp) * scale) with the product
// rounded to f32 first (byte j -> element j), and the f16 epilogue of one
// lane's 4 accumulators (rounded to f16 two at a time, the f16 bias added,
// the activation), as the two 32-bit words the lane stores.
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f16x8 dequant_u8x8_f16(uint2 u, float zp, float scale) {
  f16x8 r;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t w = j < 4 ? u.x : u.y;
    const float q = (float)((w >> (8 * (j & 3))) & 0xffu);
    float f = (q - zp) * scale;
    asm("" : "+v"(f));  // round the product to f32 before the f16 conversion
    r[j] = (_Float16)f;
  }
  return r;
}
__device__ __forceinline__ uint2 conv1x1_f16_finish(f32x4 acc, const uint16_t* bias4, int act) {
  h16x2 lo = pk_f2h(acc[0], acc[1]), hi = pk_f2h(acc[2], acc[3]);
  if (bias4) {
    lo = lo + __builtin_bit_cast(h16x2, *reinterpret_cast<const uint32_t*>(bias4));
    hi = hi + __builtin_bit_cast(h16x2, *reinterpret_cast<const uint32_t*>(bias4 + 2));
  }
  if (act == ACT_SILU) {
    lo = silu_f16_pk_lite(lo);
    hi = silu_f16_pk_lite(hi);
  } else if (act == ACT_RELU) {
    lo = pk_make(f16_act_bits(pk_lo(lo), ACT_RELU), f16_act_bits(pk_hi(lo), ACT_RELU));
    hi = pk_make(f16_act_bits(pk_lo(hi), ACT_RELU), f16_act_bits(pk_hi(hi), ACT_RELU));
  }
  return make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
}

// acc + (f16 half SEL of x) * (f16 half SEL of w), fused, in f32: the f16
// values widen exactly (subnormals at their IEEE value).  One v_fma_mix per
// product; written out because the compiler otherwise widens reused
// operands with separate conversions.
template <int SEL>
__device__ __forceinline__ float fma_mix_h(uint32_t x, uint32_t w, float acc) {
  if constexpr (SEL == 0)
    asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel_hi:[1,1,0]" : "+v"(acc) : "v"(x), "v"(w));
  else
    asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel:[1,1,0] op_sel_hi:[1,1,0]" : "+v"(acc) : "v"(x), "v"(w));
  return acc;
}
// (f16 half SEL of x) * (f16 half SEL of w) + 0: the first product of a
// chain that starts at +0 (+0 + -0 is +0, as fma gives)
template <int SEL>
__device__ __forceinline__ float fma_mix_h0(uint32_t x, uint32_t w) {
  float r;
  if constexpr (SEL == 0)
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,1,0]" : "=v"(r) : "v"(x), "v"(w));
  else
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,1,0] op_sel_hi:[1,1,0]" : "=v"(r) : "v"(x), "v"(w));
  return r;
}
// the same with an f32 weight
template <int SEL>
__device__ __forceinline__ float fma_mix_hf(uint32_t x, float w, float acc) {
  if constexpr (SEL == 0)
    asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel_hi:[1,0,0]" : "+v"(acc) : "v"(x), "v"(w));
  else
    asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(acc) : "v"(x), "v"(w));
  return acc;
}
template <int SEL>
__device__ __forceinline__ float fma_mix_hf0(uint32_t x, float w) {
  float r;
  if constexpr (SEL == 0)
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(x), "v"(w));
  else
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(x), "v"(w));
  return r;
}

}  // namespace dw
