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
__device__ __forceinline__ uint16_t f2h(float f) {
  asm("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// F16::to_f32_soft (crates/dragonwing-core/src/dtype.rs:226-263).  It is the
// IEEE decode except for subnormals, which it returns at half their IEEE
// value (the normalising loop leaves the exponent one binade low).
// dragonwing-cpu widens every f16 operand through it, so kernels that must
// reproduce the CPU results bit for bit decode with this function.
__device__ __forceinline__ float h2f(uint16_t b) {
  const float v = h2f_ieee(b);
  return ((b & 0x7C00u) == 0 && (b & 0x03FFu) != 0) ? v * 0.5f : v;
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

}  // namespace dw
