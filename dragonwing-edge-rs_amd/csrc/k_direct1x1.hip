// 1x1 convolution (no padding, any stride) with dragonwing-cpu's
// accumulation order, bit-identical to the CPU implementation:
//   acc = 0; for ic: acc = fma(x[ic], w[ic][oc], acc)       (f32, single rounding)
// (crates/dragonwing-cpu/src/ops.rs:1356-1436, :2572-2651, 1x1 case).  This
// is the detect head's last layers in the int8 graph (u8 input dequantized
// to f16, f16 output), which must match the CPU bit for bit.
//
// A register-blocked outer product on the vector ALUs: one wavefront owns
// 64*P output pixels and a group of C output channels; each lane keeps
// P x C accumulators (P pixels, lane-strided, x C channels), so every decoded
// input value feeds C FMAs and every weight P FMAs.  Weights are
// wave-uniform and come through scalar loads (SGPR operands), so the FMA
// loop uses no LDS at all.
// Input vectors (16 bytes of consecutive channels) are prefetched one
// vector ahead.  The FMA chain of each output runs over ic in order, as in
// the reference; only independent chains are interleaved.
#include "direct_util.h"

#include <stdio.h>
#include <stdlib.h>

#include <math.h>

#include <algorithm>

namespace dw {
namespace {

// Weights through the constant address space: wave-uniform rows, fetched
// with scalar loads into SGPR operands.
typedef const __attribute__((address_space(4))) float* wrow_t;

// Input element e of a raw 16-byte vector.  NOSUB (u8 input only): the
// dequantized value can never be an f16 subnormal (scale >= 2^-14), so the
// reference's subnormal decode rule is compiled out, and the value (a
// function of the byte alone) is read from a 256-entry table in LDS that
// the workgroup fills first: one address computation and one LDS read per
// input instead of five conversions.
template <int IN_KIND, bool NOSUB>
__device__ __forceinline__ float decode_x(const DirectArgs& a, const uint4& u, int e, const float* s_deq) {
  if constexpr (IN_KIND == 2 && NOSUB) {
    const uint32_t wd = e < 4 ? u.x : (e < 8 ? u.y : (e < 12 ? u.z : u.w));
    return s_deq[(wd >> (8 * (e & 3))) & 0xff];
  } else {
    return dx::decode_elem<IN_KIND>(a, u, e);
  }
}

// PK: the weights come from a.wq16 ([c_out / 16][c_in][16], C = 16), so the
// rows of one group are consecutive 64-byte lines and a block's 16 scalar
// loads take immediate offsets from one base: no address arithmetic per row.
template <int IN_KIND, int C, int P, bool NOSUB, bool PK>
__global__ __launch_bounds__(64) void conv1x1_exact_kernel(const DirectArgs a) {
  static_assert(!PK || C == 16, "packed rows hold 16 channels");
  constexpr int ES = IN_KIND == 0 ? 4 : (IN_KIND == 1 ? 2 : 1);
  constexpr int VN = dx::vec_elems<IN_KIND>();
  const int K = a.cin;
  const int oc0 = blockIdx.y * C;
  const int lane = threadIdx.x;
  const int wstride = PK ? C : a.cout;  // floats between consecutive weight rows
  const wrow_t wbase = PK ? (wrow_t)(a.wq16 + (size_t)blockIdx.y * K * C) : (wrow_t)(a.wf + oc0);
  // u8 -> f32 of the f16 dequantized value, (q - zp) * scale rounded to f16
  __shared__ float s_deq[IN_KIND == 2 && NOSUB ? 256 : 1];
  if constexpr (IN_KIND == 2 && NOSUB) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = lane * 4 + i;
      s_deq[q] = h2f_ieee(f2h((float)(q - a.in_zp) * a.in_scale));
    }
    __syncthreads();
  }

  // this lane's pixels: p = tile*64P + j*64 + lane
  const uint8_t* xp[P];
  bool pv[P];
  int pix[P];
  const int hw = a.ho * a.wo;
#pragma unroll
  for (int j = 0; j < P; ++j) {
    const int p = blockIdx.x * (64 * P) + j * 64 + lane;
    pv[j] = p < a.m;
    const int pp = pv[j] ? p : 0;
    pix[j] = pp;
    const int nn = pp / hw;
    const int r = pp - nn * hw;
    const int oh = r / a.wo;
    const int ow = r - oh * a.wo;
    xp[j] = (const uint8_t*)a.x +
            (((size_t)(nn * a.h + oh * a.sh) * a.w + ow * a.sw) * a.x_pix_stride + a.x_c_off) * ES;
  }

  float acc[P][C];
#pragma unroll
  for (int j = 0; j < P; ++j)
#pragma unroll
    for (int c = 0; c < C; ++c) acc[j][c] = 0.0f;

  uint4 cur[P], nxt[P];
#pragma unroll
  for (int j = 0; j < P; ++j) cur[j] = *reinterpret_cast<const uint4*>(xp[j]);
  wrow_t wk = wbase;  // weight row k0
  for (int k0 = 0; k0 < K; k0 += VN, wk += (size_t)VN * wstride) {
    // prefetch the next vector (the last iteration reloads the first one)
    const int kn = k0 + VN < K ? k0 + VN : 0;
#pragma unroll
    for (int j = 0; j < P; ++j) nxt[j] = *reinterpret_cast<const uint4*>(xp[j] + (size_t)kn * ES);
#pragma unroll
    for (int e = 0; e < VN; ++e) {
      float xv[P];
#pragma unroll
      for (int j = 0; j < P; ++j) xv[j] = decode_x<IN_KIND, NOSUB>(a, cur[j], e, s_deq);
      const wrow_t wr = PK ? wk + e * C : wk + (size_t)e * wstride;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const float wv = wr[c];
#pragma unroll
        for (int j = 0; j < P; ++j) acc[j][c] = fmaf(xv[j], wv, acc[j][c]);
      }
    }
#pragma unroll
    for (int j = 0; j < P; ++j) cur[j] = nxt[j];
  }

  // one loop per output type (each small enough to unroll)
#define DW_STORE(OUT, OES)                                                         \
  _Pragma("unroll") for (int j = 0; j < P; ++j) {                                  \
    if (!pv[j]) continue;                                                          \
    const size_t yo = (size_t)pix[j] * a.y_pix_stride + a.y_c_off + oc0;           \
    dx::store_outputs_t<OUT, C>(a, acc[j], oc0, (uint8_t*)a.y + yo * (OES));       \
  }
  if (a.out_kind == 0) {
    DW_STORE(0, 4)
  } else if (a.out_kind == 1) {
    DW_STORE(1, 2)
  } else {
    DW_STORE(2, 1)
  }
#undef DW_STORE
}

}  // namespace

bool launch_conv1x1_exact(hipStream_t st, const DirectArgs& a_in) {
  if (a_in.kh != 1 || a_in.kw != 1 || a_in.pt != 0 || a_in.pl != 0) return false;
  const int es = a_in.in_kind == 0 ? 4 : (a_in.in_kind == 1 ? 2 : 1);
  const int vn = 16 / es;
  if (a_in.cin % vn != 0 || (a_in.x_pix_stride * es) % 16 != 0 || (a_in.x_c_off * es) % 16 != 0 ||
      ((uintptr_t)a_in.x & 15) != 0)
    return false;
  // Channels per wave C and pixels per lane P.  Measured on the detect-head
  // shapes (u8 -> f16, 64 and 80 channels, 40x40 to 80x80, batch 32), one
  // pixel per lane with 16 channels is fastest: the wave keeps few
  // registers, so many waves per SIMD hide the scalar weight loads and the
  // input loads, and each decoded input still feeds 16 FMAs.  Narrower
  // groups are used when c_out needs them or the layer has too few pixels
  // for one wave per SIMD.  The grid runs all pixel tiles of one channel
  // group before the next, so the waves in flight share one group's weights
  // in the scalar cache.
  struct Opt {
    int c, p;
  };
  static const Opt opts[] = {{20, 4}, {16, 4}, {40, 2}, {32, 2}, {8, 4}, {40, 1}, {20, 1}, {16, 1},
                             {4, 4},  {8, 1},  {4, 1}};
  const bool nosub = a_in.in_kind == 2 && fabsf(a_in.in_scale) >= 6.103515625e-05f;
  Opt best{0, 0};
  for (int c : {16, 8, 4})
    if (a_in.cout % c == 0) {
      best = {c, 1};
      const long waves = (long)((a_in.m + 63) / 64) * (a_in.cout / c);
      if (waves >= 1024) break;
    }
  // Override for tests and tuning runs: "C,P", applied where valid.
  if (const char* env = getenv("DW_DIRECT1X1")) {
    int c = 0, pp = 0;
    if (sscanf(env, "%d,%d", &c, &pp) == 2)
      for (const Opt& o : opts)
        if (o.c == c && o.p == pp && a_in.cout % c == 0) best = o;
  }
  if (!best.c) return false;
  DirectArgs a = a_in;
  const int oes = a.out_kind == 0 ? 4 : (a.out_kind == 1 ? 2 : 1);
  auto aligned = [&](int v) {
    return (best.c * oes) % v == 0 && (a.y_pix_stride * oes) % v == 0 && (a.y_c_off * oes) % v == 0 &&
           ((uintptr_t)a.y % v) == 0;
  };
  a.vec_out = aligned(16) ? 16 : (aligned(4) ? 4 : 1);
  const dim3 grid((a.m + 64 * best.p - 1) / (64 * best.p), a.cout / best.c);
  const bool pk = best.c == 16 && a.wq16 != nullptr;
#define DW_K(KIND, CC, PP, NS)                                                                    \
  if (a.in_kind == KIND && best.c == CC && best.p == PP && nosub == NS) {                           \
    if (CC == 16 && pk)                                                                             \
      hipLaunchKernelGGL((conv1x1_exact_kernel<KIND, CC, PP, NS, CC == 16>), grid, dim3(64), 0, st, a); \
    else                                                                                            \
      hipLaunchKernelGGL((conv1x1_exact_kernel<KIND, CC, PP, NS, false>), grid, dim3(64), 0, st, a); \
    DW_HIP(hipGetLastError());                                                                      \
    return true;                                                                                    \
  }
#define DW_K_ALL(CC, PP) DW_K(0, CC, PP, false) DW_K(1, CC, PP, false) DW_K(2, CC, PP, false) DW_K(2, CC, PP, true)
  DW_K_ALL(20, 4)
  DW_K_ALL(16, 4)
  DW_K_ALL(40, 2)
  DW_K_ALL(32, 2)
  DW_K_ALL(8, 4)
  DW_K_ALL(40, 1)
  DW_K_ALL(20, 1)
  DW_K_ALL(16, 1)
  DW_K_ALL(4, 4)
  DW_K_ALL(8, 1)
  DW_K_ALL(4, 1)
#undef DW_K_ALL
#undef DW_K
  return false;
}

}  // namespace dw
