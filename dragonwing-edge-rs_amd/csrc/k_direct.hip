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
#include "direct_util.h"

namespace dw {
namespace {


// Weights are read through the constant address space: the row for one
// (tap, ic) is the same for every lane of a wavefront, so the compiler
// fetches it with scalar loads and each FMA takes its weight from an SGPR
// (no LDS traffic, no per-lane weight loads).
typedef const __attribute__((address_space(4))) float* wrow_t;

using dx::load1;
using dx::load_vec;
using dx::relu_ref;
using dx::vec_elems;

// One thread = one output pixel x OC consecutive output channels; all OC
// accumulators consume each decoded input value, so the decode is paid once
// per OC FMAs.  Per output the FMA sequence is the reference's.  VIN: the
// input rows are 16-byte aligned and c_in is a whole number of vectors.
template <int IN_KIND, int OC, bool VIN>
__global__ __launch_bounds__(256) void direct_conv_kernel(const DirectArgs a) {
  constexpr int ES = IN_KIND == 0 ? 4 : (IN_KIND == 1 ? 2 : 1);
  constexpr int VN = vec_elems<IN_KIND>();
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= a.m) return;
  const int oc0 = blockIdx.y * OC;
  const int hw = a.ho * a.wo;
  const int nn = p / hw;
  const int rem = p - nn * hw;
  const int oh = rem / a.wo;
  const int ow = rem - oh * a.wo;
  const int cin = a.cin, cout = a.cout;
  const uint8_t* __restrict__ X = (const uint8_t*)a.x;
  const wrow_t wbase = (wrow_t)(a.wf + oc0);

  float acc[OC];
#pragma unroll
  for (int j = 0; j < OC; ++j) acc[j] = 0.0f;

  for (int kh = 0; kh < a.kh; ++kh) {
    const int ih = oh * a.sh + kh - a.pt;
    if (ih < 0 || ih >= a.h) continue;
    for (int kw = 0; kw < a.kw; ++kw) {
      const int iw = ow * a.sw + kw - a.pl;
      if (iw < 0 || iw >= a.w) continue;
      const uint8_t* xp = X + (((size_t)(nn * a.h + ih) * a.w + iw) * a.x_pix_stride + a.x_c_off) * ES;
      const wrow_t wt = wbase + (size_t)(kh * a.kw + kw) * cin * cout;
      if constexpr (VIN) {
        for (int ic = 0; ic < cin; ic += VN) {
          float xv[VN];
          load_vec<IN_KIND>(a, xp + (size_t)ic * ES, xv);
#pragma unroll
          for (int e = 0; e < VN; ++e) {
            const wrow_t wr = wt + (size_t)(ic + e) * cout;
#pragma unroll
            for (int j = 0; j < OC; ++j) acc[j] = fmaf(xv[e], wr[j], acc[j]);
          }
        }
      } else {
        for (int ic = 0; ic < cin; ++ic) {
          const float xv = load1<IN_KIND>(a, xp + (size_t)ic * ES);
          const wrow_t wr = wt + (size_t)ic * cout;
#pragma unroll
          for (int j = 0; j < OC; ++j) acc[j] = fmaf(xv, wr[j], acc[j]);
        }
      }
    }
  }

  // Epilogue: the rest of the fused group, packed stores.
  const int OES = a.out_kind == 0 ? 4 : (a.out_kind == 1 ? 2 : 1);
  const size_t yo = (size_t)p * a.y_pix_stride + a.y_c_off + oc0;
  dx::store_outputs<OC>(a, acc, oc0, (uint8_t*)a.y + yo * OES);
}

// Small-kernel, few-channel case (the 3-channel stem): KH x KW x CIN known
// at compile time.  One thread = one output pixel x OC channels.  All
// KH*KW*CIN input values are loaded up front (out-of-image taps read a
// clamped in-image address and are then skipped), decoded once, and fed to
// OC FMA chains in the reference order, skipping out-of-image taps exactly
// as the reference does.  Weights come through scalar loads (SGPR operands).
// PAR >= 0 (f16 input, 3 channels, dense rows, even column stride): the 9
// values of one filter row are 18 contiguous bytes at a 2-byte offset of
// parity PAR; they come in with five 4-byte buffer loads from the 4-byte
// boundary at or below them (15 loads per output instead of 27; a load
// outside the buffer returns zeros, and out-of-image taps are skipped as
// always).
template <int IN_KIND, int OC, int KH, int KW, int CIN, bool FE, int PAR>
__global__ __launch_bounds__(256) void conv_small_kernel(const DirectArgs a) {
  static_assert(PAR < 0 || (IN_KIND == 1 && KW == 3 && CIN == 3), "row loads: f16, 3x3 taps of 3 channels");
  constexpr int ES = IN_KIND == 0 || IN_KIND == 3 ? 4 : (IN_KIND == 1 ? 2 : 1);
  constexpr int KT = KH * KW;
  // the activation table in LDS (one byte per thread)
  __shared__ uint8_t s_lut[256];
  if (a.lut) s_lut[threadIdx.x] = a.lut[threadIdx.x];
  __syncthreads();
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= a.m) return;
  const int oc0 = blockIdx.y * OC;
  const int hw = a.ho * a.wo;
  const int nn = p / hw;
  const int rem = p - nn * hw;
  const int oh = rem / a.wo;
  const int ow = rem - oh * a.wo;
  const int ih0 = oh * a.sh - a.pt, iw0 = ow * a.sw - a.pl;
  const uint8_t* __restrict__ X = (const uint8_t*)a.x;
  float xv[KT][CIN];
  bool ok[KT];
  if constexpr (PAR >= 0) {
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, a.x_bytes, 0x00020000);
#pragma unroll
    for (int kh = 0; kh < KH; ++kh) {
      const int ih = ih0 + kh;
      const bool rv = (unsigned)ih < (unsigned)a.h;
      // half index of the row's first value, less PAR: a 4-byte boundary
      const int off = rv ? (((nn * a.h + ih) * a.w + iw0) * 3 - PAR) * 2 : (int)0x80000000;
      // five 4-byte loads.  The row of image 0's first pixel row starts 8
      // bytes before the buffer when iw0 < 0: each load's offset is formed
      // here, and a negative one is sent out of range (a negative voffset
      // plus an immediate offset is not wrapped back into range).
      uint32_t dw[5];
#pragma unroll
      for (int i = 0; i < 5; ++i) {
        const int o = off + 4 * i;
        dw[i] = __builtin_amdgcn_raw_buffer_load_b32(xr, o < 0 ? (int)0x80000000 : o, 0, 0);
      }
#pragma unroll
      for (int kw = 0; kw < KW; ++kw) {
        ok[kh * KW + kw] = rv && (unsigned)(iw0 + kw) < (unsigned)a.w;
#pragma unroll
        for (int ic = 0; ic < CIN; ++ic) {
          const int hi = PAR + kw * 3 + ic;  // half index in the 20 loaded bytes
          xv[kh * KW + kw][ic] = h2f((uint16_t)(dw[hi >> 1] >> (16 * (hi & 1))));
        }
      }
    }
  } else if constexpr (IN_KIND == 3) {
    // NCHW f32 planes (the graph's input before the layout pass): each value
    // is rounded to f16 as F16::from_f32 stores it and widened with the
    // reference decode, i.e. exactly the f16 NHWC input the host conversion
    // would have produced.
    const float* Xf = (const float*)a.x;
    const size_t plane = (size_t)a.h * a.w;
#pragma unroll
    for (int kh = 0; kh < KH; ++kh)
#pragma unroll
      for (int kw = 0; kw < KW; ++kw) {
        const int ih = ih0 + kh, iw = iw0 + kw;
        const bool v = (unsigned)ih < (unsigned)a.h && (unsigned)iw < (unsigned)a.w;
        ok[kh * KW + kw] = v;
        const int ihc = min(max(ih, 0), a.h - 1), iwc = min(max(iw, 0), a.w - 1);
        const float* xp = Xf + (size_t)nn * CIN * plane + (size_t)ihc * a.w + iwc;
#pragma unroll
        for (int ic = 0; ic < CIN; ++ic) xv[kh * KW + kw][ic] = h2f(f2h(xp[(size_t)ic * plane]));
      }
  } else {
#pragma unroll
    for (int kh = 0; kh < KH; ++kh)
#pragma unroll
      for (int kw = 0; kw < KW; ++kw) {
        const int ih = ih0 + kh, iw = iw0 + kw;
        const bool v = (unsigned)ih < (unsigned)a.h && (unsigned)iw < (unsigned)a.w;
        ok[kh * KW + kw] = v;
        const int ihc = min(max(ih, 0), a.h - 1), iwc = min(max(iw, 0), a.w - 1);
        const uint8_t* xp = X + (((size_t)(nn * a.h + ihc) * a.w + iwc) * a.x_pix_stride + a.x_c_off) * ES;
#pragma unroll
        for (int ic = 0; ic < CIN; ++ic) xv[kh * KW + kw][ic] = load1<IN_KIND>(a, xp + ic * ES);
      }
  }
  const wrow_t wbase = (wrow_t)(a.wf + oc0);
  float acc[OC];
#pragma unroll
  for (int j = 0; j < OC; ++j) acc[j] = 0.0f;
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    if (!ok[t]) continue;
#pragma unroll
    for (int ic = 0; ic < CIN; ++ic) {
      const wrow_t wr = wbase + (size_t)(t * CIN + ic) * a.cout;
#pragma unroll
      for (int j = 0; j < OC; ++j) acc[j] = fmaf(xv[t][ic], wr[j], acc[j]);
    }
  }
  const size_t yo = (size_t)p * a.y_pix_stride + a.y_c_off + oc0;
  if (a.out_kind == 0)
    dx::store_outputs_t<0, OC>(a, acc, oc0, (uint8_t*)a.y + yo * 4);
  else if (a.out_kind == 1)
    dx::store_outputs_t<1, OC, FE>(a, acc, oc0, (uint8_t*)a.y + yo * 2);
  else
    dx::store_outputs_t<2, OC, FE>(a, acc, oc0, (uint8_t*)a.y + yo, s_lut);
}

// Depthwise 3x3 over f16 NHWC.  A thread owns 4 channels of a block of
// ROWS x SEG outputs; it loads the block's input window (NR rows of NC
// columns, 8 bytes each) up front with buffer loads (a load outside the
// tensor returns zeros; out-of-image rows and columns are sent out of range),
// so every input is loaded (ROWS + 2) (SEG + 2) / (ROWS SEG) times at stride
// 1 instead of 9.
// Each output is the reference's sum: taps in (kh, kw) order, fmaf in f32.
// The inputs enter the fma as f16 operands (v_fma_mix widens them exactly),
// which is the reference's widening unless the value is an f16 subnormal
// (the reference halves those): a wave in which any thread's window holds
// one takes the decoding path for all its outputs.  WPLAIN: no weight is
// subnormal (the planner checks), so the weights enter the fma as f16 too.
// Out-of-image taps contribute an exact +0, which leaves the sum as the
// reference's skip does (the running sum starts at +0 and so is never -0;
// weights are finite).
// Bias: the reference adds in f32 and rounds to f16; for f16 operands that
// is the correctly rounded f16 sum (f32 holds 2 * 11 + 2 bits), so two
// channels are added by one packed f16 add, unless the rounded sum or the
// bias is an f16 subnormal (decoded at half value by the reference): then
// the output takes the scalar decoding path.  SiLU: silu_f16_pk (fp16
// tolerance).  The buffer offsets are 32-bit: x spans at most 2^30 bytes,
// so an offset plus BAD (2^30) is always past the buffer's x_bytes records.
template <int SW, int SEG, int ROWS, bool WPLAIN, bool BIAS, int ACT>
__global__ __launch_bounds__(256) void dwconv3_f16_kernel(const DwArgs a, int segs, int rblocks, int x_bytes) {
  constexpr int CPT = 4;
  constexpr int NC = SW * (SEG - 1) + 3;
  constexpr int NR = SW * (ROWS - 1) + 3;
  constexpr int BAD = 0x40000000;  // added to an offset below 2^30: out of range
  typedef unsigned short us2 __attribute__((ext_vector_type(2)));
  const int groups = a.c / CPT;
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= a.n * rblocks * segs * groups) return;
  const int g = t % groups;
  int rest = t / groups;
  const int sg = rest % segs;
  rest /= segs;
  const int rb = rest % rblocks;
  const int nn = rest / rblocks;
  const int c0 = g * CPT;
  const int ow0 = sg * SEG;
  const int oh0 = rb * ROWS;

  // weights and bias first: the first output needs them with its columns
  uint2 wr[9];
#pragma unroll
  for (int k = 0; k < 9; ++k) wr[k] = *reinterpret_cast<const uint2*>((const uint16_t*)a.wt + (size_t)k * a.c + c0);
  uint2 br = make_uint2(0, 0);
  if constexpr (BIAS) br = *reinterpret_cast<const uint2*>((const uint16_t*)a.bias + c0);

  const __amdgpu_buffer_rsrc_t xrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, x_bytes, 0x00020000);
  const int ps2 = a.x_pix_stride * 2;
  int rowo[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int ih = oh0 * a.sh - a.pt + r;
    rowo[r] = (unsigned)ih < (unsigned)a.h ? ((nn * a.h + ih) * a.w) * ps2 + (a.x_c_off + c0) * 2 : BAD;
  }
  const int iw0 = ow0 * SW - a.pl;
  int colo[NC];
#pragma unroll
  for (int q = 0; q < NC; ++q) colo[q] = (unsigned)(iw0 + q) < (unsigned)a.w ? (iw0 + q) * ps2 : BAD;
  uint2 xc[NC][NR];
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int q = 0; q < NC; ++q) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(xrs, rowo[r] + colo[q], 0, 0);
      xc[q][r] = make_uint2(v[0], v[1]);
    }

  // any f16 subnormal in the window: (2|h| - 2) mod 2^16 < 0x7fe, both
  // halves at once (one packed multiply-add, one packed min per register)
  uint32_t mn = 0xffffffffu;
  {
    const uint32_t two = 0x00020002u, m2 = 0xfffefffeu;
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int q = 0; q < NC; ++q) {
        uint32_t t0, t1;
        asm("v_pk_mad_u16 %0, %1, %2, %3" : "=v"(t0) : "v"(xc[q][r].x), "v"(two), "s"(m2));
        asm("v_pk_mad_u16 %0, %1, %2, %3" : "=v"(t1) : "v"(xc[q][r].y), "v"(two), "s"(m2));
        mn = __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(us2, mn),
                                                                    __builtin_bit_cast(us2, t0)));
        mn = __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(us2, mn),
                                                                    __builtin_bit_cast(us2, t1)));
      }
  }
  const bool sub_any = __any((mn & 0xffffu) < 0x7feu || (mn >> 16) < 0x7feu);

  float wv[9][CPT];
  if constexpr (!WPLAIN) {
#pragma unroll
    for (int k = 0; k < 9; ++k) {
      wv[k][0] = h2f(wr[k].x & 0xffff);
      wv[k][1] = h2f(wr[k].x >> 16);
      wv[k][2] = h2f(wr[k].y & 0xffff);
      wv[k][3] = h2f(wr[k].y >> 16);
    }
  }
  const uint16_t bh[CPT] = {(uint16_t)(br.x & 0xffff), (uint16_t)(br.x >> 16), (uint16_t)(br.y & 0xffff),
                            (uint16_t)(br.y >> 16)};
  bool bias_sub = false;
  if constexpr (BIAS) {
#pragma unroll
    for (int c = 0; c < CPT; ++c) bias_sub |= (uint16_t)((bh[c] & 0x7fff) - 1) < 0x3ff;
  }

#define DW_HALVES(r_) {(uint16_t)((r_).x & 0xffff), (uint16_t)((r_).x >> 16), (uint16_t)((r_).y & 0xffff), (uint16_t)((r_).y >> 16)}
#pragma unroll
  for (int i = 0; i < ROWS; ++i) {
    if (oh0 + i >= a.ho) break;
    uint16_t* const yrow =
        (uint16_t*)a.y + ((size_t)(nn * a.ho + oh0 + i) * a.wo) * a.y_pix_stride + a.y_c_off + c0;
#pragma unroll
    for (int j = 0; j < SEG; ++j) {
      if (ow0 + j >= a.wo) break;
      float acc[CPT] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (sub_any) {
#pragma unroll
        for (int kh = 0; kh < 3; ++kh)
#pragma unroll
          for (int kw = 0; kw < 3; ++kw) {
            const uint16_t hv[CPT] = DW_HALVES(xc[SW * j + kw][SW * i + kh]);
            const uint16_t hw[CPT] = DW_HALVES(wr[kh * 3 + kw]);
#pragma unroll
            for (int c = 0; c < CPT; ++c) {
              const float wk = WPLAIN ? h2f_ieee(hw[c]) : wv[kh * 3 + kw][c];
              acc[c] = fmaf(h2f(hv[c]), wk, acc[c]);
            }
          }
      } else {
#pragma unroll
        for (int kh = 0; kh < 3; ++kh)
#pragma unroll
          for (int kw = 0; kw < 3; ++kw) {
            const uint2 xv = xc[SW * j + kw][SW * i + kh];
            const int k = kh * 3 + kw;
            if constexpr (WPLAIN) {
              if (k == 0) {
                acc[0] = fma_mix_h0<0>(xv.x, wr[k].x);
                acc[1] = fma_mix_h0<1>(xv.x, wr[k].x);
                acc[2] = fma_mix_h0<0>(xv.y, wr[k].y);
                acc[3] = fma_mix_h0<1>(xv.y, wr[k].y);
              } else {
                acc[0] = fma_mix_h<0>(xv.x, wr[k].x, acc[0]);
                acc[1] = fma_mix_h<1>(xv.x, wr[k].x, acc[1]);
                acc[2] = fma_mix_h<0>(xv.y, wr[k].y, acc[2]);
                acc[3] = fma_mix_h<1>(xv.y, wr[k].y, acc[3]);
              }
            } else {
              if (k == 0) {
                acc[0] = fma_mix_hf0<0>(xv.x, wv[k][0]);
                acc[1] = fma_mix_hf0<1>(xv.x, wv[k][1]);
                acc[2] = fma_mix_hf0<0>(xv.y, wv[k][2]);
                acc[3] = fma_mix_hf0<1>(xv.y, wv[k][3]);
              } else {
                acc[0] = fma_mix_hf<0>(xv.x, wv[k][0], acc[0]);
                acc[1] = fma_mix_hf<1>(xv.x, wv[k][1], acc[1]);
                acc[2] = fma_mix_hf<0>(xv.y, wv[k][2], acc[2]);
                acc[3] = fma_mix_hf<1>(xv.y, wv[k][3], acc[3]);
              }
            }
          }
      }
      // the conv result rounded to f16 (the reference's store)
      h16x2 p01 = pk_f2h(acc[0], acc[1]), p23 = pk_f2h(acc[2], acc[3]);
      if constexpr (BIAS) {
        const float amin = fminf(fminf(fabsf(acc[0]), fabsf(acc[1])), fminf(fabsf(acc[2]), fabsf(acc[3])));
        if (__any(bias_sub || amin < 6.103515625e-05f)) {
          uint16_t hb[CPT] = {pk_lo(p01), pk_hi(p01), pk_lo(p23), pk_hi(p23)};
#pragma unroll
          for (int c = 0; c < CPT; ++c) hb[c] = f16_add_bits(hb[c], bh[c]);
          p01 = pk_make(hb[0], hb[1]);
          p23 = pk_make(hb[2], hb[3]);
        } else {
          p01 = p01 + __builtin_bit_cast(h16x2, br.x);
          p23 = p23 + __builtin_bit_cast(h16x2, br.y);
        }
      }
      if constexpr (ACT == ACT_SILU) {
        p01 = silu_f16_pk(p01);
        p23 = silu_f16_pk(p23);
      } else if constexpr (ACT == ACT_RELU) {
        uint16_t hb[CPT] = {pk_lo(p01), pk_hi(p01), pk_lo(p23), pk_hi(p23)};
#pragma unroll
        for (int c = 0; c < CPT; ++c) hb[c] = f16_act_bits(hb[c], ACT_RELU);
        p01 = pk_make(hb[0], hb[1]);
        p23 = pk_make(hb[2], hb[3]);
      }
      *reinterpret_cast<uint2*>(yrow + (size_t)(ow0 + j) * a.y_pix_stride) =
          make_uint2(__builtin_bit_cast(uint32_t, p01), __builtin_bit_cast(uint32_t, p23));
    }
  }
#undef DW_HALVES
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

void launch_direct_conv(hipStream_t st, const DirectArgs& a_in) {
  if (launch_conv1x1_exact(st, a_in)) return;
  DirectArgs a = a_in;
  // the 3x3, 3-channel stem
  if (a.in_kind == 3 && !(a.kh == 3 && a.kw == 3 && a.cin == 3 && a.cout % 16 == 0))
    fail(-2, "direct conv: NCHW f32 input only for the 3x3 three-channel stem");
  if (a.kh == 3 && a.kw == 3 && a.cin == 3 && a.cout % 16 == 0 && (a.in_kind <= 1 || a.in_kind == 3)) {
    const int oes = a.out_kind == 0 ? 4 : (a.out_kind == 1 ? 2 : 1);
    auto aligned = [&](int v) {
      return (16 * oes) % v == 0 && (a.y_pix_stride * oes) % v == 0 && (a.y_c_off * oes) % v == 0 &&
             ((uintptr_t)a.y % v) == 0;
    };
    a.vec_out = aligned(16) ? 16 : (aligned(4) ? 4 : 1);
    const dim3 grid((a.m + 255) / 256, a.cout / 16);
    // row loads: dense f16 rows of even width, 4-byte aligned base, even
    // column stride (every output's first input pixel index then has the
    // parity of the left pad, so the loads start on 4-byte boundaries)
    const long long xb = (long long)a.n * a.h * a.w * 6;
    const bool rows = a.in_kind == 1 && a.x_pix_stride == 3 && a.x_c_off == 0 && a.sw % 2 == 0 &&
                      a.w % 2 == 0 && (uintptr_t)a.x % 4 == 0 && xb + 16 < (1ll << 31);
    a.x_bytes = rows ? (int)xb : 0;
    const int par = a.pl & 1;
#define DW_SMALL(FE_, PAR_) \
  hipLaunchKernelGGL((conv_small_kernel<1, 16, 3, 3, 3, FE_, PAR_>), grid, dim3(256), 0, st, a)
    if (a.in_kind == 0)
      hipLaunchKernelGGL((conv_small_kernel<0, 16, 3, 3, 3, false, -1>), grid, dim3(256), 0, st, a);
    else if (a.in_kind == 3 && a.fast_epi)
      hipLaunchKernelGGL((conv_small_kernel<3, 16, 3, 3, 3, true, -1>), grid, dim3(256), 0, st, a);
    else if (a.in_kind == 3)
      hipLaunchKernelGGL((conv_small_kernel<3, 16, 3, 3, 3, false, -1>), grid, dim3(256), 0, st, a);
    else if (rows && par == 1 && a.fast_epi)
      DW_SMALL(true, 1);
    else if (rows && par == 1)
      DW_SMALL(false, 1);
    else if (rows && a.fast_epi)
      DW_SMALL(true, 0);
    else if (rows)
      DW_SMALL(false, 0);
    else if (a.fast_epi)
      DW_SMALL(true, -1);
    else
      DW_SMALL(false, -1);
#undef DW_SMALL
    DW_HIP(hipGetLastError());
    return;
  }
  const int es = a.in_kind == 0 ? 4 : (a.in_kind == 1 ? 2 : 1);
  const int vn = 16 / es;
  const bool vin = a.cin % vn == 0 && (a.x_pix_stride * es) % 16 == 0 && (a.x_c_off * es) % 16 == 0 &&
                   ((uintptr_t)a.x & 15) == 0;
  // Output channels per thread: the widest chunk of c_out that still gives
  // about four wavefronts per CU (wide chunks pay the input decode once for
  // more FMAs; narrow ones spread small layers over the GPU).
  const long waves = ((long)a.m + 63) / 64;
  static const int wide[] = {80, 64, 40, 32, 16, 8, 4, 1};
  static const int narrow[] = {16, 8, 4, 1};
  const int* cand = vin ? wide : narrow;
  const int ncand = vin ? 8 : 4;
  // (chunks below 4 channels only when c_out is not a multiple of 4)
  const int min_oc = a.cout % 4 == 0 ? 4 : 1;
  int oc = 0;
  for (int i = 0; i < ncand && !oc; ++i)
    if (cand[i] >= min_oc && a.cout % cand[i] == 0 && waves * (a.cout / cand[i]) >= 1024) oc = cand[i];
  if (!oc) oc = min_oc;  // too few pixels for any chunk: the narrowest
  if (a.cout % oc != 0) fail(-2, "direct conv: no channel chunk for this c_out");
  const int oes = a.out_kind == 0 ? 4 : (a.out_kind == 1 ? 2 : 1);
  auto aligned = [&](int v) {
    return (oc * oes) % v == 0 && (a.y_pix_stride * oes) % v == 0 && (a.y_c_off * oes) % v == 0 &&
           ((uintptr_t)a.y % v) == 0;
  };
  a.vec_out = aligned(16) ? 16 : (aligned(4) ? 4 : 1);
  dim3 grid((a.m + 255) / 256, a.cout / oc);
#define DW_DC(KIND, O, V)                                                                     \
  if (a.in_kind == KIND && oc == O && vin == V) {                                             \
    hipLaunchKernelGGL((direct_conv_kernel<KIND, O, V>), grid, dim3(256), 0, st, a);          \
    DW_HIP(hipGetLastError());                                                                \
    return;                                                                                   \
  }
#define DW_DC_ALL(O, V) DW_DC(0, O, V) DW_DC(1, O, V) DW_DC(2, O, V)
  DW_DC_ALL(80, true)
  DW_DC_ALL(64, true)
  DW_DC_ALL(40, true)
  DW_DC_ALL(32, true)
  DW_DC_ALL(16, true)
  DW_DC_ALL(8, true)
  DW_DC_ALL(4, true)
  DW_DC_ALL(1, true)
  DW_DC_ALL(16, false)
  DW_DC_ALL(8, false)
  DW_DC_ALL(4, false)
  DW_DC_ALL(1, false)
#undef DW_DC_ALL
#undef DW_DC
  fail(-2, "direct conv: no kernel for this channel count");
}

void launch_dwconv(hipStream_t st, const DwArgs& a, int dtype) {
  // f16 3x3, stride 1 or 2: the sliding-window kernel (8-byte channel
  // groups; the same sums, so the same results as the generic kernel)
  const bool al8 = (uintptr_t)a.x % 8 == 0 && (uintptr_t)a.y % 8 == 0 && (uintptr_t)a.wt % 8 == 0 &&
                   (uintptr_t)a.bias % 8 == 0 && (a.x_pix_stride * 2) % 8 == 0 && (a.x_c_off * 2) % 8 == 0 &&
                   (a.y_pix_stride * 2) % 8 == 0 && (a.y_c_off * 2) % 8 == 0;
  const long long x_bytes = ((long long)a.n * a.h * a.w - 1) * a.x_pix_stride * 2 + (a.x_c_off + a.c) * 2ll;
  if (dtype == F16 && a.kh == 3 && a.kw == 3 && (a.sw == 1 || a.sw == 2) && a.sh == a.sw && a.c % 4 == 0 && al8 &&
      x_bytes <= (1ll << 30)) {
    // one row of 4 outputs per thread (3 x 6 input columns at stride 1, 3 x 9
    // at stride 2): measured faster on 32 x 40 x 40 x 384 than 8 outputs, 2
    // rows of 4 or 8, or an XCD-aware block order, whose larger windows
    // cost occupancy and overlap between the loads and the arithmetic
    constexpr int rows = 1;
    const int seg = 4;
    const int segs = (a.wo + seg - 1) / seg;
    const int rblocks = (a.ho + rows - 1) / rows;
    const long long threads = (long long)a.n * rblocks * segs * (a.c / 4);
    if (threads < (1ll << 31)) {
      const dim3 g((unsigned)((threads + 255) / 256));
      const bool bias = a.bias != nullptr;
#define DW_DW3(SW_, SEG_, WP_, B_, ACT_)                                                                    \
  if (a.sw == SW_ && (a.w_plain != 0) == WP_ && bias == B_ && a.act == ACT_)                                 \
    hipLaunchKernelGGL((dwconv3_f16_kernel<SW_, SEG_, rows, WP_, B_, ACT_>), g, dim3(256), 0, st, a, segs, \
                       rblocks, (int)x_bytes);                                                             \
  else
#define DW_DW3_ACTS(SW_, SEG_, WP_, B_) \
  DW_DW3(SW_, SEG_, WP_, B_, ACT_NONE) DW_DW3(SW_, SEG_, WP_, B_, ACT_RELU) DW_DW3(SW_, SEG_, WP_, B_, ACT_SILU)
      DW_DW3_ACTS(1, 4, true, true)
      DW_DW3_ACTS(1, 4, true, false)
      DW_DW3_ACTS(1, 4, false, true)
      DW_DW3_ACTS(1, 4, false, false)
      DW_DW3_ACTS(2, 4, true, true)
      DW_DW3_ACTS(2, 4, true, false)
      DW_DW3_ACTS(2, 4, false, true)
      DW_DW3_ACTS(2, 4, false, false)
      fail(-2, "depthwise: no kernel for this activation");
#undef DW_DW3_ACTS
#undef DW_DW3
      DW_HIP(hipGetLastError());
      return;
    }
  }
  if (a.c % 8 != 0) fail(-2, "depthwise: c must be a multiple of 8 for this shape");
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
