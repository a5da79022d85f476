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
  constexpr int ES = IN_KIND == 0 ? 4 : (IN_KIND == 1 ? 2 : 1);
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

// Depthwise 3x3 over f16 NHWC, a row segment per thread.  A thread owns 4
// channels of SEG consecutive outputs of one row; it loads the segment's
// SW * (SEG - 1) + 3 input columns of its 3 input rows up front (raw f16,
// 8 bytes each), so every input is loaded 3 times (once per output row that
// reads it) instead of 9, and all loads are in flight together.  Each output
// is the reference's sum: taps in (kh, kw) order, fmaf in f32.  The inputs
// enter the fma as f16 operands (v_fma_mix widens them exactly), which is
// the reference's widening unless the value is an f16 subnormal (the
// reference halves those): an output whose window holds one, anywhere in
// the wave, takes the decoding path.  WPLAIN: no weight is subnormal (the
// planner checks), so the weights enter the fma as f16 too.  Out-of-image
// taps contribute an exact +0, which leaves the sum as the reference's skip
// does (the running sum starts at +0 and so is never -0; weights are
// finite).  SiLU uses silu_f16_fast (fp16 tolerance).
template <int SW, int SEG, bool WPLAIN, bool BIAS, int ACT>
__global__ __launch_bounds__(256) void dwconv3_f16_kernel(const DwArgs a, int segs) {
  constexpr int CPT = 4;
  constexpr int NC = SW * (SEG - 1) + 3;
  typedef unsigned short us2 __attribute__((ext_vector_type(2)));
  const int groups = a.c / CPT;
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= a.n * a.ho * segs * groups) return;
  const int g = t % groups;
  int rest = t / groups;
  const int sg = rest % segs;
  rest /= segs;
  const int oh = rest % a.ho;
  const int nn = rest / a.ho;
  const int c0 = g * CPT;
  const int ow0 = sg * SEG;

  // weights and bias first: the first output needs them with its columns
  uint2 wr[9];
#pragma unroll
  for (int k = 0; k < 9; ++k) wr[k] = *reinterpret_cast<const uint2*>((const uint16_t*)a.wt + (size_t)k * a.c + c0);
  float bf[CPT] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (BIAS) {
    const uint2 r = *reinterpret_cast<const uint2*>((const uint16_t*)a.bias + c0);
    bf[0] = h2f(r.x & 0xffff); bf[1] = h2f(r.x >> 16); bf[2] = h2f(r.y & 0xffff); bf[3] = h2f(r.y >> 16);
  }
  const uint16_t* rowp[3];
  bool rv[3];
#pragma unroll
  for (int kh = 0; kh < 3; ++kh) {
    const int ih = oh * a.sh - a.pt + kh;
    rv[kh] = ih >= 0 && ih < a.h;
    rowp[kh] = (const uint16_t*)a.x + ((size_t)(nn * a.h + (rv[kh] ? ih : 0)) * a.w) * a.x_pix_stride + a.x_c_off + c0;
  }
  // input column q of the segment is iw0 + q
  const int iw0 = ow0 * SW - a.pl;
  uint2 xc[NC][3];
#pragma unroll
  for (int q = 0; q < NC; ++q) {
    const int iw = iw0 + q;
    const bool cv = iw >= 0 && iw < a.w;
#pragma unroll
    for (int kh = 0; kh < 3; ++kh) {
      xc[q][kh] = make_uint2(0, 0);
      if (cv && rv[kh]) xc[q][kh] = *reinterpret_cast<const uint2*>(rowp[kh] + (size_t)iw * a.x_pix_stride);
    }
  }
  float wv[3][3][CPT];
  if constexpr (!WPLAIN) {
#pragma unroll
    for (int k = 0; k < 9; ++k) {
      wv[k / 3][k % 3][0] = h2f(wr[k].x & 0xffff);
      wv[k / 3][k % 3][1] = h2f(wr[k].x >> 16);
      wv[k / 3][k % 3][2] = h2f(wr[k].y & 0xffff);
      wv[k / 3][k % 3][3] = h2f(wr[k].y >> 16);
    }
  }
  // columns holding an f16 subnormal: |h| - 1 (mod 2^16) < 0x3ff
  bool subc[NC];
#pragma unroll
  for (int q = 0; q < NC; ++q) {
    us2 mn = {0xffff, 0xffff};
    const us2 one = {1, 1};
#pragma unroll
    for (int kh = 0; kh < 3; ++kh) {
      mn = __builtin_elementwise_min(mn, __builtin_bit_cast(us2, xc[q][kh].x & 0x7fff7fffu) - one);
      mn = __builtin_elementwise_min(mn, __builtin_bit_cast(us2, xc[q][kh].y & 0x7fff7fffu) - one);
    }
    subc[q] = mn.x < 0x3ff || mn.y < 0x3ff;
  }

  uint16_t* const yrow = (uint16_t*)a.y + ((size_t)(nn * a.ho + oh) * a.wo) * a.y_pix_stride + a.y_c_off + c0;
#define DW_HALVES(r_) {(uint16_t)((r_).x & 0xffff), (uint16_t)((r_).x >> 16), (uint16_t)((r_).y & 0xffff), (uint16_t)((r_).y >> 16)}
#pragma unroll
  for (int j = 0; j < SEG; ++j) {
    if (ow0 + j < a.wo) {
      float acc[CPT] = {0.0f, 0.0f, 0.0f, 0.0f};
      const bool sub = subc[SW * j] || subc[SW * j + 1] || subc[SW * j + 2];
      if (__any(sub)) {
#pragma unroll
        for (int kh = 0; kh < 3; ++kh)
#pragma unroll
          for (int kw = 0; kw < 3; ++kw) {
            const uint16_t hv[CPT] = DW_HALVES(xc[SW * j + kw][kh]);
            const uint16_t hw[CPT] = DW_HALVES(wr[kh * 3 + kw]);
#pragma unroll
            for (int c = 0; c < CPT; ++c) {
              const float wk = WPLAIN ? h2f_ieee(hw[c]) : wv[kh][kw][c];
              acc[c] = fmaf(h2f(hv[c]), wk, acc[c]);
            }
          }
      } else {
#pragma unroll
        for (int kh = 0; kh < 3; ++kh)
#pragma unroll
          for (int kw = 0; kw < 3; ++kw) {
            const uint16_t hv[CPT] = DW_HALVES(xc[SW * j + kw][kh]);
            const uint16_t hw[CPT] = DW_HALVES(wr[kh * 3 + kw]);
#pragma unroll
            for (int c = 0; c < CPT; ++c) {
              const float wk = WPLAIN ? h2f_ieee(hw[c]) : wv[kh][kw][c];
              acc[c] = fmaf(h2f_ieee(hv[c]), wk, acc[c]);
            }
          }
      }
      uint16_t ob[CPT];
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        uint16_t hb = f2h(acc[c]);
        if constexpr (BIAS) hb = f2h(h2f(hb) + bf[c]);
        if constexpr (ACT == ACT_SILU)
          hb = silu_f16_fast(hb);
        else if constexpr (ACT == ACT_RELU)
          hb = f16_act_bits(hb, ACT_RELU);
        ob[c] = hb;
      }
      *reinterpret_cast<uint2*>(yrow + (size_t)(ow0 + j) * a.y_pix_stride) =
          make_uint2((uint32_t)ob[0] | ((uint32_t)ob[1] << 16), (uint32_t)ob[2] | ((uint32_t)ob[3] << 16));
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
  if (a.kh == 3 && a.kw == 3 && a.cin == 3 && a.cout % 16 == 0 && a.in_kind <= 1) {
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
  if (dtype == F16 && a.kh == 3 && a.kw == 3 && (a.sw == 1 || a.sw == 2) && a.c % 4 == 0 && al8) {
    // 8 outputs per thread at stride 1, 4 at stride 2 (10 and 9 input columns)
    const int seg = a.sw == 1 ? 8 : 4;
    const int segs = (a.wo + seg - 1) / seg;
    const long long threads = (long long)a.n * a.ho * segs * (a.c / 4);
    if (threads < (1ll << 31)) {
      const dim3 g((unsigned)((threads + 255) / 256));
      const bool bias = a.bias != nullptr;
#define DW_DW3(SW_, SEG_, WP_, B_, ACT_)                                                          \
  if (a.sw == SW_ && (a.w_plain != 0) == WP_ && bias == B_ && a.act == ACT_)                       \
    hipLaunchKernelGGL((dwconv3_f16_kernel<SW_, SEG_, WP_, B_, ACT_>), g, dim3(256), 0, st, a, segs); \
  else
#define DW_DW3_ACTS(SW_, SEG_, WP_, B_) \
  DW_DW3(SW_, SEG_, WP_, B_, ACT_NONE) DW_DW3(SW_, SEG_, WP_, B_, ACT_RELU) DW_DW3(SW_, SEG_, WP_, B_, ACT_SILU)
      DW_DW3_ACTS(1, 8, true, true)
      DW_DW3_ACTS(1, 8, true, false)
      DW_DW3_ACTS(1, 8, false, true)
      DW_DW3_ACTS(1, 8, false, false)
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
