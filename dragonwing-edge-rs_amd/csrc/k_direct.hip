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

#include <stdlib.h>

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

// f32 convolutions whose input window fits LDS (3x3 at stride 1 with c_in
// 32 or 64, as the 1 x 56 x 56 x 64 -> 64 fp32 layer).  direct_conv_kernel
// reads each input vector straight from
// global memory, 16 bytes per lane at the pixel stride, so every wave
// instruction touches 64 distinct lines and the per-CU load path, not the
// FMAs, sets its pace.  Here a workgroup owns a TH x TW tile of output
// pixels (one per thread) x 4 output channels:
//  * it copies the tile's input window, all c_in channels of every pixel,
//    into LDS with 16-byte buffer loads (consecutive lanes: consecutive
//    channel quads of one pixel; zeros outside the image), and its 4
//    channels' weights (kh * kw * c_in x 4 floats, packed by the host as
//    [c_out / 4][kh * kw * c_in][4]), every load in flight before the
//    first LDS store;
//  * the LDS pixel stride is c_in + 4 floats, so the 8 lanes of one
//    ds_read_b128 cycle (8 neighbouring pixels) hit 8 distinct bank groups;
//  * the weights reach the FMAs through DPP: one VGPR holds the 16 weights
//    of 4 input x 4 output channels in lanes 0..15 of every row of 16
//    lanes, and v_fmac_f32_dpp row_newbcast:n multiplies by lane n's value,
//    so a weight costs neither an SGPR load (whose latency cannot be
//    overlapped: scalar loads complete out of order, so every wait on one
//    is a wait for all) nor a broadcast LDS read per FMA.  All LDS reads
//    complete in order, so the next block's reads are in flight while this
//    block's FMAs run;
//  * every lane runs every tap with all lanes enabled (DPP reads its
//    source lane whatever that lane's own tap is), and a lane whose tap
//    lies outside the image restores its accumulators after that tap, so
//    its chain is exactly the reference's with the tap skipped.
// The FMA chain of each output is the reference's: kh, kw, ic in order,
// one fused multiply-add per (tap, ic), fma(w, x, acc) = fma(x, w, acc).
constexpr int kTileLdsFloats = 22 * 1024;  // 88 KB: the input window of one workgroup
constexpr int kTileWRows = 1536;           // kh * kw * c_in (24 KB of weights)

// One block of 16 input channels for 4 outputs:
//   acc[j] = fma(w[ic e][oc j], x[e], acc[j]) for e = 0..15 in order, j = 0..3,
// where lane 4 (e % 4) + j of each row of VGPR w[e / 4] holds w[ic e][oc j].
// The s_nop covers the two wait states a DPP source needs after a VALU
// write.
#define DW_FMAC_DPP(N, J, W, XI) \
  "v_fmac_f32_dpp %" #J ", %" #W ", %" #XI " row_newbcast:" #N " row_mask:0xf bank_mask:0xf\n"
#define DW_FMAC_QUAD(W, X0, X1, X2, X3)                                                        \
  DW_FMAC_DPP(0, 0, W, X0) DW_FMAC_DPP(1, 1, W, X0) DW_FMAC_DPP(2, 2, W, X0) DW_FMAC_DPP(3, 3, W, X0) \
  DW_FMAC_DPP(4, 0, W, X1) DW_FMAC_DPP(5, 1, W, X1) DW_FMAC_DPP(6, 2, W, X1) DW_FMAC_DPP(7, 3, W, X1) \
  DW_FMAC_DPP(8, 0, W, X2) DW_FMAC_DPP(9, 1, W, X2) DW_FMAC_DPP(10, 2, W, X2) DW_FMAC_DPP(11, 3, W, X2) \
  DW_FMAC_DPP(12, 0, W, X3) DW_FMAC_DPP(13, 1, W, X3) DW_FMAC_DPP(14, 2, W, X3) DW_FMAC_DPP(15, 3, W, X3)
__device__ __forceinline__ void fma16x4_dpp(float (&acc)[4], const float4& w, const float4 (&x)[4]) {
  asm("s_nop 1\n"
      DW_FMAC_QUAD(4, 8, 9, 10, 11) DW_FMAC_QUAD(5, 12, 13, 14, 15)
      DW_FMAC_QUAD(6, 16, 17, 18, 19) DW_FMAC_QUAD(7, 20, 21, 22, 23)
      : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3])
      : "v"(w.x), "v"(w.y), "v"(w.z), "v"(w.w),
        "v"(x[0].x), "v"(x[0].y), "v"(x[0].z), "v"(x[0].w), "v"(x[1].x), "v"(x[1].y), "v"(x[1].z), "v"(x[1].w),
        "v"(x[2].x), "v"(x[2].y), "v"(x[2].z), "v"(x[2].w), "v"(x[3].x), "v"(x[3].y), "v"(x[3].z), "v"(x[3].w));
}
#undef DW_FMAC_QUAD
#undef DW_FMAC_DPP

template <int TH, int TW, int NBT>
__global__ __launch_bounds__(TH * TW) void conv_tile_f32_kernel(const DirectArgs a, int tiles_w, int tiles_hw,
                                                                int iwin_w, int pstr) {
  constexpr int C = 4;
  __shared__ __attribute__((aligned(16))) float s_x[kTileLdsFloats];
  __shared__ __attribute__((aligned(16))) float s_w[kTileWRows * 4];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int tile = blockIdx.x;
  const int nn = tile / tiles_hw;
  const int tr = tile - nn * tiles_hw;
  const int tyi = tr / tiles_w;
  const int ty0 = tyi * TH, tx0 = (tr - tyi * tiles_w) * TW;
  const int oc0 = blockIdx.y * C;
  const int cin = a.cin;
  const int ih0 = ty0 * a.sh - a.pt, iw0 = tx0 * a.sw - a.pl;
  const int iwin_h = (TH - 1) * a.sh + a.kh;
  const int quads = cin >> 2;
  const int rows = a.kh * a.kw * cin;
  // All global loads of the workgroup are issued before any LDS store: the
  // weights (up to 6 float4 per thread) and the input window (up to 24
  // float4 per thread: c_in 64 at 16 x 16 pixels and a 3 x 3 window), so
  // their latencies overlap.
  //
  // weights: block b of 16 input channels (64 floats of [row][4]) stored so
  // that float v of lane n's 16-byte read is element 16 v + n of the block
  constexpr int kWLoads = kTileWRows / (TH * TW);
  const float4* __restrict__ wq4 = reinterpret_cast<const float4*>(a.wq + (size_t)blockIdx.y * rows * 4);
  float4 wv4[kWLoads];
#pragma unroll
  for (int k = 0; k < kWLoads; ++k) {
    const int f4 = tid + k * TH * TW;
    if (f4 < rows) wv4[k] = wq4[f4];
  }
  // input window: thread tid loads channel quad q = tid % quads of window
  // columns c and c + cpp (c = tid / quads, cpp = 256 / quads) in every
  // window row: at most 2 x 24 loads, all in flight together.  Buffer
  // loads: a pixel outside the image (or past the window) reads with an
  // offset past the buffer, which returns zeros with no memory access.
  constexpr int kXRows = 24;
  const int cpp = (TH * TW) / quads;
  const int q = tid % quads, c = tid / quads;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, a.x_bytes, 0x00020000);
  const int ps4 = a.x_pix_stride * 4, rstep = a.w * ps4;
  // rows rlo..rhi-1 of the window lie in the image; an offset with bit 31
  // set is past the buffer (x_bytes < 2^31)
  const int rlo = max(0, -ih0), rhi = min(iwin_h, a.h - ih0);
  float4 xv4[2][kXRows];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int cc = c + h * cpp, iw = iw0 + cc;
    const bool col_ok = cc < iwin_w && iw >= 0 && iw < a.w;
    int goff = col_ok ? (((nn * a.h + ih0) * a.w + iw) * a.x_pix_stride + a.x_c_off + 4 * q) * 4 : (int)0x80000000;
#pragma unroll
    for (int r = 0; r < kXRows; ++r) {
      const int roff = (r >= rlo && r < rhi) ? 0 : (int)0x80000000;
      xv4[h][r] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, goff | roff, 0, 0));
      goff += rstep;
    }
  }
#pragma unroll
  for (int k = 0; k < kWLoads; ++k) {
    const int f4 = tid + k * TH * TW;
    if (f4 < rows) {
      // float4 f4 holds elements 4 f4 .. 4 f4 + 3 of the [row][4] layout
      const float e[4] = {wv4[k].x, wv4[k].y, wv4[k].z, wv4[k].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int f = 4 * f4 + i, rr = f & 63;
        s_w[(f & ~63) + (rr & 15) * 4 + (rr >> 4)] = e[i];
      }
    }
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int cc = c + h * cpp;
    if (cc < iwin_w) {
#pragma unroll
      for (int r = 0; r < kXRows; ++r)
        if (r < iwin_h) *reinterpret_cast<float4*>(s_x + (r * iwin_w + cc) * pstr + 4 * q) = xv4[h][r];
    }
  }
  __syncthreads();

  const int ty = tid / TW, tx = tid - (tid / TW) * TW;
  const int oh = ty0 + ty, ow = tx0 + tx;
  const bool valid = oh < a.ho && ow < a.wo;
  float acc[C] = {0.0f, 0.0f, 0.0f, 0.0f};
  static_assert(NBT % 2 == 0, "blocks alternate between two register sets within a tap");
  const float* const xpix = s_x + (ty * a.sh * iwin_w + tx * a.sw) * pstr;
  const float* const wl = s_w + 4 * (lane & 15);
  const int taps = a.kh * a.kw;
  // block b of the tap whose input offset is xoff, weights of block t
  auto load = [&](int xoff, int t, float4 (&xv)[4], float4& wv) {
    const float* xs = xpix + xoff;
#pragma unroll
    for (int i = 0; i < 4; ++i) xv[i] = *reinterpret_cast<const float4*>(xs + 4 * i);
    wv = *reinterpret_cast<const float4*>(wl + 64 * t);
  };
  // Taps in order (kh, kw); within a tap NBT blocks of 16 input channels,
  // each block's reads issued before the previous block's FMAs (two
  // register sets).  The read after the last block repeats it, so every
  // iteration issues the same reads and the compiler's LDS wait counts stay
  // exact.  A lane whose tap lies outside the image restores the
  // accumulators it had before the tap.
  float4 xa[4], wa, xb[4], wb;
  load(0, 0, xa, wa);
  int kh = 0, kw = 0, xoff = 0;
  for (int tap = 0; tap < taps; ++tap) {
    const bool last_tap = tap + 1 == taps;
    const int nxoff = kw + 1 == a.kw ? xoff + (iwin_w - a.kw + 1) * pstr : xoff + pstr;
    float keep[C];
#pragma unroll
    for (int j = 0; j < C; ++j) keep[j] = acc[j];
#pragma unroll
    for (int b = 0; b < NBT; b += 2) {
      const int t = tap * NBT + b;
      load(xoff + 16 * (b + 1), t + 1, xb, wb);
      __builtin_amdgcn_sched_barrier(0);
      fma16x4_dpp(acc, wa, xa);
      __builtin_amdgcn_sched_barrier(0);
      if (b + 2 < NBT)
        load(xoff + 16 * (b + 2), t + 2, xa, wa);
      else
        load(last_tap ? xoff + 16 * (b + 1) : nxoff, last_tap ? t + 1 : t + 2, xa, wa);
      __builtin_amdgcn_sched_barrier(0);
      fma16x4_dpp(acc, wb, xb);
      __builtin_amdgcn_sched_barrier(0);
    }
    const int ih = oh * a.sh - a.pt + kh, iw = ow * a.sw - a.pl + kw;
    const bool skip = !(ih >= 0 && ih < a.h && iw >= 0 && iw < a.w);
#pragma unroll
    for (int j = 0; j < C; ++j) acc[j] = skip ? keep[j] : acc[j];
    xoff = nxoff;
    if (++kw == a.kw) {
      kw = 0;
      ++kh;
    }
  }
  if (!valid) return;
  const size_t p = ((size_t)nn * a.ho + oh) * a.wo + ow;
  const int OES = a.out_kind == 0 ? 4 : (a.out_kind == 1 ? 2 : 1);
  dx::store_outputs<C>(a, acc, oc0, (uint8_t*)a.y + (p * a.y_pix_stride + a.y_c_off + oc0) * OES);
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

// The INT8 graph's stem (3x3, stride 2, pad 1, three dense f16 channels in,
// u8 out through QuantizeLinear and the activation table): one output pixel x
// 16 channels a thread, as conv_small_kernel, with less work per output:
//  * no per-tap skip: an out-of-image tap is accumulated as +0.  The
//    running sum starts at +0; fma(+0, w, acc) is acc for a finite weight w
//    unless acc is a zero, where only the zero's sign may change, and no u8
//    output depends on a zero's sign (a later nonzero term replaces it; a
//    final +0 or -0 rounds to an f16 zero and quantizes to the zero point's
//    byte).  The rows above the image load as zeros (buffer loads out of
//    range), and the column left of the image is cleared in registers.  The
//    host sets w_finite after checking the weights;
//  * the input values stay packed, two halves a register, and enter each
//    FMA as its f16 operand (v_fma_mix widens exactly, at the issue rate of
//    the SGPR-operand FMA it replaces), unless a lane of the wave holds an
//    f16 subnormal among them (checked on the packed registers): that wave
//    widens every value with the reference decode (half a subnormal's IEEE
//    value) first.
// The FMA chain of every output is the reference's: taps in (kh, kw) order,
// channels in order, one fmaf each (ops.rs:1356-1436).
template <bool FE, bool SUB>
__device__ __forceinline__ void stem_pad_accumulate(const uint32_t (&dw)[3][5], const wrow_t wbase, int cout,
                                                    float (&acc)[16]) {
#pragma unroll
  for (int kh = 0; kh < 3; ++kh)
#pragma unroll
    for (int kw = 0; kw < 3; ++kw)
#pragma unroll
      for (int ic = 0; ic < 3; ++ic) {
        const int hi = 1 + kw * 3 + ic;  // half index in the row's 20 loaded bytes (PAR 1)
        const uint16_t hb = (uint16_t)(dw[kh][hi >> 1] >> (16 * (hi & 1)));
        const float xv = SUB ? h2f(hb) : h2f_ieee(hb);
        const wrow_t wr = wbase + (size_t)((kh * 3 + kw) * 3 + ic) * cout;
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[j] = fmaf(xv, wr[j], acc[j]);
      }
}

template <bool FE>
__global__ __launch_bounds__(256) void stem_pad_u8_kernel(const DirectArgs a) {
  __shared__ uint8_t s_lut[256];
  if (a.lut) s_lut[threadIdx.x] = a.lut[threadIdx.x];
  __syncthreads();
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= a.m) return;
  const int oc0 = blockIdx.y * 16;
  const int hw = a.ho * a.wo;
  const int nn = p / hw;
  const int rem = p - nn * hw;
  const int oh = rem / a.wo;
  const int ow = rem - oh * a.wo;
  const int ih0 = 2 * oh - 1, iw0 = 2 * ow - 1;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, a.x_bytes, 0x00020000);
  // each window row: 9 halves from half index 3 iw0 of the image row, which
  // is odd: five 4-byte loads from the boundary one half below it
  uint32_t dw[3][5];
#pragma unroll
  for (int kh = 0; kh < 3; ++kh) {
    const int ih = ih0 + kh;
    const bool rv = (unsigned)ih < (unsigned)a.h;
    const int off = rv ? (((nn * a.h + ih) * a.w + iw0) * 3 - 1) * 2 : (int)0x80000000;
#pragma unroll
    for (int i = 0; i < 5; ++i) {
      const int o = off + 4 * i;
      dw[kh][i] = __builtin_amdgcn_raw_buffer_load_b32(xr, o < 0 ? (int)0x80000000 : o, 0, 0);
    }
  }
  if (ow == 0) {
    // the column left of the image (halves 1..3: dword 0's high half and
    // dword 1) holds the previous image row's last pixel: zeros
#pragma unroll
    for (int kh = 0; kh < 3; ++kh) {
      dw[kh][0] &= 0xffffu;
      dw[kh][1] = 0;
    }
  }
  // any f16 subnormal among the loaded halves, in the wave:
  // (2|h| - 2) mod 2^16 < 0x7fe
  typedef unsigned short us2 __attribute__((ext_vector_type(2)));
  uint32_t mn = 0xffffffffu;
  {
    const uint32_t two = 0x00020002u, m2 = 0xfffefffeu;
#pragma unroll
    for (int kh = 0; kh < 3; ++kh)
#pragma unroll
      for (int i = 0; i < 5; ++i) {
        uint32_t tv;
        asm("v_pk_mad_u16 %0, %1, %2, %3" : "=v"(tv) : "v"(dw[kh][i]), "v"(two), "s"(m2));
        mn = __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(us2, mn),
                                                                    __builtin_bit_cast(us2, tv)));
      }
  }
  const bool sub = __any((mn & 0xffffu) < 0x7feu || (mn >> 16) < 0x7feu);
  const wrow_t wbase = (wrow_t)(a.wf + oc0);
  float acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
  if (sub)
    stem_pad_accumulate<FE, true>(dw, wbase, a.cout, acc);
  else
    stem_pad_accumulate<FE, false>(dw, wbase, a.cout, acc);
  const size_t yo = (size_t)p * a.y_pix_stride + a.y_c_off + oc0;
  dx::store_outputs_t<2, 16, FE>(a, acc, oc0, (uint8_t*)a.y + yo, s_lut);
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
// the output takes the scalar decoding path.  SiLU: silu_f16_pk_lite (fp16
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
        p01 = silu_f16_pk_lite(p01);
        p23 = silu_f16_pk_lite(p23);
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

bool stem_pad_ok(const DirectArgs& a) {
  const char* e = getenv("DW_STEM_PAD");
  if (e && e[0] == '0') return false;
  return a.kh == 3 && a.kw == 3 && a.cin == 3 && a.cout % 16 == 0 && a.in_kind == 1 && a.out_kind == 2 &&
         a.w_finite && a.sh == 2 && a.sw == 2 && a.pt == 1 && a.pl == 1 && a.h % 2 == 0 && a.w % 2 == 0 &&
         a.ho == a.h / 2 && a.wo == a.w / 2 && a.x_pix_stride == 3 && a.x_c_off == 0 && (uintptr_t)a.x % 4 == 0 &&
         (long long)a.n * a.h * a.w * 6 + 16 < (1ll << 31);
}

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
    if (stem_pad_ok(a)) {
      a.x_bytes = (int)((long long)a.n * a.h * a.w * 6);
      if (a.m > 0) {
        if (a.fast_epi)
          hipLaunchKernelGGL((stem_pad_u8_kernel<true>), grid, dim3(256), 0, st, a);
        else
          hipLaunchKernelGGL((stem_pad_u8_kernel<false>), grid, dim3(256), 0, st, a);
        DW_HIP(hipGetLastError());
      }
      return;
    }
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
  // f32 input whose tile window fits LDS, weights packed by channel quads:
  // the tiled kernel (4 channels per thread, 16 x 16 output pixels per
  // workgroup)
  if (a.wq && a.in_kind == 0 && vin && (a.cin == 32 || a.cin == 64) && a.cout % 4 == 0 &&
      a.kh * a.kw * a.cin <= kTileWRows) {
    constexpr int TH = 16, TW = 16, C = 4;
    const int iwin_w = (TW - 1) * a.sw + a.kw, iwin_h = (TH - 1) * a.sh + a.kh;
    const int pstr = a.cin + 4;
    const size_t lds = (size_t)iwin_h * iwin_w * pstr;
    // (the window's channel quads in at most 24 loads per thread)
    const long long xbytes = (((long long)a.n * a.h * a.w - 1) * a.x_pix_stride + a.x_c_off + a.cin) * 4;
    const int cpp = TH * TW / (a.cin / 4);  // window columns one pass of the workgroup loads
    if (lds <= (size_t)kTileLdsFloats && iwin_h <= 24 && iwin_w <= 2 * cpp && xbytes < (1ll << 31)) {
      const int oes = a.out_kind == 0 ? 4 : (a.out_kind == 1 ? 2 : 1);
      auto aligned = [&](int v) {
        return (C * oes) % v == 0 && (a.y_pix_stride * oes) % v == 0 && (a.y_c_off * oes) % v == 0 &&
               ((uintptr_t)a.y % v) == 0;
      };
      a.vec_out = aligned(16) ? 16 : (aligned(4) ? 4 : 1);
      a.x_bytes = (int)xbytes;
      const int tiles_w = (a.wo + TW - 1) / TW, tiles_h = (a.ho + TH - 1) / TH;
      const dim3 grid((unsigned)(a.n * tiles_w * tiles_h), a.cout / C);
      if (a.cin == 64)
        hipLaunchKernelGGL((conv_tile_f32_kernel<TH, TW, 4>), grid, dim3(TH * TW), 0, st, a, tiles_w,
                           tiles_w * tiles_h, iwin_w, pstr);
      else
        hipLaunchKernelGGL((conv_tile_f32_kernel<TH, TW, 2>), grid, dim3(TH * TW), 0, st, a, tiles_w,
                           tiles_w * tiles_h, iwin_w, pstr);
      DW_HIP(hipGetLastError());
      return;
    }
  }
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

namespace {
__global__ __launch_bounds__(256) void repack_oc4_kernel(const float* __restrict__ w, float4* __restrict__ wq,
                                                         int rows, int cout) {
  const int i = blockIdx.x * 256 + threadIdx.x;  // output float4: (quad, row)
  const int quads = cout / 4;
  if (i >= rows * quads) return;
  const int g = i / rows, r = i - (i / rows) * rows;
  wq[i] = *reinterpret_cast<const float4*>(w + (size_t)r * cout + 4 * g);
}
}  // namespace

void launch_repack_oc4(hipStream_t st, const float* w, float* wq, int rows, int cout) {
  if (cout % 4 != 0 || ((uintptr_t)w & 15) != 0 || ((uintptr_t)wq & 15) != 0) fail(-2, "repack_oc4: alignment");
  const long long n = (long long)rows * (cout / 4);
  if (n == 0) return;
  hipLaunchKernelGGL(repack_oc4_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, w, (float4*)wq, rows,
                     cout);
  DW_HIP(hipGetLastError());
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
