// Implicit-GEMM convolution kernel for CDNA4 matrix cores (gfx950): the
// kernel template shared by the translation units that instantiate it.
//
// The convolution is the GEMM  Y[c][p] = sum_k W[k][c] * X[p][k]  with
//   c = output channel, p = output pixel (n, oh, ow), k = (kh, kw, ci).
// Both operands are consumed as 64-byte rows per k-step (64 int8 or 32 fp16
// values): one wavefront instruction is v_mfma_i32_16x16x64_i8 (int8) or
// v_mfma_f32_16x16x32_f16 (fp16), and each lane supplies a 16-byte slice of
// one row of each operand (row = lane % 16, slice = lane / 16).
//
// Work split: a workgroup (4 waves) owns BC output channels x 64*PB output
// pixels; every wave computes all BC channels of its own 16*PB pixels.
//
// Data movement:
//  * weights (operand A), pre-packed as [k-step][c_out][64 B] rows, are
//    copied to LDS with direct global->LDS loads, in fragment order (one
//    1 KB fragment per wave instruction), in chunks of up to 64 KB (one
//    chunk holds all of K for almost every layer);
//  * im2col rows (operand B) go straight from the NHWC input to the MFMA
//    source registers, through a ring of PD k-steps loaded PD - 1 steps
//    ahead.  The per-lane address arithmetic is a lookup: a per-workgroup
//    LDS table gives, for every 16-byte slice of K, its offset from the
//    pixel's top-left tap and its tap number, and a per-pixel bitmask says
//    which taps lie inside the image.  A 16-byte slice is 16 int8 / 8 fp16
//    consecutive input channels of one tap, so c_in * esize must be a
//    multiple of 16.  Out-of-image taps and k-steps past the end of K use
//    buffer loads with an out-of-range offset (no memory access);
//  * the per-channel epilogue data (bias', multipliers, activation table)
//    are staged in LDS with the first weight chunk, so all start-up loads
//    of a workgroup are in flight together;
//  * workgroups are numbered so that neighbouring tiles land on the same
//    XCD (the hardware deals workgroups round-robin over the 8 XCDs, each
//    with its own L2), so input halos and weights are shared in L2.
//
// u8 inputs are mapped to s8 by xor 0x80 (x - 128); the missing
// (128 - x_zp) * sum_k W is folded into the per-channel bias by the host, so
// int8 results are exact.  Epilogues fuse what the reference runs as
// separate passes: bias, the requantization with its rounding rule, a u8
// activation table, the residual QLinearAdd, or the f16 rounding chain; all
// stores go to channel-strided views, so concat outputs are written in place.
// The common int8 epilogues are compiled as specialisations (EPV) so that
// the per-value work is a straight instruction sequence.
#pragma once

#include "dw_common.h"
#include "dw_device.h"

#include <type_traits>

namespace dw {

// Tile shape of one launch.
struct TileCfg {
  int bc, pb, pd, kchunk;
  int tpw;  // > 0: the persistent small-K kernel with this many pixel tiles per workgroup
};

// Epilogue specialisations.
enum EpiVariant : int {
  EPV_GENERIC = 0,     // any epilogue, decided at run time
  EPV_QU8 = 1,         // requantize to u8
  EPV_QU8_LUT = 2,     // requantize, then the activation table
  EPV_QU8_LUT_RES = 3, // requantize, table, then the residual QLinearAdd
  EPV_QU8_LUT_HEAD = 4 // requantize, table, then the fused u8 -> f16 1x1 head conv
};

// Launch one instantiation (defined in the k_igemm_*.hip files); false if
// no kernel exists for the shape.
bool igemm_launch_i8_a(hipStream_t st, const IgemmArgs& a, const TileCfg& t, int epv);  // generic, QU8
bool igemm_launch_i8_b(hipStream_t st, const IgemmArgs& a, const TileCfg& t, int epv);  // LUT variants
bool igemm_launch_f16(hipStream_t st, const IgemmArgs& a, const TileCfg& t);
bool igemm_launch_head_i8(hipStream_t st, const IgemmArgs& a, const TileCfg& t);  // EPV_QU8_LUT_HEAD

namespace ig {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// LDS layout of a workgroup (bytes):
//   [0, 256)                 activation table (u8)
//   [256, 256 + 4 BC)        bias' (i32) or the f16 bias
//   [256 + 4 BC, 256 + 8 BC) multipliers (f32)
//   then the k-slice table ((ksteps + 2 PD) * 4 int2), then the weight chunk
__host__ __device__ constexpr int lds_table_off(int bc) { return 256 + 8 * bc; }
__host__ __device__ constexpr int lds_chunk_off(int bc, int ksteps, int pd) {
  return lds_table_off(bc) + (ksteps + 2 * pd) * 4 * 8;
}
inline size_t lds_bytes(const TileCfg& t, int ksteps) {
  return (size_t)lds_chunk_off(t.bc, ksteps, t.pd) + (size_t)t.kchunk * t.bc * 64;
}

// n / d for 0 <= n < 2^24 and 1 <= d < 2^23, given rd = 1.0f / d rounded to
// nearest.  The float product n * rd is within 1 of n / d (its relative
// error is below 2^-23, and it is exact for d <= 2), so its truncation is
// floor(n / d) - 1, + 0 or + 1, and one remainder test corrects it.  Every
// intermediate is an integer below 2^24 in magnitude, so the float
// arithmetic is exact (and full rate, unlike 32-bit integer multiplies).
__device__ __forceinline__ int div_small(int n, int d, float rd) {
  const float nf = (float)n, df = (float)d;
  float q = truncf(nf * rd);
  const float r = fmaf(-q, df, nf);
  q += (r < 0.0f) ? -1.0f : ((r >= df) ? 1.0f : 0.0f);
  return (int)q;
}

// Per-channel epilogue parameters of the workgroup's channel tile, staged
// in LDS at the start (indexed by the channel's position in the tile).
struct EpiLds {
  const int* bias;         // EPI_QU8 bias' or null
  const float* ms;         // EPI_QU8 multipliers
  const uint8_t* lut;      // EPI_QU8 table (256 entries) or null
  const uint16_t* bias_h;  // EPI_F16 bias or null
};

// f16 epilogue (EPI_F16) is CpuGraphRuntime's chain: conv result rounded to
// f16, then the bias pass, the activation and the residual add, each on
// stored f16.  The MFMA sums already differ from the reference's order, so
// these results are held to the fp16 tolerance, and the store runs the
// chain two channels at a time in packed f16 (IEEE operands, silu_f16_pk_lite).

// QLinearConv requantization of one accumulator (bias' already added):
// rint(acc * M) + y_zp, saturated to [0, 255] (ONNX QLinearConv, RNE).
__device__ __forceinline__ int requant_u8(int acc, float m, float zp) {
  const float q = rintf((float)acc * m) + zp;
  return (int)__builtin_amdgcn_fmed3f(q, 0.0f, 255.0f);
}

// The same value with fewer instructions, for the specialised epilogues.
// With f = acc * M rounded to f32 (as above), f + 1.5 * 2^23 rounds f to an
// integer by the current mode (nearest, ties to even: the constant is even,
// so the parity of the sum is that of rint(f)); for |f| < 2^22 the sum is
// exactly 1.5 * 2^23 + rint(f), and outside that range it still grows with
// f, so clamping the sum to [1.5 * 2^23 - y_zp, 1.5 * 2^23 + 255 - y_zp]
// saturates exactly as above.  Returns the clamped sum's bit pattern, which
// is qbase + rint(f) + y_zp with qbase = 0x4B400000 - y_zp (lo, hi: the
// clamp bounds as floats).
__device__ __forceinline__ int requant_bits(int acc, float m, float lo, float hi) {
  const float f = (float)acc * m;
  return __builtin_bit_cast(int, __builtin_amdgcn_fmed3f(f + 12582912.0f, lo, hi));
}

// QLinearAdd of the table output a and the residual b (QuantizeLinear of
// the sum of both dequantized operands, RNE, saturated).
__device__ __forceinline__ int qadd_u8(int qa, int rb, const IgemmArgs& a) {
  const float f = (float)(qa - a.za) * a.ra + (float)(rb - a.zb) * a.rb;
  const float g = rintf(f) + (float)a.zy;
  return (int)__builtin_amdgcn_fmed3f(g, 0.0f, 255.0f);
}

// qadd_u8 of the table output of requant byte qt and the residual rb from
// the tables of IgemmArgs::rtab in LDS (rt: its 512 floats): the sum of the
// two rounded products, rounded to the nearest even integer by adding
// 1.5 * 2^23 (exact while the sum is below 2^22 in magnitude), the zero
// point and the clamp to 0..255 in one med3 of the biased value, as
// requant_bits does.
typedef const __attribute__((address_space(3))) float* lds_f32p;
__device__ __forceinline__ int qadd_u8_tab(lds_f32p rt, int qt, int rb, int zy) {
  const float s = rt[qt] + rt[256 + rb];
  const float lo = 12582912.0f - (float)zy;
  const float t = __builtin_amdgcn_fmed3f(s + 12582912.0f, lo, lo + 255.0f);
  return __builtin_bit_cast(int, t) - (0x4B400000 - zy);
}

// Generic epilogue for one 16x16 block: this lane holds channels ch..ch+3
// of pixel p (channel cl..cl+3 of the tile).
template <int ESZ, typename AccT>
__device__ __forceinline__ void epilogue4(const IgemmArgs& a, const EpiLds& e, const AccT& v, int ch, int cl,
                                          int p) {
  const size_t yo = (size_t)p * a.y_pix_stride + a.y_c_off + ch;
  if constexpr (ESZ == 1) {
    if (a.epi == EPI_QU8) {
      const int4 bi = e.bias ? *reinterpret_cast<const int4*>(e.bias + cl) : make_int4(0, 0, 0, 0);
      const float4 ms = *reinterpret_cast<const float4*>(e.ms + cl);
      uint32_t rres = 0;
      if (a.res)
        rres = *reinterpret_cast<const uint32_t*>((const uint8_t*)a.res + (size_t)p * a.r_pix_stride +
                                                  a.r_c_off + ch);
      const int accs[4] = {v[0] + bi.x, v[1] + bi.y, v[2] + bi.z, v[3] + bi.w};
      const float mss[4] = {ms.x, ms.y, ms.z, ms.w};
      uint32_t out = 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        int qi = requant_u8(accs[r], mss[r], (float)a.y_zp);
        if (e.lut) qi = e.lut[qi];
        if (a.res) qi = qadd_u8(qi, (rres >> (8 * r)) & 0xff, a);
        out |= (uint32_t)qi << (8 * r);
      }
      *reinterpret_cast<uint32_t*>((uint8_t*)a.y + yo) = out;
    } else if (a.epi == EPI_QS8_REF) {
      uint32_t out = 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float f = (float)v[r] * a.tscale;
        f = fminf(fmaxf(f, -128.0f), 127.0f);
        f = roundf(f);
        if (a.act == ACT_RELU) f = fmaxf(f, 0.0f);
        out |= ((uint32_t)(int)f & 0xffu) << (8 * r);
      }
      *reinterpret_cast<uint32_t*>((uint8_t*)a.y + yo) = out;
    } else {  // EPI_I32
      *reinterpret_cast<int4*>((int*)a.y + yo) = make_int4(v[0], v[1], v[2], v[3]);
    }
  } else {
    uint2 rres = make_uint2(0, 0);
    if (a.res)
      rres = *reinterpret_cast<const uint2*>((const uint16_t*)a.res + (size_t)p * a.r_pix_stride +
                                             a.r_c_off + ch);
    // the f16 chain two channels at a time in packed f16
    h16x2 p01 = pk_f2h(v[0], v[1]), p23 = pk_f2h(v[2], v[3]);
    if (e.bias_h) {
      p01 = p01 + pk_make(e.bias_h[cl], e.bias_h[cl + 1]);
      p23 = p23 + pk_make(e.bias_h[cl + 2], e.bias_h[cl + 3]);
    }
    if (a.act == ACT_SILU) {
      p01 = silu_f16_pk_lite(p01);
      p23 = silu_f16_pk_lite(p23);
    } else if (a.act != ACT_NONE) {
      p01 = pk_make(f16_act_bits(pk_lo(p01), a.act), f16_act_bits(pk_hi(p01), a.act));
      p23 = pk_make(f16_act_bits(pk_lo(p23), a.act), f16_act_bits(pk_hi(p23), a.act));
    }
    if (a.res) {
      p01 = p01 + __builtin_bit_cast(h16x2, rres.x);
      p23 = p23 + __builtin_bit_cast(h16x2, rres.y);
    }
    const uint2 out = make_uint2(__builtin_bit_cast(uint32_t, p01), __builtin_bit_cast(uint32_t, p23));
    // a sibling GEMM's second conv stores to its own output view; a channel
    // tile lies wholly on one side of the split, so the choice is made once
    // per tile (scalar selects, one store)
    const bool g2 = a.y2 && __builtin_amdgcn_readfirstlane(ch - cl) >= a.split;
    uint16_t* const ybase = (uint16_t*)(g2 ? a.y2 : a.y);
    const int ypix = g2 ? a.y2_pix_stride : a.y_pix_stride;
    const int ycoff = g2 ? a.y2_c_off - a.split : a.y_c_off;
    *reinterpret_cast<uint2*>(ybase + (size_t)p * ypix + ycoff + ch) = out;
    if (a.y_up) {
      // the nearest 2x upsample: the same values at the pixel's four pixels
      const int hw = a.ho * a.wo;
      const int nn = div_small(p, hw, a.r_hwo);
      const int r = p - nn * hw;
      const int oh = div_small(r, a.wo, a.r_wo);
      const int ow = r - oh * a.wo;
      uint16_t* u = (uint16_t*)a.y_up +
                    ((size_t)(nn * 2 * a.ho + 2 * oh) * (2 * a.wo) + 2 * ow) * a.up_pix_stride + a.up_c_off + ch;
      const size_t upr = (size_t)2 * a.wo * a.up_pix_stride;
      *reinterpret_cast<uint2*>(u) = out;
      *reinterpret_cast<uint2*>(u + a.up_pix_stride) = out;
      *reinterpret_cast<uint2*>(u + upr) = out;
      *reinterpret_cast<uint2*>(u + upr + a.up_pix_stride) = out;
    }
  }
}

// k-slice table: slice q of K (16 bytes, one filter tap) is at element
// offset .x from the pixel's top-left tap and belongs to tap .y (31 = past
// the end of K: always padding).  It does not depend on the pixel, so a
// workgroup builds it once, for nq slices.
__device__ __forceinline__ void build_ktab(int2* ktab, int nq, int ce, const IgemmArgs& a, int tid) {
  const int kelems = a.kh * a.kw * a.cin;
  for (int q = tid; q < nq; q += 256) {
    const int e = q * ce;
    int2 t = make_int2(0, 31);
    if (e < kelems) {
      const int tap = div_small(e, a.cin, a.r_cin);
      const int ci = e - tap * a.cin;
      const int kh = div_small(tap, a.kw, a.r_kw);
      const int kw = tap - kh * a.kw;
      t = make_int2((kh * a.w + kw) * a.x_pix_stride + ci, tap);
    }
    ktab[q] = t;
  }
}

// This lane's pixels p0 + pb*16 + (lane & 15): element offset of the
// top-left tap and the in-image bit of every tap (none for pixels past the
// end, or for every pixel when !live).  Each pixel of the wave is
// decomposed once (lane L takes pixel p0 + L mod 16 PB), and lanes fetch
// their pixels' values from there.
template <int PB>
__device__ __forceinline__ void pixel_setup(const IgemmArgs& a, int p0, int lane, bool live, int (&pbase)[PB],
                                            uint32_t (&tmask)[PB]) {
  const int hw_o = a.ho * a.wo;
  const int p = p0 + (lane & (16 * PB - 1));
  const bool pv = live && p < a.m;
  const int pp = pv ? p : 0;
  const int nn = div_small(pp, hw_o, a.r_hwo);
  const int r = pp - nn * hw_o;
  const int oh = div_small(r, a.wo, a.r_wo);
  const int ow = r - oh * a.wo;
  const int ih0 = oh * a.sh - a.pt, iw0 = ow * a.sw - a.pl;
  const int base = ((nn * a.h + ih0) * a.w + iw0) * a.x_pix_stride + a.x_c_off;
  // filter rows [rlo, rhi) and columns [clo, chi) fall inside the image
  const int rlo = max(0, -ih0), rhi = min(a.kh, a.h - ih0);
  const int clo = max(0, -iw0), chi = min(a.kw, a.w - iw0);
  const uint32_t cols = chi > clo ? (1u << chi) - (1u << clo) : 0u;
  uint32_t m = 0;
  for (int kh = 0; kh < a.kh; ++kh) m |= (kh >= rlo && kh < rhi) ? cols << (kh * a.kw) : 0u;
  m = pv ? m : 0u;
#pragma unroll
  for (int pb = 0; pb < PB; ++pb) {
    const int src = pb * 16 + (lane & 15);
    pbase[pb] = __shfl(base, src);
    tmask[pb] = (uint32_t)__shfl((int)m, src);
  }
}

// The table of channel tile c0: a sibling GEMM's second conv has its own.
__device__ __forceinline__ const uint8_t* tile_lut(const IgemmArgs& a, int c0) {
  return (a.y2 && c0 >= a.split) ? a.lut2 : a.lut;
}

// LDS rows the int8 epilogue uses to regroup results (per wave: 16 pixels
// x xpose_row(BC) bytes).  A row of d dwords puts the 64 lanes' 4-byte writes
// (16 pixels x 4 channel quads, dwords d * i + j) in 64 distinct banks when
// d = 4 (mod 8): BC + 16 bytes for BC a multiple of 32, BC bytes otherwise
// (48, 80).
__host__ __device__ constexpr int xpose_row(int bc) { return bc % 32 == 0 ? bc + 16 : bc; }
__host__ __device__ constexpr int xpose_bytes(int bc) { return 4 * 16 * xpose_row(bc); }

// EPV_QU8_LUT_HEAD: the tile holds every channel of its pixels (BC >= the
// conv's c_out, c0 = 0).  Per 16-pixel block the u8 results (requantized,
// table) go to this wave's LDS rows xp (16 pixels x xpose_row(BC) bytes),
// and each lane reads back the 8 consecutive channels of its pixel that the
// fp16 MFMA's B operand takes, dequantized as DequantizeLinear does; the
// head's 1x1 conv then runs on the fp16 matrix cores and its f16 outputs
// are stored: conv1x1_u8_f16_mfma_kernel's arithmetic (same operands, same
// k-order, same epilogue), so the outputs are that kernel's.  The 1x1's
// weight fragments come from global memory (L2) into registers.
template <int BC, int PB>
__device__ __forceinline__ void igemm_store_head(const IgemmArgs& a, const v4i (&acc)[BC / 16][PB], int p0, int lane,
                                                 const uint8_t* s_ms, const uint8_t* s_lut, uint8_t* xp,
                                                 int pend) {
  constexpr int CB = BC / 16;
  constexpr int KS2 = (BC + 31) / 32;  // the 1x1's k-steps over the BC u8 channels
  const int cq = 4 * (lane >> 4);
  const int qbase = 0x4B400000 - a.y_zp;
  const float qlo = 12582912.0f - (float)a.y_zp, qhi = qlo + 255.0f;
  const __attribute__((address_space(3))) uint8_t* lut3 = (const __attribute__((address_space(3))) uint8_t*)s_lut;
  uint8_t* const xrow = xp + (lane & 15) * xpose_row(BC);
  const int ncb2 = (a.h_cout + 15) / 16;
  v8h wf[CB][KS2];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
#pragma unroll
    for (int ks = 0; ks < KS2; ++ks)
      wf[cb][ks] = cb < ncb2 ? *reinterpret_cast<const v8h*>(a.h_wfrag + (((size_t)cb * KS2 + ks) * 64 + lane) * 8)
                             : v8h{};
  float4 msr[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) msr[cb] = *reinterpret_cast<const float4*>(s_ms + 4 * (cb * 16 + cq));
  const float zp = (float)a.h_zp, scale = a.h_scale;
  const uint32_t zpb = (uint32_t)(a.h_zp & 0xff) * 0x01010101u;
#pragma unroll
  for (int pb = 0; pb < PB; ++pb) {
    const int p = p0 + pb * 16 + (lane & 15);
    asm volatile("" ::: "memory");  // the previous block's reads are issued
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const float ms4[4] = {msr[cb].x, msr[cb].y, msr[cb].z, msr[cb].w};
      uint32_t out = 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int qb = requant_bits(acc[cb][pb][r], ms4[r], qlo, qhi);
        out |= (uint32_t)lut3[(uint32_t)qb - (uint32_t)qbase] << (8 * r);
      }
      *reinterpret_cast<uint32_t*>(xrow + cb * 16 + cq) = out;
    }
    asm volatile("" ::: "memory");  // one wave's LDS operations run in order
    v8h xf[KS2];
#pragma unroll
    for (int ks = 0; ks < KS2; ++ks) {
      const int k = ks * 32 + (lane >> 4) * 8;
      const uint2 raw = k < BC ? *reinterpret_cast<const uint2*>(xrow + k) : make_uint2(zpb, zpb);
      xf[ks] = dequant_u8x8_f16(raw, zp, scale);
    }
    uint16_t* yrow = a.h_y + (size_t)p * a.h_y_pix_stride + a.h_y_c_off;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const int ch = cb * 16 + cq;
      if (cb >= ncb2) break;  // wave-uniform
      v4f acc2 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < KS2; ++ks) acc2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[cb][ks], xf[ks], acc2, 0, 0, 0);
      if (p < pend && ch < a.h_cout)
        *reinterpret_cast<uint2*>(yrow + ch) = conv1x1_f16_finish(acc2, a.h_bias ? a.h_bias + ch : nullptr, a.h_act);
    }
  }
}

// Epilogue of a workgroup's tile: this lane holds channels c0 + cb*16 + cq
// .. +3 of pixel p0 + pb*16 + (lane & 15) for every block (cb, pb).  The
// specialised int8 epilogues (EPV) take bias' from the accumulators' start
// values and the multipliers and table from LDS.  With xp (this wave's
// xpose_row(BC) x 16 bytes of LDS), a pixel's u8 results are regrouped
// there so that each lane stores 16 consecutive channels: one 16-byte store
// per lane and 4 blocks, whole cache lines when the output rows are dense,
// instead of a 4-byte store per lane and block (a 16-channel tile gains
// nothing: it has one block).  Pixels at or past min(a.m, pend) are not
// stored (pend: the end of the caller's pixel range, when its last blocks
// belong to another wave).
template <int ESZ, int BC, int PB, int EPV, typename AccT>
__device__ __forceinline__ void igemm_store(const IgemmArgs& a, const EpiLds& ep, AccT (&acc)[BC / 16][PB], int c0,
                                            int p0, int lane, const uint8_t* s_ms, const uint8_t* s_lut,
                                            uint8_t* xp = nullptr, int pend = 0x7fffffff) {
  constexpr int CB = BC / 16;
  constexpr bool FAST = EPV != EPV_GENERIC;
  const int cq = 4 * (lane >> 4);
  const int plim = min(a.m, pend);
  if constexpr (EPV == EPV_QU8_LUT_HEAD) {
    igemm_store_head<BC, PB>(a, acc, p0, lane, s_ms, s_lut, xp, plim);
  } else if constexpr (FAST) {
    // the output view of this channel tile: a sibling GEMM's second conv
    // (c0 >= split) writes its own tensor, channel c0 - split of it
    const bool g2 = a.y2 != nullptr && c0 >= a.split;
    uint8_t* const ybase = (uint8_t*)(g2 ? a.y2 : a.y);
    const int ypix = g2 ? a.y2_pix_stride : a.y_pix_stride;
    const int ycoff = g2 ? a.y2_c_off - a.split : a.y_c_off;
    const bool full = c0 + BC <= a.cout;
    const bool wide = CB >= 2 && xp != nullptr && full && (ypix & 15) == 0 &&
                      ((ycoff + c0) & 15) == 0 && (((uintptr_t)ybase) & 15) == 0 &&
                      (!a.y_up || ((a.up_pix_stride & 15) == 0 && ((a.up_c_off + c0) & 15) == 0 &&
                                   (((uintptr_t)a.y_up) & 15) == 0));
    uint8_t* const xrow = wide ? xp + (lane & 15) * xpose_row(BC) : nullptr;
    const int qbase = 0x4B400000 - a.y_zp;
    const float qlo = 12582912.0f - (float)a.y_zp, qhi = qlo + 255.0f;
    const __attribute__((address_space(3))) uint8_t* lut3 = (const __attribute__((address_space(3))) uint8_t*)s_lut;
    float4 msr[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) msr[cb] = *reinterpret_cast<const float4*>(s_ms + 4 * (cb * 16 + cq));
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) {
      const int p = p0 + pb * 16 + (lane & 15);
      if (p >= plim) continue;
      uint8_t* yrow = ybase + (size_t)p * ypix + ycoff + c0 + cq;
      // the pixel's top-left pixel in the upsampled view, if any
      size_t up = 0;
      if (a.y_up) {
        const int hw = a.ho * a.wo;
        const int nn = div_small(p, hw, a.r_hwo);
        const int r = p - nn * hw;
        const int oh = div_small(r, a.wo, a.r_wo);
        const int ow = r - oh * a.wo;
        up = ((size_t)(nn * 2 * a.ho + 2 * oh) * (2 * a.wo) + 2 * ow) * a.up_pix_stride + a.up_c_off + c0;
      }
      const size_t upr = (size_t)2 * a.wo * a.up_pix_stride;  // one upsampled row
      uint32_t rres[CB];
      if constexpr (EPV == EPV_QU8_LUT_RES) {
        const uint8_t* rrow = (const uint8_t*)a.res + (size_t)p * a.r_pix_stride + a.r_c_off + c0 + cq;
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
          rres[cb] = (full || c0 + cb * 16 + cq < a.cout) ? *reinterpret_cast<const uint32_t*>(rrow + cb * 16) : 0u;
      }
      if (wide) asm volatile("" ::: "memory");  // the previous block's reads are issued
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        if (!full && c0 + cb * 16 + cq >= a.cout) continue;
        const float ms4[4] = {msr[cb].x, msr[cb].y, msr[cb].z, msr[cb].w};
        uint32_t out = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int qb = requant_bits(acc[cb][pb][r], ms4[r], qlo, qhi);
          int qi;
          if constexpr (EPV != EPV_QU8)
            qi = lut3[(uint32_t)qb - (uint32_t)qbase];
          else
            qi = qb - qbase;
          if constexpr (EPV == EPV_QU8_LUT_RES) qi = qadd_u8(qi, (rres[cb] >> (8 * r)) & 0xff, a);
          out |= (uint32_t)qi << (8 * r);
        }
        if (wide) {
          *reinterpret_cast<uint32_t*>(xrow + cb * 16 + cq) = out;
        } else {
          *reinterpret_cast<uint32_t*>(yrow + cb * 16) = out;
          if (a.y_up) {
            uint8_t* u = (uint8_t*)a.y_up + up + cb * 16 + cq;
            *reinterpret_cast<uint32_t*>(u) = out;
            *reinterpret_cast<uint32_t*>(u + a.up_pix_stride) = out;
            *reinterpret_cast<uint32_t*>(u + upr) = out;
            *reinterpret_cast<uint32_t*>(u + upr + a.up_pix_stride) = out;
          }
        }
      }
      if (wide) {
        // the pixel's 4 lanes wrote its BC channels; lane g now stores
        // blocks g, g + 4, ... (one wave's LDS operations run in order)
        asm volatile("" ::: "memory");
        uint8_t* const ydst = yrow - cq;
#pragma unroll
        for (int i = 0; i < (CB + 3) / 4; ++i) {
          const int cb = 4 * i + (lane >> 4);
          if (cb < CB) {
            const uint4 v = *reinterpret_cast<const uint4*>(xrow + cb * 16);
            *reinterpret_cast<uint4*>(ydst + cb * 16) = v;
            if (a.y_up) {
              uint8_t* u = (uint8_t*)a.y_up + up + cb * 16;
              *reinterpret_cast<uint4*>(u) = v;
              *reinterpret_cast<uint4*>(u + a.up_pix_stride) = v;
              *reinterpret_cast<uint4*>(u + upr) = v;
              *reinterpret_cast<uint4*>(u + upr + a.up_pix_stride) = v;
            }
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const int ch = c0 + cb * 16 + cq;
      if (ch >= a.cout) continue;
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) {
        const int p = p0 + pb * 16 + (lane & 15);
        if (p < plim) epilogue4<ESZ>(a, ep, acc[cb][pb], ch, ch - c0, p);
      }
    }
  }
}

// SK: K fits in the start-up loads (ksteps <= PD - 1, and in one weight
// chunk), so the k-loop issues no loads.
template <int ESZ, int BC, int PB, int PD, int EPV, bool SK>
__global__ __launch_bounds__(256) void igemm_kernel(const IgemmArgs a) {
  constexpr int CB = BC / 16;       // 16-channel blocks (all channels of the tile per wave)
  constexpr int CE = 16 / ESZ;      // elements per 16-byte slice
  constexpr int WPIX = 16 * PB;     // pixels per wave
  constexpr int WGPIX = 4 * WPIX;   // pixels per workgroup
  constexpr bool FAST = EPV != EPV_GENERIC;
  using acc_t = typename std::conditional<ESZ == 1, v4i, v4f>::type;
  static_assert(BC % 16 == 0 && PD >= 2, "tile");
  static_assert(!FAST || ESZ == 1, "specialised epilogues are int8");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const uint8_t* __restrict__ X = a.x;
  const uint8_t* __restrict__ WPK = a.wpk;
  const int KSTEPS = a.ksteps, COUTP = a.cout_pad;
  const int KCH = a.kchunk;
  const uint32_t XXOR = a.xxor;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  // XCD-aware tile order: workgroup b runs on XCD b % 8; give each XCD a
  // contiguous range of tiles (channel tiles of one pixel tile adjacent).
  const int nwg = gridDim.x;
  const int bid = blockIdx.x;
  const int xcd = bid & 7, idx = bid >> 3;
  const int base = nwg >> 3, rem = nwg & 7;
  const int tile = xcd * base + min(xcd, rem) + idx;
  const int ctiles = COUTP / BC;
  const int ptile = tile / ctiles;
  const int c0 = (tile - ptile * ctiles) * BC;
  const int p0 = ptile * WGPIX + wave * WPIX;

  uint8_t* const s_lut = smem;
  uint8_t* const s_bias = smem + 256;
  uint8_t* const s_ms = smem + 256 + 4 * BC;
  int2* const ktab = reinterpret_cast<int2*>(smem + lds_table_off(BC));
  uint8_t* const s_chunk = smem + lds_chunk_off(BC, KSTEPS, PD);

  // ---- k-slice table (the ring reads up to k-step KSTEPS + 2 * PD - 3,
  // see the main loop) and this lane's pixels
  build_ktab(ktab, (KSTEPS + 2 * PD) * 4, CE, a, tid);
  int pbase[PB];
  uint32_t tmask[PB];
  pixel_setup<PB>(a, p0, lane, true, pbase, tmask);

  // Weight chunks go to LDS with direct global->LDS loads: one 1 KB
  // fragment per wave instruction, lane l writing bytes [16 l, 16 l + 16).
  const int frag_lane = ((lane & 15) * 64 + (lane >> 4) * 16);  // this lane's slice in a 16-row block
#define DW_ISSUE_A(s_first)                                                                         \
  {                                                                                                 \
    const int nfr_ = (min(KSTEPS, (s_first) + KCH) - (s_first)) * CB;                               \
    for (int f = wave; f < nfr_; f += 4) {                                                          \
      const int sl = f / CB, cb = f - (f / CB) * CB;                                                \
      const uint8_t* src = WPK + (((uint32_t)((s_first) + sl) * COUTP + c0 + cb * 16) * 64u + frag_lane); \
      __builtin_amdgcn_global_load_lds((const void*)src,                                            \
                                       (__attribute__((address_space(3))) void*)(s_chunk + f * 1024), \
                                       16, 0, 0);                                                   \
    }                                                                                               \
  }
  // this wave's LDS writes (and loads) have landed, then everyone's have
#define DW_LDS_FENCE()              \
  __builtin_amdgcn_s_waitcnt(0);    \
  __syncthreads();

  // Epilogue parameters of the channel tile (one wave each): bias' and
  // multipliers, the activation table, or the f16 bias.
  const int nvalid = min(BC, a.cout - c0);  // a multiple of 4
  EpiLds ep{nullptr, nullptr, nullptr, nullptr};
  if (a.epi == EPI_QU8) {
    ep.bias = a.bias_i ? reinterpret_cast<const int*>(s_bias) : nullptr;
    ep.ms = reinterpret_cast<const float*>(s_ms);
    ep.lut = a.lut ? s_lut : nullptr;
  } else if (a.epi == EPI_F16 && a.bias_h) {
    ep.bias_h = reinterpret_cast<const uint16_t*>(s_bias);
  }

  __syncthreads();  // the k-slice table is complete

  // im2col loads are buffer loads over the input view: padding taps and
  // k-steps past the end of K use an out-of-range offset, which returns
  // zero without a memory access.
  const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc((void*)X, (short)0, a.x_bytes, 0x00020000);
  const int2* my_tab = ktab + (lane >> 4);
#define DW_LOAD_B(tab_entry, dst, dkey)                                                              \
  {                                                                                                 \
    const int2 t_ = (tab_entry);                                                                    \
    _Pragma("unroll") for (int pb = 0; pb < PB; ++pb) {                                             \
      const bool ok = (tmask[pb] >> t_.y) & 1u;                                                     \
      const int off = ok ? (pbase[pb] + t_.x) * ESZ : (int)0x80000000;                              \
      dst[pb] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrsrc, off, 0, 0)); \
      dkey[pb] = ok ? XXOR : a.xpad;                                                                \
    }                                                                                               \
  }

  // ---- im2col ring: k-step s lives in bq[s % PD], loaded PD - 1 steps
  // ahead.  The ring holds the raw loads and their in-image flags; the xor
  // and the pad select happen when the k-step is consumed, so nothing waits
  // for a load before its k-step comes up.  Every k-step issues exactly PB
  // loads, also past the last k-step, so the compiler's load counters stay
  // exact and a k-step waits only for its own loads.
  u32x4 bq[PD][PB];
  uint32_t bkey[PD][PB];  // xor key: u8 -> s8 for in-image taps, the pad value for padding
#pragma unroll
  for (int r = 0; r < PD - 1; ++r) DW_LOAD_B(my_tab[r * 4], bq[r], bkey[r]);
  // table entry of the next k-step to load, read one k-step ahead so that a
  // load's address never waits for an LDS read
  int2 tnext = my_tab[(PD - 1) * 4];

  // All of the workgroup's start-up loads are in flight together: the first
  // PD - 1 im2col k-steps, the first weight chunk and the epilogue data.
  DW_ISSUE_A(0);
  if (a.epi == EPI_QU8) {
    if (wave == 0 && a.bias_i && lane < nvalid / 4)
      __builtin_amdgcn_global_load_lds((const void*)(a.bias_i + c0 + lane * 4),
                                       (__attribute__((address_space(3))) void*)s_bias, 16, 0, 0);
    if (wave == 1 && lane < nvalid / 4)
      __builtin_amdgcn_global_load_lds((const void*)(a.mscale + c0 + lane * 4),
                                       (__attribute__((address_space(3))) void*)s_ms, 16, 0, 0);
    if (wave == 2 && a.lut && lane < 16)
      __builtin_amdgcn_global_load_lds((const void*)(tile_lut(a, c0) + lane * 16),
                                       (__attribute__((address_space(3))) void*)s_lut, 16, 0, 0);
  } else if (a.epi == EPI_F16 && a.bias_h) {
    if (wave == 0 && lane < nvalid / 2)
      __builtin_amdgcn_global_load_lds((const void*)(a.bias_h + c0 + lane * 2),
                                       (__attribute__((address_space(3))) void*)s_bias, 4, 0, 0);
  }
  DW_LDS_FENCE();

  // Accumulators; the specialised int8 epilogues start them at bias'.
  const int cq = 4 * (lane >> 4);  // this lane's first channel within a 16-channel block
  acc_t acc[CB][PB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    acc_t init = acc_t{0, 0, 0, 0};
    if constexpr (FAST) {
      if (a.bias_i) init = *reinterpret_cast<const v4i*>(s_bias + 4 * (cb * 16 + cq));
    }
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) acc[cb][pb] = init;
  }

  // Weight fragments are read FA fragments ahead of their MFMA: fragment
  // j = k-step * CB + cb lives in afr[j % (2 FA)], and its read goes to a
  // slot no live fragment occupies, so the ring needs no register copies
  // (PD * CB is a multiple of 2 FA, so the slots repeat every PD k-steps).
  // A read ahead that falls past the current chunk reads a stale row (the
  // row index is clamped into the chunk) and is read again once that chunk
  // has been loaded.
  constexpr int FA = (PB >= 4 && CB >= 2) ? 2 : CB;
  constexpr int RS = 2 * FA;
  static_assert((PD * CB) % RS == 0 && FA <= CB, "fragment ring");
  const uint8_t* const a_lane = s_chunk + lane * 16;
#define DW_FRAG(row_, cb_) (*reinterpret_cast<const v4i*>(a_lane + ((row_) * CB + (cb_)) * 1024))
  v4i afr[RS];
#pragma unroll
  for (int i = 0; i < FA; ++i) afr[i] = DW_FRAG(0, i);

  // k-step s_, held in ring slot r_ (a compile-time index): the pad select,
  // then each weight fragment's MFMAs, with the read of fragment j + FA
  // issued ahead of them.
#define DW_MMA_STEP(r_, s_)                                                                          \
  {                                                                                                  \
    u32x4 bcur[PB];                                                                                  \
    _Pragma("unroll") for (int pb = 0; pb < PB; ++pb) {                                              \
      if constexpr (ESZ == 1)                                                                        \
        bcur[pb] = bq[r_][pb] ^ bkey[r_][pb];                                                        \
      else                                                                                           \
        bcur[pb] = bq[r_][pb]; /* f16 padding is +0, what the out-of-range load returns */          \
    }                                                                                                \
    _Pragma("unroll") for (int cb = 0; cb < CB; ++cb) {                                              \
      const int j_ = (r_) * CB + cb;                                                                 \
      const v4i af = afr[j_ % RS];                                                                   \
      const int ahead_row = min((s_) + (cb + FA) / CB - chunk0, KCH - 1); /* fragment j + FA */      \
      afr[(j_ + FA) % RS] = DW_FRAG(ahead_row, (cb + FA) % CB);                                      \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); /* this read, then the MFMAs */            \
      __builtin_amdgcn_sched_group_barrier(0x008, PB, 0);                                            \
      _Pragma("unroll") for (int pb = 0; pb < PB; ++pb) {                                            \
        if constexpr (ESZ == 1) {                                                                    \
          acc[cb][pb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, __builtin_bit_cast(v4i, bcur[pb]), \
                                                              acc[cb][pb], 0, 0, 0);                 \
        } else {                                                                                     \
          acc[cb][pb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(                                      \
              __builtin_bit_cast(v8h, af), __builtin_bit_cast(v8h, bcur[pb]), acc[cb][pb], 0, 0, 0); \
        }                                                                                            \
      }                                                                                              \
    }                                                                                                \
  }

  int next_chunk = KCH, chunk0 = 0;
  if constexpr (SK) {
    // Small K: the start-up loads brought all of it.
#pragma unroll
    for (int r = 0; r < PD - 1; ++r)
      if (r < KSTEPS) DW_MMA_STEP(r, r);
  } else {
    for (int s0 = 0; s0 < KSTEPS; s0 += PD) {
#pragma unroll
      for (int r = 0; r < PD; ++r) {
        const int s = s0 + r;
        if (s < KSTEPS && s == next_chunk) {
          __syncthreads();  // every wave is done with the previous chunk
          chunk0 = s;
          next_chunk = s + KCH;
          DW_ISSUE_A(s);
          DW_LDS_FENCE();
#pragma unroll
          for (int i = 0; i < FA; ++i) afr[(r * CB + i) % RS] = DW_FRAG(0, i);
        }
        DW_LOAD_B(tnext, bq[(r + PD - 1) % PD], bkey[(r + PD - 1) % PD]);
        tnext = my_tab[(s + PD) * 4];
        if (s < KSTEPS) DW_MMA_STEP(r, s);
      }
    }
  }
#undef DW_MMA_STEP
#undef DW_FRAG
#undef DW_ISSUE_A
#undef DW_LDS_FENCE
#undef DW_LOAD_B

  // int8 epilogue: the weight chunk's LDS, once every wave is done with it,
  // regroups the results (when the chunk is large enough)
  uint8_t* xp = nullptr;
  if constexpr (FAST && BC >= 32) {
    if (KCH * BC * 64 >= xpose_bytes(BC)) {
      __syncthreads();
      xp = s_chunk + wave * 16 * xpose_row(BC);
    }
  }
  igemm_store<ESZ, BC, PB, EPV>(a, ep, acc, c0, p0, lane, s_ms, s_lut, xp);
}

// Launch of the instantiation for a tile shape (the caller checked that it
// is one of the shapes below).
template <int ESZ, int BC, int EPV>
bool launch_bc(hipStream_t st, const IgemmArgs& a, const TileCfg& t, dim3 grid) {
  const size_t lds = lds_bytes(t, a.ksteps);
#define DW_T(PB, PD)                                                                             \
  if (t.pb == PB && t.pd == PD) {                                                                \
    if (a.ksteps <= PD - 1 && a.ksteps <= t.kchunk)                                              \
      hipLaunchKernelGGL((igemm_kernel<ESZ, BC, PB, PD, EPV, true>), grid, dim3(256), lds, st, a);  \
    else                                                                                         \
      hipLaunchKernelGGL((igemm_kernel<ESZ, BC, PB, PD, EPV, false>), grid, dim3(256), lds, st, a); \
    return true;                                                                                 \
  }
  DW_T(4, 4)
  DW_T(2, 6)
  DW_T(1, 8)
#undef DW_T
  return false;
}

template <int ESZ, int EPV>
bool launch_tiles(hipStream_t st, const IgemmArgs& a, const TileCfg& t) {
  const int wgpix = 64 * t.pb;
  const dim3 grid((unsigned)(((a.m + wgpix - 1) / wgpix) * (a.cout_pad / t.bc)));
  switch (t.bc) {
    case 128: return launch_bc<ESZ, 128, EPV>(st, a, t, grid);
    case 96: return launch_bc<ESZ, 96, EPV>(st, a, t, grid);
    case 80: return launch_bc<ESZ, 80, EPV>(st, a, t, grid);
    case 64: return launch_bc<ESZ, 64, EPV>(st, a, t, grid);
    case 48: return launch_bc<ESZ, 48, EPV>(st, a, t, grid);
    case 32: return launch_bc<ESZ, 32, EPV>(st, a, t, grid);
    case 16: return launch_bc<ESZ, 16, EPV>(st, a, t, grid);
  }
  return false;
}

}  // namespace ig
}  // namespace dw
