// Band-tile implicit GEMM for 3x3 convolutions (stride 1 or 2, padding 1,
// int8 or fp16): one workgroup of 8 or 16 waves owns R whole output rows of one image
// (R chosen by the graph runtime's tuner, a divisor of the height) and BC
// output channels, so a layer runs as one round of workgroups, about one a
// CU, whatever its width.
//
// The row-tile kernel (igemm_rows.h) fixes its tile at 320 output pixels,
// which on the 80x80 maps of a batch-32 graph makes 640 workgroups for 512
// slots: a second, quarter-full round, and each round pays the start-up
// loads, the k-loop and the epilogue one after the other.  Here the start-up
// is the row-tile kernel's (all of K's weights and the R + 2 input rows, with
// halo and padding, go to LDS once, the rows converted to the MFMA operand:
// int8 u8 xor 0x80 or the padding pattern, fp16 as they are), and then each
// wave walks its own contiguous range of the band's 16-pixel blocks, PBC
// blocks at a time, both operands read from LDS (the next k-step's
// fragments while this one's MFMAs run).  The ranges of the waves differ
// by at most one block; blocks past a range's end in its last chunk are
// skipped (wave-uniform) and never stored.  Each wave has its own LDS rows
// for the epilogue's regrouping, so a wave's epilogue overlaps the other
// waves' k-loops.
//
// LDS layout: epilogue data [table 256][bias' 4 BC][multipliers 4 BC], the
// k-slice offsets, the weights (fragment order, [k-step][block][64 lanes x
// 16 B]), the input tile (S (R - 1) + 3 rows of S (W - 1) + 3 pixels for
// output rows W wide at stride S, pixels of SU 16-byte units, SU = c_in *
// esize / 16 made odd: 8 consecutive pixels' units fall in 8 distinct bank
// groups), the waves' regroup rows.
//
// The per-output arithmetic and the epilogues are igemm_kernel's
// (igemm_store), and integer sums do not depend on the k-order, so int8
// results are those of every other tile shape; fp16 sums run over the same
// k-steps in the same order as the row-tile kernel.
#pragma once

#include "igemm_kernel.h"

namespace dw {

bool igemm_launch_band_i8_a(hipStream_t st, const IgemmArgs& a, const TileCfg& t, int epv);  // generic, QU8
bool igemm_launch_band_i8_b(hipStream_t st, const IgemmArgs& a, const TileCfg& t, int epv);  // LUT variants
bool igemm_launch_band_f16(hipStream_t st, const IgemmArgs& a, const TileCfg& t);

namespace ig {

constexpr int kBandFill = 16;  // input units each thread of an 8-wave workgroup loads at start-up (at most)

// 16-pixel blocks per chunk (accumulators CB x PBC) for NW waves: with 8
// waves (256 VGPRs) 64-channel tiles take a wave's whole range (6 or 7
// blocks on the large maps) in one pass of the k-loop, 80-channel tiles
// measured fastest at 4 (6 was slower, 7 spills); with 16 waves (four a
// SIMD, 128 VGPRs) the chunks are what fits without spilling
__host__ __device__ constexpr int band_pbc(int cb, int nw) {
  return nw == 8 ? (cb <= 2 ? 8 : (cb <= 4 ? 7 : (cb == 5 ? 4 : 2)))
                 : (cb == 1 ? 6 : (cb == 2 ? 4 : (cb <= 5 ? 2 : 1)));
}
__host__ __device__ constexpr int band_su(int cu) { return cu | 1; }
__host__ __device__ constexpr int band_tab_off(int bc) { return 256 + 8 * bc; }
__host__ __device__ constexpr int band_w_off(int bc, int ks) { return (band_tab_off(bc) + ks * 16 + 15) / 16 * 16; }
__host__ __device__ constexpr int band_x_off(int bc, int ks) { return band_w_off(bc, ks) + ks * bc * 64; }
// input tile of a band of `rows` output rows `wo` pixels wide at stride s
// (1 or 2): s (rows - 1) + 3 input rows of s (wo - 1) + 3 columns
__host__ __device__ constexpr int band_tile_rows(int rows, int s) { return s * (rows - 1) + 3; }
__host__ __device__ constexpr int band_tile_w(int wo, int s) { return s * (wo - 1) + 3; }
__host__ __device__ constexpr int band_tile_bytes(int rows, int wo, int cu, int s) {
  return band_tile_rows(rows, s) * band_tile_w(wo, s) * band_su(cu) * 16;
}
__host__ __device__ constexpr int band_xp_off(int bc, int ks, int rows, int wo, int cu, int s) {
  return band_x_off(bc, ks) + band_tile_bytes(rows, wo, cu, s);
}
inline size_t band_lds_bytes(int bc, int ks, int rows, int wo, int cu, int nw, int s) {
  return (size_t)band_xp_off(bc, ks, rows, wo, cu, s) + (size_t)nw * 16 * xpose_row(bc);
}

template <int ESZ, int BC, int EPV, int NW, int S>
__global__ __launch_bounds__(64 * NW) void igemm_band_kernel(const IgemmArgs a) {
  static_assert(S == 1 || S == 2, "stride 1 or 2 (both axes)");
  constexpr int CB = BC / 16;
  constexpr int PBC = band_pbc(CB, NW);
  constexpr int kBandWaves = NW;
  constexpr int kBandThreads = 64 * NW;
  constexpr int FILL = kBandFill * 8 / NW;  // input units a thread loads at start-up (at most)
  constexpr bool FAST = EPV != EPV_GENERIC;
  static_assert(!FAST || ESZ == 1, "specialised epilogues are int8");
  using acc_t = typename std::conditional<ESZ == 1, v4i, v4f>::type;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int KSTEPS = a.ksteps, COUTP = a.cout_pad, CIN = a.cin;
  const int W = a.wo, H = a.ho, R = a.band_rows;  // output map and band height
  const int TW = band_tile_w(W, S);
  const int TE = (TW + 1) >> 1;  // stride 2: the tile's even columns, stored first
  const int CU = CIN * ESZ / 16;  // 16-byte units per pixel
  const int SU = band_su(CU);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // XCD-aware tile order, as igemm_kernel: tile = (image, band, channel tile)
  const int nwg = gridDim.x;
  const int bid = blockIdx.x;
  const int xcd = bid & 7, idx = bid >> 3;
  const int base = nwg >> 3, rem = nwg & 7;
  const int tile = xcd * base + min(xcd, rem) + idx;
  const int ctiles = COUTP / BC;
  const int ptile = tile / ctiles;
  const int c0 = (tile - ptile * ctiles) * BC;
  const int bands = H / R;
  const int n = ptile / bands;
  const int r0 = (ptile - n * bands) * R;
  const int pw0 = (n * H + r0) * W;  // the band's first output pixel

  uint8_t* const s_lut = smem;
  uint8_t* const s_bias = smem + 256;
  uint8_t* const s_ms = smem + 256 + 4 * BC;
  int* const s_tab = reinterpret_cast<int*>(smem + band_tab_off(BC));
  uint8_t* const s_w = smem + band_w_off(BC, KSTEPS);
  uint8_t* const s_x = smem + band_x_off(BC, KSTEPS);
  uint8_t* const s_xp = smem + band_xp_off(BC, KSTEPS, R, W, CU, S);

  // ---- weights (all of K, fragment order) and epilogue data, direct to LDS
  const int frag_lane = ((lane & 15) * 64 + (lane >> 4) * 16);
  {
    const int nfr = KSTEPS * CB;
    for (int f = wave; f < nfr; f += kBandWaves) {
      const int sl = f / CB, cb = f - sl * CB;
      const uint8_t* src = a.wpk + (((uint32_t)sl * COUTP + c0 + cb * 16) * 64u + frag_lane);
      __builtin_amdgcn_global_load_lds((const void*)src, (__attribute__((address_space(3))) void*)(s_w + f * 1024),
                                       16, 0, 0);
    }
  }
  const int nvalid = min(BC, a.cout - c0);
  EpiLds ep{nullptr, nullptr, nullptr, nullptr};
  if (a.epi == EPI_QU8) {
    ep.bias = a.bias_i ? reinterpret_cast<const int*>(s_bias) : nullptr;
    ep.ms = reinterpret_cast<const float*>(s_ms);
    ep.lut = a.lut ? s_lut : nullptr;
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
    ep.bias_h = reinterpret_cast<const uint16_t*>(s_bias);
    if (wave == 0 && lane < nvalid / 2)
      __builtin_amdgcn_global_load_lds((const void*)(a.bias_h + c0 + lane * 2),
                                       (__attribute__((address_space(3))) void*)s_bias, 4, 0, 0);
  }

  // ---- input tile: input rows S r0 - 1 .. S (r0 + R - 1) + 1, columns
  // -1 .. S (W - 1) + 1, raw 16-byte units (out-of-image units: out-of-range
  // loads, which return zero), all in flight together.  At stride 2 a row
  // keeps its even columns first, then its odd ones, so the pixels a tap
  // reads for consecutive output pixels stay one pixel (SU units) apart.
  const int IH = a.h, IW = a.w;
  const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, a.x_bytes, 0x00020000);
  const int units = band_tile_rows(R, S) * TW * CU;
  const float r_cu = 1.0f / (float)CU, r_tw = 1.0f / (float)TW;
  u32x4 xv[FILL];
  int xdst[FILL];  // LDS offset of the unit, or -1 for none
  bool xin[FILL];
#pragma unroll
  for (int i = 0; i < FILL; ++i) {
    const int u = tid + i * kBandThreads;
    xdst[i] = -1;
    xin[i] = false;
    if (u < units) {
      const int ip = div_small(u, CU, r_cu);
      const int cu = u - ip * CU;
      const int tr = div_small(ip, TW, r_tw), tc = ip - tr * TW;
      const int ih = S * r0 - 1 + tr, iw = tc - 1;
      const bool ok = (unsigned)ih < (unsigned)IH && (unsigned)iw < (unsigned)IW;
      // byte offset: the view's element offset times the element size
      const int off = ok ? ((((n * IH + ih) * IW + iw) * a.x_pix_stride + a.x_c_off) * ESZ + cu * 16) : (int)0x80000000;
      xv[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrsrc, off, 0, 0));
      const int pos = S == 1 ? tc : ((tc & 1) ? TE + (tc >> 1) : (tc >> 1));
      xdst[i] = ((tr * TW + pos) * SU + cu) * 16;
      xin[i] = ok;
    }
  }

  // ---- k-slice offsets: slice s of k-step q is 16 bytes of input channels
  // of one tap; its unit's offset from the pixel's top-left tap in the tile
  // (slices past K: any unit, their weights are zero)
  for (int e = tid; e < KSTEPS * 4; e += kBandThreads) {
    const int k = e * (16 / ESZ);  // the slice's first element of K
    int off = 0;
    if (k < 9 * CIN) {
      const int tap = k / CIN, ci = k - (k / CIN) * CIN;
      const int kh = tap / 3, kw = tap - (tap / 3) * 3;
      const int kc = S == 1 ? kw : ((kw & 1) ? TE : (kw >> 1));  // column position from the pixel's
      off = ((kh * TW + kc) * SU + ci * ESZ / 16) * 16;
    }
    s_tab[e] = off;
  }

  // everything above has landed (direct loads included); write the tile
  __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
  for (int i = 0; i < FILL; ++i) {
    if (xdst[i] >= 0) {
      if constexpr (ESZ == 1) {
        const uint32_t key = xin[i] ? a.xxor : a.xpad;
        *reinterpret_cast<u32x4*>(s_x + xdst[i]) = xv[i] ^ key;
      } else {
        *reinterpret_cast<u32x4*>(s_x + xdst[i]) = xv[i];  // padding: the zeros of the out-of-range load
      }
    }
  }
  __syncthreads();

  // ---- this wave's blocks [bbeg, bend) of the band's R * W pixels
  const int np = R * W;
  const int nb = (np + 15) / 16;
  const int bbeg = (wave * nb) / kBandWaves, bend = ((wave + 1) * nb) / kBandWaves;
  const int pend = pw0 + min(bend * 16, np);  // pixels from here on are another wave's
  const int cq = 4 * (lane >> 4);
  const int* const my_tab = s_tab + (lane >> 4);
  const uint8_t* const a_lane = s_w + lane * 16;
  uint8_t* const xp = (FAST && (BC >= 32 || EPV == EPV_QU8_LUT_HEAD)) ? s_xp + wave * 16 * xpose_row(BC) : nullptr;

  for (int b0 = bbeg; b0 < bend; b0 += PBC) {
    const int nvb = min(PBC, bend - b0);  // blocks of this chunk (wave-uniform)
    int pbase[PBC];
#pragma unroll
    for (int pb = 0; pb < PBC; ++pb) {
      const int pl = (b0 + pb) * 16 + (lane & 15);
      const int q = (pb < nvb && pl < np) ? pl : 0;
      const int r = div_small(q, W, a.r_wo), c = q - r * W;
      pbase[pb] = (S * r * TW + c) * SU * 16;
    }
    acc_t acc[CB][PBC];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      acc_t init = acc_t{0, 0, 0, 0};
      if constexpr (FAST) {
        if (a.bias_i) init = *reinterpret_cast<const v4i*>(s_bias + 4 * (cb * 16 + cq));
      }
#pragma unroll
      for (int pb = 0; pb < PBC; ++pb) acc[cb][pb] = init;
    }

    v4i afr[2][CB], bfr[2][PBC];
#define DW_READ_K(q_, slot_)                                                                 \
  {                                                                                          \
    const int toff_ = my_tab[(q_) * 4];                                                      \
    _Pragma("unroll") for (int cb = 0; cb < CB; ++cb)                                        \
      afr[slot_][cb] = *reinterpret_cast<const v4i*>(a_lane + ((q_) * CB + cb) * 1024);      \
    _Pragma("unroll") for (int pb = 0; pb < PBC; ++pb)                                       \
      bfr[slot_][pb] = *reinterpret_cast<const v4i*>(s_x + pbase[pb] + toff_);               \
  }
    DW_READ_K(0, 0);
    for (int q0 = 0; q0 < KSTEPS; q0 += 2) {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int q = q0 + r;
        if (q < KSTEPS) {
          if (q + 1 < KSTEPS) DW_READ_K(q + 1, (r + 1) & 1);
#pragma unroll
          for (int pb = 0; pb < PBC; ++pb) {
            if (pb >= nvb) break;  // wave-uniform
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
              if constexpr (ESZ == 1)
                acc[cb][pb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(afr[r][cb], bfr[r][pb], acc[cb][pb], 0, 0, 0);
              else
                acc[cb][pb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    __builtin_bit_cast(v8h, afr[r][cb]), __builtin_bit_cast(v8h, bfr[r][pb]), acc[cb][pb], 0, 0, 0);
            }
          }
        }
      }
    }
#undef DW_READ_K
    igemm_store<ESZ, BC, PBC, EPV>(a, ep, acc, c0, pw0 + b0 * 16, lane, s_ms, s_lut, xp, pend);
  }
}

template <int ESZ, int BC, int EPV, int NW>
void launch_band_bc(hipStream_t st, const IgemmArgs& a, const TileCfg& t) {
  const int rows = a.band_rows;
  const dim3 grid((unsigned)(a.n * (a.ho / rows) * (a.cout_pad / t.bc)));
  const size_t lds = band_lds_bytes(t.bc, a.ksteps, rows, a.wo, a.cin * ESZ / 16, NW, a.sh);
  // the stride is a template argument: the stride-1 code has no stride-2 terms
  if (a.sh == 2)
    hipLaunchKernelGGL((igemm_band_kernel<ESZ, BC, EPV, NW, 2>), grid, dim3(64 * NW), lds, st, a);
  else
    hipLaunchKernelGGL((igemm_band_kernel<ESZ, BC, EPV, NW, 1>), grid, dim3(64 * NW), lds, st, a);
}

// t.tpw: -4 the 8-wave form, -5 the 16-wave form
template <int ESZ, int EPV>
bool launch_band_tiles(hipStream_t st, const IgemmArgs& a, const TileCfg& t) {
#define DW_BAND(BC_)                                                              \
  case BC_:                                                                       \
    if (t.tpw == -5)                                                              \
      launch_band_bc<ESZ, BC_, EPV, 16>(st, a, t);                                \
    else                                                                          \
      launch_band_bc<ESZ, BC_, EPV, 8>(st, a, t);                                 \
    return true;
  switch (t.bc) {
    DW_BAND(128)
    DW_BAND(80)
    DW_BAND(64)
    DW_BAND(32)
    DW_BAND(16)
  }
#undef DW_BAND
  return false;
}

}  // namespace ig
}  // namespace dw
