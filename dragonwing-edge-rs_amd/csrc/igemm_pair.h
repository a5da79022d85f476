// Two chained int8 3x3 convolutions (stride 1, padding 1, c -> c -> c
// channels, c = 16, 32 or 64) in one launch, the intermediate tensor kept in
// LDS: the bottleneck of a C2f block (QLinearConv + SiLU table, QLinearConv
// + SiLU table, optionally + the block input through QLinearAdd).
//
// Each launch of a small layer carries a fixed cost of several
// microseconds (dispatch, the first loads' latency, the epilogue, the
// kernel's end), which on the 20x20 .. 160x160 maps of a batch-32 graph is
// most of the layer's time.  Here a workgroup owns R whole output rows of
// one image and every channel (R chosen by the runtime's tuner, a divisor of
// the height):
//
//  * start-up: both convs' weights (all of K, fragment order), their
//    epilogue data and the R + 4 input rows the two 3x3 windows reach (with
//    the one-pixel halo and padding) go to LDS, the rows as whole 16-byte
//    units converted to the MFMA operand (u8 xor 0x80, or the padding
//    pattern), as igemm_rows_kernel stages them;
//  * phase 1: the first conv over the R + 2 rows the second conv's window
//    needs (its halo rows computed twice, once by each neighbouring band),
//    all operands from LDS; its epilogue (requantize, table) writes the
//    u8 results, converted to the second conv's operand form, into a second
//    LDS tile whose padding (the columns beside the image and rows outside
//    it) holds the second conv's padding pattern;
//  * phase 2: the second conv over the R rows from that tile; its epilogue
//    (requantize, table, QLinearAdd of the block input read back from the
//    first tile) stores the u8 output.
//
// The per-output arithmetic is igemm_kernel's (bias' as the accumulator's
// start, requant_bits, the table, qadd_u8), and integer sums do not depend
// on the k-order, so the results are those of the two separate launches.
#pragma once

#include "igemm_kernel.h"

namespace dw {
namespace ig {

struct PairArgs {
  IgemmArgs a1, a2;
  int rows;  // output rows per workgroup
};

// LDS pixel stride in 16-byte units: 8 lanes reading one unit of 8
// consecutive pixels each hit 8 distinct 16-byte bank groups
__host__ __device__ constexpr int pair_su(int c) { return c == 32 ? 2 : (c / 16) | 1; }
// LDS layout (bytes): two epilogue blocks (table 256, bias' 4c, multipliers
// 4c), the k-slice table, both weight sets, the input tile, the
// intermediate tile.
__host__ __device__ constexpr int pair_epi_bytes(int c) { return 256 + 8 * c; }
__host__ __device__ constexpr int pair_tab_off(int c) { return 2 * pair_epi_bytes(c); }
__host__ __device__ constexpr int pair_w_off(int c, int ks) { return (pair_tab_off(c) + ks * 16 + 15) / 16 * 16; }
__host__ __device__ constexpr int pair_x_off(int c, int ks) { return pair_w_off(c, ks) + 2 * ks * c * 64; }
__host__ __device__ constexpr int pair_m_off(int c, int ks, int w, int rows) {
  return pair_x_off(c, ks) + (rows + 4) * (w + 2) * pair_su(c) * 16;
}
// and the second conv's QLinearAdd tables (IgemmArgs::rtab, 2 KB)
__host__ __device__ constexpr int pair_rt_off(int c, int ks, int w, int rows) {
  return pair_m_off(c, ks, w, rows) + (rows + 2) * (w + 2) * pair_su(c) * 16;
}
__host__ __device__ constexpr int pair_lds_bytes(int c, int ks, int w, int rows) {
  return pair_rt_off(c, ks, w, rows) + 2048;
}
constexpr int kPairFill = 8;  // input units each thread of a 4-wave workgroup loads at start-up (at most)
// 16-pixel blocks a wave computes at a time (accumulators CB x PBC): 4
// waves take 128 VGPRs (256 for 64 channels, one workgroup a CU), 16 waves
// (four a SIMD) 128
__host__ __device__ constexpr int pair_pbc(int cb, int nw, bool res) {
  return nw == 4 ? (cb == 1 ? 8 : (cb == 2 ? 6 : 5)) : (cb == 1 ? 4 : (cb == 2 ? 3 : (res ? 1 : 2)));
}

// CB: 16-channel blocks (c / 16); RES: the second epilogue adds the block
// input; NW: waves (4 or 16).  Both phases walk their 16-pixel blocks PBC at
// a time per wave (blocks wave * PBC + NW * PBC * j ..), so any band height
// fits the registers.
template <int CB, bool RES, int NW>
__global__ __launch_bounds__(64 * NW, NW == 4 ? (CB <= 2 ? 2 : 1) : 1) void igemm_pair_kernel(const PairArgs p) {
  constexpr int C = CB * 16;
  constexpr int PBC = pair_pbc(CB, NW, RES);
  constexpr int NT = 64 * NW;
  constexpr int FILL = kPairFill * 4 / NW;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const IgemmArgs& a1 = p.a1;
  const IgemmArgs& a2 = p.a2;
  const int W = a1.w, H = a1.h, R = p.rows;
  const int TW = W + 2;
  constexpr int CU = C / 16;       // 16-byte units per pixel
  constexpr int SU = pair_su(C);   // LDS pixel stride in units
  const int KS = a1.ksteps;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // XCD-aware tile order, as igemm_kernel: tile = (image, band)
  const int nwg = gridDim.x;
  const int bid = blockIdx.x;
  const int xcd = bid & 7, idx = bid >> 3;
  const int base = nwg >> 3, rem = nwg & 7;
  const int tile = xcd * base + min(xcd, rem) + idx;
  const int bands = H / R;
  const int n = tile / bands;
  const int r0 = (tile - n * bands) * R;

  uint8_t* const s_lut1 = smem;
  uint8_t* const s_bias1 = smem + 256;
  uint8_t* const s_ms1 = smem + 256 + 4 * C;
  uint8_t* const s_lut2 = smem + pair_epi_bytes(C);
  uint8_t* const s_bias2 = s_lut2 + 256;
  uint8_t* const s_ms2 = s_lut2 + 256 + 4 * C;
  int* const s_tab = reinterpret_cast<int*>(smem + pair_tab_off(C));
  uint8_t* const s_w1 = smem + pair_w_off(C, KS);
  uint8_t* const s_w2 = s_w1 + KS * C * 64;
  uint8_t* const s_x = smem + pair_x_off(C, KS);
  uint8_t* const s_m = smem + pair_m_off(C, KS, W, R);
  const lds_f32p s_rt = (lds_f32p)(smem + pair_rt_off(C, KS, W, R));

  // ---- both weight sets (fragment order) and both epilogue blocks, direct to LDS
  const int frag_lane = ((lane & 15) * 64 + (lane >> 4) * 16);
  {
    const int nfr = KS * CB;
    for (int f = wave; f < 2 * nfr; f += NW) {
      const int second = f >= nfr;
      const int ff = f - second * nfr;
      const int sl = ff / CB, cb = ff - sl * CB;
      const uint8_t* src = (second ? a2.wpk : a1.wpk) +
                           (((uint32_t)sl * (second ? a2.cout_pad : a1.cout_pad) + cb * 16) * 64u + frag_lane);
      __builtin_amdgcn_global_load_lds((const void*)src,
                                       (__attribute__((address_space(3))) void*)((second ? s_w2 : s_w1) + ff * 1024),
                                       16, 0, 0);
    }
  }
  if (wave == 0 && lane < C / 4) {
    __builtin_amdgcn_global_load_lds((const void*)(a1.bias_i + lane * 4), (__attribute__((address_space(3))) void*)s_bias1,
                                     16, 0, 0);
    __builtin_amdgcn_global_load_lds((const void*)(a2.bias_i + lane * 4), (__attribute__((address_space(3))) void*)s_bias2,
                                     16, 0, 0);
  }
  if (wave == 1 && lane < C / 4) {
    __builtin_amdgcn_global_load_lds((const void*)(a1.mscale + lane * 4), (__attribute__((address_space(3))) void*)s_ms1,
                                     16, 0, 0);
    __builtin_amdgcn_global_load_lds((const void*)(a2.mscale + lane * 4), (__attribute__((address_space(3))) void*)s_ms2,
                                     16, 0, 0);
  }
  if (wave == 2 && lane < 16) {
    __builtin_amdgcn_global_load_lds((const void*)(a1.lut + lane * 16), (__attribute__((address_space(3))) void*)s_lut1,
                                     16, 0, 0);
    __builtin_amdgcn_global_load_lds((const void*)(a2.lut + lane * 16), (__attribute__((address_space(3))) void*)s_lut2,
                                     16, 0, 0);
  }
  // the QLinearAdd tables: 2 KB, two loads of 64 lanes from lane 0 up
  if (RES && a2.rtab && wave == 3) {
    __builtin_amdgcn_global_load_lds((const void*)(a2.rtab + lane * 4),
                                     (__attribute__((address_space(3))) void*)(smem + pair_rt_off(C, KS, W, R)), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((const void*)(a2.rtab + 256 + lane * 4),
                                     (__attribute__((address_space(3))) void*)(smem + pair_rt_off(C, KS, W, R) + 1024), 16,
                                     0, 0);
  }

  // ---- input tile: rows r0 - 2 .. r0 + R + 1, columns -1 .. W, raw
  // 16-byte units (out-of-image units: out-of-range loads, which return
  // zero), all in flight together
  const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc((void*)a1.x, (short)0, a1.x_bytes, 0x00020000);
  const int units = (R + 4) * TW * CU;
  const float r_tw = 1.0f / (float)TW;
  u32x4 xv[FILL];
  int xdst[FILL];  // LDS offset of the unit, or -1 for none
  bool xin[FILL];
#pragma unroll
  for (int i = 0; i < FILL; ++i) {
    const int u = tid + i * NT;
    xdst[i] = -1;
    xin[i] = false;
    if (u < units) {
      const int ip = u / CU;  // CU is a power of two
      const int cu = u - ip * CU;
      const int tr = div_small(ip, TW, r_tw), tc = ip - tr * TW;
      const int ih = r0 - 2 + tr, iw = tc - 1;
      const bool ok = (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W;
      const int off = ok ? (((n * H + ih) * W + iw) * a1.x_pix_stride + a1.x_c_off + cu * 16) : (int)0x80000000;
      xv[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrsrc, off, 0, 0));
      xdst[i] = (ip * SU + cu) * 16;
      xin[i] = ok;
    }
  }

  // ---- k-slice offsets (shared by both convs: same tile geometry and
  // channel count): slice s of k-step q is 16 input channels of one tap
  for (int e = tid; e < KS * 4; e += NT) {
    const int k = e * 16;
    int off = 0;
    if (k < 9 * C) {
      const int tap = k / C, ci = k - (k / C) * C;
      const int kh = tap / 3, kw = tap - (tap / 3) * 3;
      off = ((kh * TW + kw) * SU + ci / 16) * 16;
    }
    s_tab[e] = off;
  }

  // ---- the intermediate tile's padding: columns -1 and W of every row,
  // and whole rows outside the image, hold the second conv's padding
  // pattern (phase 1 writes the rest)
  {
    const u32x4 pad2 = u32x4{a2.xpad, a2.xpad, a2.xpad, a2.xpad};
    const int mun = (R + 2) * TW * CU;
    for (int u = tid; u < mun; u += NT) {
      const int ip = u / CU;
      const int cu = u - ip * CU;
      const int tr = div_small(ip, TW, r_tw), tc = ip - tr * TW;
      const int ih = r0 - 1 + tr;
      if (tc == 0 || tc == TW - 1 || (unsigned)ih >= (unsigned)H)
        *reinterpret_cast<u32x4*>(s_m + (ip * SU + cu) * 16) = pad2;
    }
  }

  // everything above has landed (direct loads included); write the tile
  __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
  for (int i = 0; i < FILL; ++i) {
    if (xdst[i] >= 0) {
      const uint32_t key = xin[i] ? a1.xxor : a1.xpad;
      *reinterpret_cast<u32x4*>(s_x + xdst[i]) = xv[i] ^ key;
    }
  }
  __syncthreads();

  const int cq = 4 * (lane >> 4);
  const int* const my_tab = s_tab + (lane >> 4);

  // One chunk of PBC blocks: the k-loop over both operands in LDS (the next
  // k-step's fragments read while this one's MFMAs run).  src: the tile the
  // windows read; wl: this lane's weight fragments; pbase: each block's
  // top-left tap in the tile.
  auto chunk_gemm = [&](v4i (&acc)[CB][PBC], const uint8_t* src, const uint8_t* wl, const int (&pbase)[PBC]) {
    v4i afr[2][CB], bfr[2][PBC];
#define DW_READ_K(q_, slot_)                                                            \
  {                                                                                     \
    const int toff_ = my_tab[(q_) * 4];                                                 \
    _Pragma("unroll") for (int cb = 0; cb < CB; ++cb)                                   \
      afr[slot_][cb] = *reinterpret_cast<const v4i*>(wl + ((q_) * CB + cb) * 1024);     \
    _Pragma("unroll") for (int pb = 0; pb < PBC; ++pb)                                  \
      bfr[slot_][pb] = *reinterpret_cast<const v4i*>(src + pbase[pb] + toff_);          \
  }
    DW_READ_K(0, 0);
    for (int q0 = 0; q0 < KS; q0 += 2) {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int q = q0 + r;
        if (q < KS) {
          if (q + 1 < KS) DW_READ_K(q + 1, (r + 1) & 1);
#pragma unroll
          for (int cb = 0; cb < CB; ++cb)
#pragma unroll
            for (int pb = 0; pb < PBC; ++pb)
              acc[cb][pb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(afr[r][cb], bfr[r][pb], acc[cb][pb], 0, 0, 0);
        }
      }
    }
#undef DW_READ_K
  };

  // ================= phase 1: (R + 2) x W pixels of the intermediate
  {
    const int np = (R + 2) * W;
    const int nb = (np + 15) / 16;
    const int qbase = 0x4B400000 - a1.y_zp;
    const float qlo = 12582912.0f - (float)a1.y_zp, qhi = qlo + 255.0f;
    const __attribute__((address_space(3))) uint8_t* lut3 = (const __attribute__((address_space(3))) uint8_t*)s_lut1;
    for (int b0 = wave * PBC; b0 < nb; b0 += NW * PBC) {
      int pbase[PBC], poff[PBC];  // window in the input tile; result in the intermediate tile (-1: none)
#pragma unroll
      for (int pb = 0; pb < PBC; ++pb) {
        const int pl = (b0 + pb) * 16 + (lane & 15);
        const int q = pl < np ? pl : 0;
        const int r = div_small(q, W, a1.r_wo), c = q - r * W;
        pbase[pb] = (r * TW + c) * SU * 16;  // tile rows r .. r + 2 feed intermediate row r
        const int ih = r0 - 1 + r;
        poff[pb] = (pl < np && (unsigned)ih < (unsigned)H) ? ((r * TW + c + 1) * SU * 16 + cq) : -1;
      }
      v4i acc[CB][PBC];
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const v4i init = *reinterpret_cast<const v4i*>(s_bias1 + 4 * (cb * 16 + cq));
#pragma unroll
        for (int pb = 0; pb < PBC; ++pb) acc[cb][pb] = init;
      }
      chunk_gemm(acc, s_x, s_w1 + lane * 16, pbase);
      // epilogue 1: requantize, table, then the second conv's operand form
      // (u8 xor 0x80) into the intermediate tile; rows outside the image
      // keep their padding
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const float4 m4 = *reinterpret_cast<const float4*>(s_ms1 + 4 * (cb * 16 + cq));
        const float ms4[4] = {m4.x, m4.y, m4.z, m4.w};
#pragma unroll
        for (int pb = 0; pb < PBC; ++pb) {
          if (poff[pb] < 0) continue;
          uint32_t out = 0;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int qb = requant_bits(acc[cb][pb][r], ms4[r], qlo, qhi);
            const int qi = lut3[(uint32_t)qb - (uint32_t)qbase];
            out |= (uint32_t)qi << (8 * r);
          }
          *reinterpret_cast<uint32_t*>(s_m + poff[pb] + cb * 16) = out ^ a2.xxor;
        }
      }
    }
  }
  __syncthreads();

  // ================= phase 2: R x W output pixels
  {
    const int np = R * W;
    const int nb = (np + 15) / 16;
    const int qbase = 0x4B400000 - a2.y_zp;
    const float qlo = 12582912.0f - (float)a2.y_zp, qhi = qlo + 255.0f;
    const __attribute__((address_space(3))) uint8_t* lut3 = (const __attribute__((address_space(3))) uint8_t*)s_lut2;
    for (int b0 = wave * PBC; b0 < nb; b0 += NW * PBC) {
      int pbase[PBC], pixel[PBC], xres[PBC];  // window; output pixel (-1: none); the residual's unit
#pragma unroll
      for (int pb = 0; pb < PBC; ++pb) {
        const int pl = (b0 + pb) * 16 + (lane & 15);
        const int q = pl < np ? pl : 0;
        const int r = div_small(q, W, a1.r_wo), c = q - r * W;
        pbase[pb] = (r * TW + c) * SU * 16;
        pixel[pb] = pl < np ? (n * H + r0 + r) * W + c : -1;
        xres[pb] = ((r + 2) * TW + c + 1) * SU * 16 + cq;
      }
      v4i acc[CB][PBC];
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const v4i init = *reinterpret_cast<const v4i*>(s_bias2 + 4 * (cb * 16 + cq));
#pragma unroll
        for (int pb = 0; pb < PBC; ++pb) acc[cb][pb] = init;
      }
      chunk_gemm(acc, s_m, s_w2 + lane * 16, pbase);
      // epilogue 2: requantize, table, QLinearAdd of the block input, u8 out
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const float4 m4 = *reinterpret_cast<const float4*>(s_ms2 + 4 * (cb * 16 + cq));
        const float ms4[4] = {m4.x, m4.y, m4.z, m4.w};
#pragma unroll
        for (int pb = 0; pb < PBC; ++pb) {
          if (pixel[pb] < 0) continue;
          uint32_t rres = 0;
          if constexpr (RES) rres = *reinterpret_cast<const uint32_t*>(s_x + xres[pb] + cb * 16) ^ a1.xxor;
          uint32_t out = 0;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int qb = requant_bits(acc[cb][pb][r], ms4[r], qlo, qhi);
            int qi;
            if (RES && a2.rtab) {
              qi = qadd_u8_tab(s_rt, qb - qbase, (rres >> (8 * r)) & 0xff, a2.zy);
            } else {
              qi = lut3[(uint32_t)qb - (uint32_t)qbase];
              if constexpr (RES) qi = qadd_u8(qi, (rres >> (8 * r)) & 0xff, a2);
            }
            out |= (uint32_t)qi << (8 * r);
          }
          uint8_t* yrow = (uint8_t*)a2.y + (size_t)pixel[pb] * a2.y_pix_stride + a2.y_c_off + cb * 16 + cq;
          *reinterpret_cast<uint32_t*>(yrow) = out;
        }
      }
    }
  }
}

}  // namespace ig
}  // namespace dw
