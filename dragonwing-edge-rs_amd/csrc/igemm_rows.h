// Implicit-GEMM 3x3 convolution (stride 1, padding 1, int8 or fp16) over
// whole output rows, with the input rows staged in LDS: the variant for the
// large feature maps.
//
// igemm_kernel loads every im2col row from the input view, so each input
// pixel passes the vector-memory path 9 times (once per tap), 16 pixels x
// 64 bytes per wave instruction; that path's per-CU throughput bounds the
// large 3x3 layers.  Here a workgroup owns NPIX = 320 output pixels, which
// are R = 320 / W whole rows of one image, and BC output channels.  It loads
// the R + 2 input rows its taps touch (with the one-pixel halo, padding
// included) into LDS once, as whole 16-byte units of consecutive channels
// (16 u8 or 8 f16), converted to the MFMA operand there (int8: u8 xor 0x80,
// or the padding pattern; fp16: as they are, padding +0),
// together with all of K's weights; the k-loop then reads both operands
// from LDS and issues no global load.
//
// LDS layout of the input tile: tile pixel (tr, tc) (tr in [0, R + 2), tc
// in [0, W + 2), tile pixel (0, 0) = image pixel (r0 - 1, -1)) holds its
// CU = c_in * esize / 16 units at ((tr * (W + 2) + tc) * SU + u) * 16, with
// SU = CU made odd: the 8 lanes that one LDS cycle serves (8 consecutive
// pixels, one unit each) then fall in 8 distinct 16-byte bank groups.
// A k-step is 64 bytes of K either way (v_mfma_i32_16x16x64_i8 or
// v_mfma_f32_16x16x32_f16), so the same tables serve both element sizes.
//
// Work split: wave w owns the output pixels w * 80 .. w * 80 + 79 of the
// workgroup (PB = 5 blocks of 16) and all BC channels, as igemm_kernel's
// waves do, so the epilogue is igemm_kernel's.
#pragma once

#include "igemm_kernel.h"

namespace dw {

bool igemm_launch_rows_i8_a(hipStream_t st, const IgemmArgs& a, const TileCfg& t, int epv);  // generic, QU8
bool igemm_launch_rows_i8_b(hipStream_t st, const IgemmArgs& a, const TileCfg& t, int epv);  // LUT variants
bool igemm_launch_rows_f16(hipStream_t st, const IgemmArgs& a, const TileCfg& t);

namespace ig {

constexpr int kRowsPix = 320;  // output pixels per workgroup
constexpr int kRowsPB = 5;     // 16-pixel blocks per wave

// LDS pixel stride in 16-byte units for c_in channels of esize bytes
__host__ __device__ constexpr int rows_su(int cin, int esize) { return (cin * esize / 16) | 1; }
// LDS: epilogue data, k-slice offsets, all of K's weights, the input tile.
__host__ __device__ constexpr int rows_tab_off(int bc) { return 256 + 8 * bc; }
__host__ __device__ constexpr int rows_w_off(int bc, int ksteps) { return (rows_tab_off(bc) + ksteps * 16 + 15) / 16 * 16; }
__host__ __device__ constexpr int rows_x_off(int bc, int ksteps) { return rows_w_off(bc, ksteps) + ksteps * bc * 64; }
inline size_t rows_lds_bytes(int bc, int ksteps, int w, int cin, int esize) {
  const int r = kRowsPix / w;
  return (size_t)rows_x_off(bc, ksteps) + (size_t)(r + 2) * (w + 2) * rows_su(cin, esize) * 16;
}
// Input units each thread loads at start-up (at most).
constexpr int kRowsFill = 16;

template <int ESZ, int BC, int EPV>
__global__ __launch_bounds__(256) void igemm_rows_kernel(const IgemmArgs a) {
  constexpr int CB = BC / 16;
  constexpr int PB = kRowsPB;
  constexpr bool FAST = EPV != EPV_GENERIC;
  static_assert(!FAST || ESZ == 1, "specialised epilogues are int8");
  using acc_t = typename std::conditional<ESZ == 1, v4i, v4f>::type;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int KSTEPS = a.ksteps, COUTP = a.cout_pad, CIN = a.cin;
  const int W = a.w, H = a.h;
  const int R = kRowsPix / W;
  const int TW = W + 2;
  const int CU = CIN * ESZ / 16;  // 16-byte units per pixel
  const int SU = CU | 1;          // LDS pixel stride in units

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  // XCD-aware tile order, as igemm_kernel: tile = (image, row tile, channel tile)
  const int nwg = gridDim.x;
  const int bid = blockIdx.x;
  const int xcd = bid & 7, idx = bid >> 3;
  const int base = nwg >> 3, rem = nwg & 7;
  const int tile = xcd * base + min(xcd, rem) + idx;
  const int ctiles = COUTP / BC;
  const int ptile = tile / ctiles;
  const int c0 = (tile - ptile * ctiles) * BC;
  const int rtiles = H / R;
  const int n = ptile / rtiles;
  const int r0 = (ptile - n * rtiles) * R;
  const int pw0 = (n * H + r0) * W;        // the workgroup's first output pixel
  const int p0 = pw0 + wave * (16 * PB);   // this wave's first output pixel

  uint8_t* const s_lut = smem;
  uint8_t* const s_bias = smem + 256;
  uint8_t* const s_ms = smem + 256 + 4 * BC;
  int* const s_tab = reinterpret_cast<int*>(smem + rows_tab_off(BC));
  uint8_t* const s_w = smem + rows_w_off(BC, KSTEPS);
  uint8_t* const s_x = smem + rows_x_off(BC, KSTEPS);

  // ---- weights (all of K, fragment order) and epilogue data, direct to LDS
  const int frag_lane = ((lane & 15) * 64 + (lane >> 4) * 16);
  {
    const int nfr = KSTEPS * CB;
    for (int f = wave; f < nfr; f += 4) {
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
      __builtin_amdgcn_global_load_lds((const void*)(a.lut + lane * 16),
                                       (__attribute__((address_space(3))) void*)s_lut, 16, 0, 0);
  } else if (a.epi == EPI_F16 && a.bias_h) {
    ep.bias_h = reinterpret_cast<const uint16_t*>(s_bias);
    if (wave == 0 && lane < nvalid / 2)
      __builtin_amdgcn_global_load_lds((const void*)(a.bias_h + c0 + lane * 2),
                                       (__attribute__((address_space(3))) void*)s_bias, 4, 0, 0);
  }

  // ---- input tile: raw 16-byte units (out-of-image units: out-of-range
  // loads, which return zero), all in flight together
  const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, a.x_bytes, 0x00020000);
  const int units = (R + 2) * TW * CU;
  const float r_cu = 1.0f / (float)CU, r_tw = 1.0f / (float)TW;
  u32x4 xv[kRowsFill];
  int xdst[kRowsFill];  // LDS offset of the unit, or -1 for none
  bool xin[kRowsFill];
#pragma unroll
  for (int i = 0; i < kRowsFill; ++i) {
    const int u = tid + i * 256;
    xdst[i] = -1;
    xin[i] = false;
    if (u < units) {
      const int ip = div_small(u, CU, r_cu);
      const int cu = u - ip * CU;
      const int tr = div_small(ip, TW, r_tw), tc = ip - tr * TW;
      const int ih = r0 - 1 + tr, iw = tc - 1;
      const bool ok = (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W;
      // byte offset: the view's element offset times the element size
      const int off = ok ? ((((n * H + ih) * W + iw) * a.x_pix_stride + a.x_c_off) * ESZ + cu * 16) : (int)0x80000000;
      xv[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrsrc, off, 0, 0));
      xdst[i] = (ip * SU + cu) * 16;
      xin[i] = ok;
    }
  }

  // ---- k-slice offsets: slice s of k-step q is 16 input channels of one
  // tap; its unit's offset from the pixel's top-left tap in the tile (slices
  // past K: any unit, their weights are zero)
  for (int e = tid; e < KSTEPS * 4; e += 256) {
    const int k = e * (16 / ESZ);  // the slice's first element of K
    int off = 0;
    if (k < 9 * CIN) {
      const int tap = k / CIN, ci = k - (k / CIN) * CIN;
      const int kh = tap / 3, kw = tap - (tap / 3) * 3;
      off = ((kh * TW + kw) * SU + ci * ESZ / 16) * 16;
    }
    s_tab[e] = off;
  }

  // everything above has landed (direct loads included); write the tile
  __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
  for (int i = 0; i < kRowsFill; ++i) {
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

  // this lane's pixels: LDS offset of each block's top-left tap
  int pbase[PB];
#pragma unroll
  for (int pb = 0; pb < PB; ++pb) {
    const int pl = wave * (16 * PB) + pb * 16 + (lane & 15);  // 0 .. 319
    const int r = div_small(pl, W, a.r_wo), c = pl - r * W;
    pbase[pb] = (r * TW + c) * SU * 16;
  }

  acc_t acc[CB][PB];
  const int cq = 4 * (lane >> 4);
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    acc_t init = acc_t{0, 0, 0, 0};
    if constexpr (FAST) {
      if (a.bias_i) init = *reinterpret_cast<const v4i*>(s_bias + 4 * (cb * 16 + cq));
    }
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) acc[cb][pb] = init;
  }

  // ---- k-loop, all operands from LDS; the next k-step's fragments are
  // read while this one's MFMAs run
  const int* const my_tab = s_tab + (lane >> 4);
  const uint8_t* const a_lane = s_w + lane * 16;
  v4i afr[2][CB], bfr[2][PB];
#define DW_READ_K(q_, slot_)                                                                 \
  {                                                                                          \
    const int toff_ = my_tab[(q_) * 4];                                                      \
    _Pragma("unroll") for (int cb = 0; cb < CB; ++cb)                                        \
      afr[slot_][cb] = *reinterpret_cast<const v4i*>(a_lane + ((q_) * CB + cb) * 1024);      \
    _Pragma("unroll") for (int pb = 0; pb < PB; ++pb)                                        \
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
        for (int cb = 0; cb < CB; ++cb)
#pragma unroll
          for (int pb = 0; pb < PB; ++pb) {
            if constexpr (ESZ == 1)
              acc[cb][pb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(afr[r][cb], bfr[r][pb], acc[cb][pb], 0, 0, 0);
            else
              acc[cb][pb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, afr[r][cb]),
                                                                   __builtin_bit_cast(v8h, bfr[r][pb]), acc[cb][pb], 0, 0, 0);
          }
      }
    }
  }
#undef DW_READ_K

  // int8 epilogue: the input tile's LDS, once every wave is done with it,
  // regroups the results (the tile is at least 4 rows of 42 16-byte units)
  uint8_t* xp = nullptr;
  if constexpr (FAST && BC >= 32) {
    __syncthreads();
    xp = s_x + wave * 16 * xpose_row(BC);
  }
  igemm_store<ESZ, BC, PB, EPV>(a, ep, acc, c0, p0, lane, s_ms, s_lut, xp);
}

template <int ESZ, int EPV>
bool launch_rows_tiles(hipStream_t st, const IgemmArgs& a, const TileCfg& t) {
  const int r = kRowsPix / a.w;
  const dim3 grid((unsigned)(a.n * (a.h / r) * (a.cout_pad / t.bc)));
  const size_t lds = rows_lds_bytes(t.bc, a.ksteps, a.w, a.cin, ESZ);
#define DW_B(BC_)                                                                          \
  case BC_:                                                                                \
    hipLaunchKernelGGL((igemm_rows_kernel<ESZ, BC_, EPV>), grid, dim3(256), lds, st, a); \
    return true;
  switch (t.bc) {
    DW_B(96)
    DW_B(80)
    DW_B(64)
    DW_B(48)
    DW_B(32)
    DW_B(16)
  }
#undef DW_B
  return false;
}

}  // namespace ig
}  // namespace dw
