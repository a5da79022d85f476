// Implicit-GEMM convolution with the weights streamed through LDS one k-step
// at a time: the variant for long K.
//
// The tile, the im2col ring and the epilogue are those of igemm_kernel.h.
// What differs is the weight path.  igemm_kernel stages a whole chunk of
// the channel tile's weights before its k-loop starts (and again at every
// chunk boundary), so every workgroup of a launch first waits for its whole
// chunk, all at the same time.  Here each wave loads its share of k-step
// s + LW's weights (whole 1 KB fragments, cb = wave + 4 i) into a register
// ring at k-step s, writes k-step s + 2's share into a 4-slot LDS ring, and
// one barrier per k-step makes it visible to the other waves before they
// read it (one k-step ahead of its MFMAs).  The weight traffic overlaps the
// MFMAs and a workgroup starts after its first two k-steps have landed.
//
// Every load goes to registers (no direct-to-LDS loads anywhere in the
// kernel), so the compiler's own waits for loads are exact: it counts loads
// of one kind completing in order, which it cannot assume once
// direct-to-LDS loads are in flight (it then waits for all of them), and
// the start-up waits only for k-steps 0 and 1 and the first im2col k-step.  LDS slot reuse: k-step
// s + 2's slot last held k-step s - 2, whose fragments every wave read
// before the barrier of k-step s.
#pragma once

#include "igemm_kernel.h"

namespace dw {

bool igemm_launch_st_i8_a(hipStream_t st, const IgemmArgs& a, const TileCfg& t, int epv);  // generic, QU8
bool igemm_launch_st_i8_b(hipStream_t st, const IgemmArgs& a, const TileCfg& t, int epv);  // LUT variants
bool igemm_launch_st_f16(hipStream_t st, const IgemmArgs& a, const TileCfg& t);

namespace ig {

// LDS ring slots (BC * 64 bytes each) after the k-slice table, then 1 KB
// per wave for the writes that are not part of the ring (see below).
constexpr int kStSlots = 4;
inline size_t st_lds_bytes(int bc, int ksteps, int pd) {
  return (size_t)lds_chunk_off(bc, ksteps, pd) + (size_t)kStSlots * bc * 64 + 4096;
}

template <int ESZ, int BC, int PB, int PD, int EPV>
__global__ __launch_bounds__(256) void igemm_stream_kernel(const IgemmArgs a) {
  constexpr int CB = BC / 16;
  constexpr int CE = 16 / ESZ;
  constexpr int WPIX = 16 * PB;
  constexpr int WGPIX = 4 * WPIX;
  constexpr bool FAST = EPV != EPV_GENERIC;
  constexpr int NWV = (CB + 3) / 4;  // weight fragments per wave and k-step (at most)
  // weight loads run LW k-steps ahead (a multiple or divisor of PD, so the
  // rings line up over the unrolled loop)
  constexpr int LW = PD == 4 ? (NWV > 1 ? 4 : 8) : PD;
  constexpr int NW = kStSlots;
  using acc_t = typename std::conditional<ESZ == 1, v4i, v4f>::type;
  static_assert(BC % 16 == 0 && CB <= 8 && PD >= 2 && PD % 2 == 0 && LW > 2, "tile");
  static_assert(!FAST || ESZ == 1, "specialised epilogues are int8");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const uint8_t* __restrict__ X = a.x;
  const uint8_t* __restrict__ WPK = a.wpk;
  const int KSTEPS = a.ksteps, COUTP = a.cout_pad;
  const uint32_t XXOR = a.xxor;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  // XCD-aware tile order, as igemm_kernel
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
  uint8_t* const s_ring = smem + lds_chunk_off(BC, KSTEPS, PD);

  build_ktab(ktab, (KSTEPS + 2 * PD) * 4, CE, a, tid);
  int pbase[PB];
  uint32_t tmask[PB];
  pixel_setup<PB>(a, p0, lane, true, pbase, tmask);
  const int nvalid = min(BC, a.cout - c0);
  EpiLds ep{nullptr, nullptr, nullptr, nullptr};
  if (a.epi == EPI_QU8) {
    ep.bias = a.bias_i ? reinterpret_cast<const int*>(s_bias) : nullptr;
    ep.ms = reinterpret_cast<const float*>(s_ms);
    ep.lut = a.lut ? s_lut : nullptr;
  } else if (a.epi == EPI_F16 && a.bias_h) {
    ep.bias_h = reinterpret_cast<const uint16_t*>(s_bias);
  }
  __syncthreads();  // the k-slice table is complete

  // epilogue data, through registers (written to LDS below, after the
  // start-up loads are issued): no direct-to-LDS load is in flight anywhere
  // in this kernel, so every wait the compiler places is exact
  // (one load site, so no wave waits for one load before issuing the next)
  const uint8_t* epi_src = nullptr;
  uint8_t* epi_dst = nullptr;
  if constexpr (ESZ == 1) {
    if (a.epi == EPI_QU8) {
      if (wave == 0 && a.bias_i && lane < nvalid / 4) {
        epi_src = reinterpret_cast<const uint8_t*>(a.bias_i + c0 + lane * 4);
        epi_dst = s_bias + lane * 16;
      } else if (wave == 1 && lane < nvalid / 4) {
        epi_src = reinterpret_cast<const uint8_t*>(a.mscale + c0 + lane * 4);
        epi_dst = s_ms + lane * 16;
      } else if (wave == 2 && a.lut && lane < 16) {
        epi_src = tile_lut(a, c0) + lane * 16;
        epi_dst = s_lut + lane * 16;
      }
    }
  } else {
    if (a.epi == EPI_F16 && a.bias_h && wave == 0 && lane < nvalid / 2) {
      epi_src = reinterpret_cast<const uint8_t*>(a.bias_h + c0 + lane * 2);
      epi_dst = s_bias + lane * 4;
    }
  }
  uint4 epi_v = make_uint4(0, 0, 0, 0);
  if (epi_src) {
    if constexpr (ESZ == 1)
      epi_v = *reinterpret_cast<const uint4*>(epi_src);
    else
      epi_v.x = *reinterpret_cast<const uint32_t*>(epi_src);
  }

  // ---- weights: this wave's fragments cb = wave + 4 i (i < NWV) of k-step
  // k, lane l holding bytes [16 l, 16 l + 16) of each.  Every wave issues
  // exactly NWV loads and NWV writes per k-step, on every path, so the
  // compiler's load and LDS counts are the same for all waves and k-steps: a
  // fragment past the channel tile (cb >= CB) reloads the wave's first
  // fragment, and its write, like every write of a k-step past the end of
  // K, goes to the wave's 1 KB of scratch.
  const int frag_lane = ((lane & 15) * 64 + (lane >> 4) * 16);
  const bool wv = wave < CB;  // the wave has fragment wave + 4 * 0
  const uint8_t* const wsrc = WPK + (size_t)(c0 + (wv ? wave : 0) * 16) * 64 + frag_lane;
  const size_t wstep = (size_t)COUTP * 64;  // bytes per k-step of the packed weights
  uint8_t* const w_scratch = s_ring + NW * (CB * 1024) + wave * 1024 + lane * 16;
  u32x4 wq[LW][NWV];
#define DW_LOAD_W(k_, slot_)                                                                     \
  {                                                                                              \
    const int kk_ = min((k_), KSTEPS - 1);                                                       \
    _Pragma("unroll") for (int i_ = 0; i_ < NWV; ++i_) {                                         \
      const int io_ = wave + 4 * i_ < CB ? i_ * 4096 : 0;                                        \
      wq[slot_][i_] = *reinterpret_cast<const u32x4*>(wsrc + (size_t)kk_ * wstep + io_);         \
    }                                                                                            \
  }
#define DW_STORE_W(k_, slot_)                                                                    \
  {                                                                                              \
    const int k__ = (k_);                                                                        \
    uint8_t* const dst_ = s_ring + (k__ % NW) * (CB * 1024) + wave * 1024 + lane * 16;           \
    _Pragma("unroll") for (int i_ = 0; i_ < NWV; ++i_) {                                         \
      const bool real_ = k__ < KSTEPS && wave + 4 * i_ < CB;                                     \
      *reinterpret_cast<u32x4*>(real_ ? dst_ + i_ * 4096 : w_scratch) = wq[slot_][i_];           \
    }                                                                                            \
  }

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

  // ---- start-up: weights of k-steps 0 .. LW - 1, im2col k-steps 0 .. PD - 2
#pragma unroll
  for (int k = 0; k < LW; ++k) DW_LOAD_W(k, k);
  u32x4 bq[PD][PB];
  uint32_t bkey[PD][PB];
#pragma unroll
  for (int r = 0; r < PD - 1; ++r) DW_LOAD_B(my_tab[r * 4], bq[r], bkey[r]);
  int2 tnext = my_tab[(PD - 1) * 4];
  if (epi_dst) {
    if constexpr (ESZ == 1)
      *reinterpret_cast<uint4*>(epi_dst) = epi_v;
    else
      *reinterpret_cast<uint32_t*>(epi_dst) = epi_v.x;
  }
  DW_STORE_W(0, 0);
  DW_STORE_W(1, 1);
  // this wave's LDS writes (epilogue data, k-steps 0 and 1) are done; then
  // everyone's
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

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

  // weight fragments of k-step s in afr[s & 1], read one k-step ahead
  const uint8_t* const a_lane = s_ring + lane * 16;
  v4i afr[2][CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) afr[0][cb] = *reinterpret_cast<const v4i*>(a_lane + cb * 1024);

  // The loop is unrolled over max(PD, LW) k-steps so that every ring index
  // is a compile-time constant.  Loads are issued on every unrolled k-step,
  // also past the end of K (clamped weight rows, out-of-range im2col), so
  // the compiler's load counts are the same on every path.
  constexpr int UN = PD > LW ? PD : LW;
  static_assert(UN % 2 == 0 && UN % PD == 0 && UN % LW == 0, "unroll");
  for (int s0 = 0; s0 < KSTEPS; s0 += UN) {
#pragma unroll
    for (int r = 0; r < UN; ++r) {
      const int s = s0 + r;
      if (s < KSTEPS) {
        // k-step s + 1's weights are in LDS for everyone (written at k-step
        // s - 1); k-step s - 2's fragments are read by everyone
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes and reads
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
      }
      DW_STORE_W(s + 2, (r + 2) % LW);
      DW_LOAD_W(s + LW, r % LW);
      DW_LOAD_B(tnext, bq[(r + PD - 1) % PD], bkey[(r + PD - 1) % PD]);
      // (entries past the end of K all read as padding)
      tnext = my_tab[min(s + PD, KSTEPS + 2 * PD - 1) * 4];
      if (s < KSTEPS) {
        u32x4 bcur[PB];
#pragma unroll
        for (int pb = 0; pb < PB; ++pb) {
          if constexpr (ESZ == 1)
            bcur[pb] = bq[r % PD][pb] ^ bkey[r % PD][pb];
          else
            bcur[pb] = bq[r % PD][pb];  // f16 padding is +0, what the out-of-range load returns
        }
        // the next k-step's slot (past the end of K: a stale slot, read and
        // never used)
        const uint8_t* const nslot = a_lane + ((s + 1) % NW) * (CB * 1024);
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          afr[(r + 1) & 1][cb] = *reinterpret_cast<const v4i*>(nslot + cb * 1024);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, PB, 0);
#pragma unroll
          for (int pb = 0; pb < PB; ++pb) {
            if constexpr (ESZ == 1) {
              acc[cb][pb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(afr[r & 1][cb], __builtin_bit_cast(v4i, bcur[pb]),
                                                                  acc[cb][pb], 0, 0, 0);
            } else {
              acc[cb][pb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, afr[r & 1][cb]),
                                                                   __builtin_bit_cast(v8h, bcur[pb]), acc[cb][pb],
                                                                   0, 0, 0);
            }
          }
        }
      }
    }
  }
#undef DW_LOAD_W
#undef DW_STORE_W
#undef DW_LOAD_B

  // int8 epilogue: the weight ring's LDS, once every wave is done with it,
  // regroups the results
  uint8_t* xp = nullptr;
  if constexpr (FAST && BC >= 32) {
    static_assert(NW * BC * 64 >= xpose_bytes(BC), "regroup area");
    __syncthreads();
    xp = s_ring + wave * 16 * xpose_row(BC);
  }
  igemm_store<ESZ, BC, PB, EPV>(a, ep, acc, c0, p0, lane, s_ms, s_lut, xp);
}

template <int ESZ, int BC, int EPV>
bool launch_st_bc(hipStream_t st, const IgemmArgs& a, const TileCfg& t, dim3 grid) {
  const size_t lds = st_lds_bytes(BC, a.ksteps, t.pd);
#define DW_T(PB, PD)                                                                                  \
  if (t.pb == PB && t.pd == PD) {                                                                     \
    hipLaunchKernelGGL((igemm_stream_kernel<ESZ, BC, PB, PD, EPV>), grid, dim3(256), lds, st, a);     \
    return true;                                                                                      \
  }
  DW_T(4, 4)
  DW_T(2, 6)
  DW_T(1, 8)
#undef DW_T
  return false;
}

template <int ESZ, int EPV>
bool launch_st_tiles(hipStream_t st, const IgemmArgs& a, const TileCfg& t) {
  const int wgpix = 64 * t.pb;
  const dim3 grid((unsigned)(((a.m + wgpix - 1) / wgpix) * (a.cout_pad / t.bc)));
  switch (t.bc) {
    case 128: return launch_st_bc<ESZ, 128, EPV>(st, a, t, grid);
    case 96: return launch_st_bc<ESZ, 96, EPV>(st, a, t, grid);
    case 80: return launch_st_bc<ESZ, 80, EPV>(st, a, t, grid);
    case 64: return launch_st_bc<ESZ, 64, EPV>(st, a, t, grid);
    case 48: return launch_st_bc<ESZ, 48, EPV>(st, a, t, grid);
    case 32: return launch_st_bc<ESZ, 32, EPV>(st, a, t, grid);
    case 16: return launch_st_bc<ESZ, 16, EPV>(st, a, t, grid);
  }
  return false;
}

}  // namespace ig
}  // namespace dw
