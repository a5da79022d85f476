// Persistent implicit-GEMM convolution for small K (gfx950), shared by the
// translation units that instantiate it.
//
// When all of K is a few k-steps (1x1 convolutions over up to 256 input
// channels, 3x3 over 16), a workgroup of igemm_kernel spends most of its
// life on fixed costs: the k-slice table, the weight copy to LDS, the
// epilogue parameters, and the wait for its first loads.  Here a workgroup
// pays those once: it keeps the weights of its channel tile in LDS and
// walks a contiguous range of pixel tiles.  The im2col rows of the next
// tile are loaded right after the current tile's MFMAs, so their latency is
// covered by the current tile's epilogue.
//
// Tile geometry, operand layouts and epilogue arithmetic are those of
// igemm_kernel (a wave computes all BC channels of its 16 * PB pixels, one
// k-step is a 64-byte row per pixel), and so are the results: every output
// is the same exact int32 sum (or f32 sum in the same order of k-steps).
// NS is the number of k-steps (exactly a.ksteps).
#pragma once

#include "igemm_kernel.h"

namespace dw {

bool igemm_launch_sk_i8_a(hipStream_t st, const IgemmArgs& a, const TileCfg& t, int epv);  // generic, QU8
bool igemm_launch_sk_i8_b(hipStream_t st, const IgemmArgs& a, const TileCfg& t, int epv);  // LUT variants
bool igemm_launch_sk_f16(hipStream_t st, const IgemmArgs& a, const TileCfg& t);

namespace ig {

// LDS layout: [activation table 256][bias 4 BC][multipliers 4 BC]
// [k-slice table NS * 4 int2][weights NS * BC * 64]
__host__ __device__ constexpr int sk_weights_off(int bc, int ns) { return lds_table_off(bc) + ns * 4 * 8; }
inline size_t sk_lds_bytes(int bc, int ns) { return (size_t)sk_weights_off(bc, ns) + (size_t)ns * bc * 64; }

template <int ESZ, int BC, int PB, int NS, int EPV>
__global__ __launch_bounds__(256) void igemm_sk_kernel(const IgemmArgs a) {
  constexpr int CB = BC / 16;
  constexpr int CE = 16 / ESZ;
  constexpr int WPIX = 16 * PB;
  constexpr int WGPIX = 4 * WPIX;
  constexpr bool FAST = EPV != EPV_GENERIC;
  // Weight fragments: all held in registers when there are at most 8, else
  // read 2 ahead through a ring of 4 (NS * CB is then a multiple of 4, so
  // the ring runs on into the next tile, whose weights are the same).
  constexpr int NF = NS * CB;
  constexpr bool RESIDENT = NF <= 8;
  constexpr int FA = 2, RS = 4;
  using acc_t = typename std::conditional<ESZ == 1, v4i, v4f>::type;
  static_assert(!FAST || ESZ == 1, "specialised epilogues are int8");
  static_assert(RESIDENT || NF % RS == 0, "fragment ring");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int COUTP = a.cout_pad;

  // Logical workgroup number, XCD-aware as in igemm_kernel: consecutive
  // numbers run on one XCD and share a pixel range (one per channel tile).
  const int nwg = gridDim.x;
  const int bid = blockIdx.x;
  const int xcd = bid & 7, idx = bid >> 3;
  const int base = nwg >> 3, rem = nwg & 7;
  const int lw = xcd * base + min(xcd, rem) + idx;
  const int ctiles = COUTP / BC;
  const int gp = lw / ctiles;
  const int c0 = (lw - gp * ctiles) * BC;
  const int ptiles = (a.m + WGPIX - 1) / WGPIX;
  int pt = gp * a.tile_tpw;
  const int pt_end = min(pt + a.tile_tpw, ptiles);
  if (pt >= pt_end) return;  // the whole workgroup leaves; no barrier waits for it

  uint8_t* const s_lut = smem;
  uint8_t* const s_bias = smem + 256;
  uint8_t* const s_ms = smem + 256 + 4 * BC;
  int2* const ktab = reinterpret_cast<int2*>(smem + lds_table_off(BC));
  uint8_t* const s_w = smem + sk_weights_off(BC, NS);

  build_ktab(ktab, NS * 4, CE, a, tid);
  int p0 = pt * WGPIX + wave * WPIX;
  int pbase[PB];
  uint32_t tmask[PB];
  pixel_setup<PB>(a, p0, lane, true, pbase, tmask);

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

  const __amdgpu_buffer_rsrc_t xrsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, a.x_bytes, 0x00020000);
  const int2* my_tab = ktab + (lane >> 4);
  // All NS k-steps of the tile, PB loads each, always issued (padding taps
  // and pixels past the end use an out-of-range offset: no memory access),
  // so the compiler's load counters stay exact.
  u32x4 bq[NS][PB];
  uint32_t bkey[NS][PB];  // xor key: u8 -> s8 for in-image taps, the pad value for padding
#define DW_SK_LOADS()                                                                                 \
  _Pragma("unroll") for (int s = 0; s < NS; ++s) {                                                    \
    const int2 t_ = my_tab[s * 4];                                                                    \
    _Pragma("unroll") for (int pb = 0; pb < PB; ++pb) {                                               \
      const bool ok = (tmask[pb] >> t_.y) & 1u;                                                       \
      const int off = ok ? (pbase[pb] + t_.x) * ESZ : (int)0x80000000;                                \
      bq[s][pb] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrsrc, off, 0, 0)); \
      bkey[s][pb] = ok ? a.xxor : a.xpad;                                                             \
    }                                                                                                 \
  }
  DW_SK_LOADS();

  // Weights of the channel tile (NS * CB fragments of 1 KB, in fragment
  // order) and the epilogue parameters, with direct global->LDS loads.
  {
    const int frag_lane = ((lane & 15) * 64 + (lane >> 4) * 16);
    for (int f = wave; f < NS * CB; f += 4) {
      const int sl = f / CB, cb = f - (f / CB) * CB;
      const uint8_t* src = a.wpk + (((uint32_t)sl * COUTP + c0 + cb * 16) * 64u + frag_lane);
      __builtin_amdgcn_global_load_lds((const void*)src, (__attribute__((address_space(3))) void*)(s_w + f * 1024),
                                       16, 0, 0);
    }
  }
  if (a.epi == EPI_QU8) {
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
    if (wave == 0 && lane < nvalid / 2)
      __builtin_amdgcn_global_load_lds((const void*)(a.bias_h + c0 + lane * 2),
                                       (__attribute__((address_space(3))) void*)s_bias, 4, 0, 0);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // Per-channel constants of this lane's channels c0 + cb*16 + cq .. +3.
  const int cq = 4 * (lane >> 4);
  acc_t init[CB];
  float4 msr[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    init[cb] = acc_t{0, 0, 0, 0};
    if constexpr (FAST) {
      if (a.bias_i) init[cb] = *reinterpret_cast<const v4i*>(s_bias + 4 * (cb * 16 + cq));
      msr[cb] = *reinterpret_cast<const float4*>(s_ms + 4 * (cb * 16 + cq));
    }
  }
  const bool full = c0 + BC <= a.cout;
  const __amdgpu_buffer_rsrc_t yrsrc = __builtin_amdgcn_make_buffer_rsrc(a.y, (short)0, a.y_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rrsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.res, (short)0, a.r_bytes, 0x00020000);

  // Weight fragment j = k-step * CB + cb sits at s_w + j KB.
  const uint8_t* const w_lane = s_w + lane * 16;
  v4i afr[RESIDENT ? NF : RS];
#pragma unroll
  for (int i = 0; i < (RESIDENT ? NF : FA); ++i) afr[i] = *reinterpret_cast<const v4i*>(w_lane + i * 1024);

  for (;;) {
    acc_t acc[CB][PB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) acc[cb][pb] = init[cb];

#pragma unroll
    for (int s = 0; s < NS; ++s) {
      u32x4 bcur[PB];
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) {
        if constexpr (ESZ == 1)
          bcur[pb] = bq[s][pb] ^ bkey[s][pb];
        else
          bcur[pb] = bq[s][pb];  // f16 padding is +0, what the out-of-range load returns
      }
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int j = s * CB + cb;
        v4i af;
        if constexpr (RESIDENT) {
          af = afr[j];
        } else {
          af = afr[j % RS];
          afr[(j + FA) % RS] = *reinterpret_cast<const v4i*>(w_lane + ((j + FA) % NF) * 1024);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // this read, then the MFMAs
          __builtin_amdgcn_sched_group_barrier(0x008, PB, 0);
        }
#pragma unroll
        for (int pb = 0; pb < PB; ++pb) {
          if constexpr (ESZ == 1) {
            acc[cb][pb] =
                __builtin_amdgcn_mfma_i32_16x16x64_i8(af, __builtin_bit_cast(v4i, bcur[pb]), acc[cb][pb], 0, 0, 0);
          } else {
            acc[cb][pb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                __builtin_bit_cast(v8h, af), __builtin_bit_cast(v8h, bcur[pb]), acc[cb][pb], 0, 0, 0);
          }
        }
      }
    }

    const int pc = p0;  // this tile's first pixel (of the wave)
    ++pt;
    const bool more = pt < pt_end;
    p0 = pt * WGPIX + wave * WPIX;

    // Residual rows of this tile, ahead of the next tile's loads.
    uint32_t rres[CB][PB];
    if constexpr (EPV == EPV_QU8_LUT_RES) {
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) {
        const int p = pc + pb * 16 + (lane & 15);
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          const bool v = p < a.m && (full || c0 + cb * 16 + cq < a.cout);
          const int off = v ? p * a.r_pix_stride + a.r_c_off + c0 + cb * 16 + cq : (int)0x80000000;
          rres[cb][pb] = __builtin_amdgcn_raw_buffer_load_b32(rrsrc, off, 0, 0);
        }
      }
    }

    // The next tile's pixels and im2col rows (out of range after the last).
    pixel_setup<PB>(a, p0, lane, more, pbase, tmask);
    DW_SK_LOADS();

    // Epilogue of this tile.
    if constexpr (FAST) {
      const int qbase = 0x4B400000 - a.y_zp;
      const float qlo = 12582912.0f - (float)a.y_zp, qhi = qlo + 255.0f;
      const __attribute__((address_space(3))) uint8_t* lut3 = (const __attribute__((address_space(3))) uint8_t*)s_lut;
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) {
        const int p = pc + pb * 16 + (lane & 15);
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
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
            if constexpr (EPV == EPV_QU8_LUT_RES) qi = qadd_u8(qi, (rres[cb][pb] >> (8 * r)) & 0xff, a);
            out |= (uint32_t)qi << (8 * r);
          }
          const bool v = p < a.m && (full || c0 + cb * 16 + cq < a.cout);
          const int off = v ? p * a.y_pix_stride + a.y_c_off + c0 + cb * 16 + cq : (int)0x80000000;
          __builtin_amdgcn_raw_buffer_store_b32(out, yrsrc, off, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int ch = c0 + cb * 16 + cq;
        if (ch >= a.cout) continue;
#pragma unroll
        for (int pb = 0; pb < PB; ++pb) {
          const int p = pc + pb * 16 + (lane & 15);
          if (p < a.m) epilogue4<ESZ>(a, ep, acc[cb][pb], ch, ch - c0, p);
        }
      }
    }
    if (!more) break;
  }
#undef DW_SK_LOADS
}

// Launch of the persistent instantiation for a tile (the caller checked the
// shape: bc in {128, 64, 32, 16}, pb in {2, 4}, 1 <= ksteps <= 4).
template <int ESZ, int BC, int EPV>
bool launch_sk_bc(hipStream_t st, const IgemmArgs& a, const TileCfg& t, dim3 grid) {
  const size_t lds = sk_lds_bytes(t.bc, a.ksteps);
#define DW_T(PB, NS)                                                                           \
  if (t.pb == PB && a.ksteps == NS) {                                                          \
    hipLaunchKernelGGL((igemm_sk_kernel<ESZ, BC, PB, NS, EPV>), grid, dim3(256), lds, st, a);  \
    return true;                                                                               \
  }
  DW_T(4, 1)
  DW_T(4, 2)
  DW_T(4, 3)
  DW_T(4, 4)
  DW_T(2, 1)
  DW_T(2, 2)
  DW_T(2, 3)
  DW_T(2, 4)
#undef DW_T
  return false;
}

template <int ESZ, int EPV>
bool launch_sk_tiles(hipStream_t st, const IgemmArgs& a, const TileCfg& t) {
  const int wgpix = 64 * t.pb;
  const int ptiles = (a.m + wgpix - 1) / wgpix;
  const dim3 grid((unsigned)(((ptiles + t.tpw - 1) / t.tpw) * (a.cout_pad / t.bc)));
  switch (t.bc) {
    case 128: return launch_sk_bc<ESZ, 128, EPV>(st, a, t, grid);
    case 64: return launch_sk_bc<ESZ, 64, EPV>(st, a, t, grid);
    case 32: return launch_sk_bc<ESZ, 32, EPV>(st, a, t, grid);
    case 16: return launch_sk_bc<ESZ, 16, EPV>(st, a, t, grid);
  }
  return false;
}

}  // namespace ig
}  // namespace dw
