// A whole int8 C2f block with one bottleneck in one launch:
//   y = cv1(x) (1x1, c1 -> 2c), y0, y1 = split(y),
//   t = m.cv1(y1) (3x3, c -> c), z = m.cv2(t) (3x3, c -> c) [+ y1],
//   out = cv2(concat(y0, y1, z)) (1x1, 3c -> c2),
// every conv a QLinearConv with its SiLU table, the shortcut a QLinearAdd.
// In separate launches y, t and z go through HBM and four launches pay
// their fixed costs; here only x is read and only out is written.
//
// A workgroup of 16 waves owns R whole rows of one image (R tuned, a
// divisor of the height).  LDS holds all four weight sets and epilogue blocks and
// three tiles:
//  * Y1: y1 over rows r0 - 2 .. r0 + R + 1 with a one-pixel column halo, in
//    the operand form of m.cv1 (u8 xor 0x80; columns beside the image and
//    rows outside it hold its padding pattern), the pair kernel's input tile;
//  * T: t over rows r0 - 1 .. r0 + R, the same way for m.cv2;
//  * Y0: y0 over the R rows, in cv2's operand form.
// Phase 0 computes cv1 over the in-image rows of Y1's range (operands
// straight from x, as igemm_kernel loads them) and writes y0 / y1; phases 1
// and 2 are the pair kernel's (its halo rows computed twice, once by each
// neighbouring band).  Phase 2's epilogue regroups each 16-pixel block's z
// in the wave's own LDS rows, and cv2 runs on that block at once: its
// operand is read from Y0, Y1's centre and those rows, its weight
// fragments from LDS.
//
// Every conv's arithmetic is igemm_kernel's (bias' as the accumulator's
// start, requant_bits, the table, qadd_u8) over the same integer sums, so
// the output is the separate launches'.
#pragma once

#include "igemm_kernel.h"

namespace dw {
namespace ig {

struct C2fArgs {
  IgemmArgs a0, a1, a2, a3;  // cv1, m.cv1, m.cv2 (+ y1), cv2
  int rows;
};

constexpr int kC2fWaves = 16;
constexpr int kC2fThreads = 64 * kC2fWaves;

// LDS pixel stride of the 3x3 tiles in 16-byte units (the pair kernel's)
__host__ __device__ constexpr int c2f_su(int c) { return c == 32 ? 2 : (c / 16) | 1; }
// z regroup row of one pixel: c bytes and a 16-byte pad
__host__ __device__ constexpr int c2f_zrow(int c) { return c + 16; }

// LDS layout (bytes): the four epilogue blocks [table 256][bias' 4 cout]
// [multipliers 4 cout], the 3x3 k-slice table, the four weight sets
// (fragment order), Y1, T, Y0, the 8 waves' z rows.
struct C2fLayout {
  int epi[4], tab, w[4], y1, t, y0, zr, rt, total;
};
__host__ __device__ inline C2fLayout c2f_layout(int c, int c2, int ks0, int ks1, int ks3, int w, int rows) {
  C2fLayout L{};
  const int couts[4] = {2 * c, c, c, c2};
  const int kss[4] = {ks0, ks1, ks1, ks3};
  int off = 0;
  for (int i = 0; i < 4; ++i) {
    L.epi[i] = off;
    off += 256 + 8 * couts[i];
  }
  L.tab = off;
  off = (off + ks1 * 16 + 15) / 16 * 16;
  for (int i = 0; i < 4; ++i) {
    L.w[i] = off;
    off += kss[i] * couts[i] * 64;
  }
  const int su = c2f_su(c), tw = w + 2;
  L.y1 = off;
  off += (rows + 4) * tw * su * 16;
  L.t = off;
  off += (rows + 2) * tw * su * 16;
  L.y0 = off;
  off += rows * w * c;
  L.zr = off;
  off += kC2fWaves * 16 * c2f_zrow(c);
  L.rt = off;  // m.cv2's QLinearAdd tables (IgemmArgs::rtab, 2 KB)
  off += 2048;
  L.total = off;
  return L;
}

// 16-pixel blocks a wave takes at a time in each phase: within 128 VGPRs, so
// that 16 waves (four a SIMD) hide each other's LDS and table latencies in
// the VALU-bound epilogues (b2's block: 55.9 us with 8 waves, 47.9 with 12,
// 44.3 with 16)
__host__ __device__ constexpr int c2f_pbc0(int cb, int ks0) { return cb == 1 ? (ks0 == 1 ? 4 : 3) : 2; }
__host__ __device__ constexpr int c2f_pbc(int cb) { return cb == 1 ? 5 : 3; }

// CB: c / 16 (1 or 2); CBD: c2 / 16 (2 CB: c2 = 2c); KS0: cv1's k-steps
// (c1 / 64 rounded up); RES: the bottleneck's shortcut.
template <int CB, int CBD, int KS0, bool RES>
__global__ __launch_bounds__(kC2fThreads) void igemm_c2f_kernel(const C2fArgs p) {
  constexpr int C = CB * 16;
  constexpr int CBA = 2 * CB;  // cv1's output blocks
  constexpr int PBC0 = c2f_pbc0(CB, KS0);
  constexpr int PBC = c2f_pbc(CB);
  constexpr int CU = C / 16;
  constexpr int SU = c2f_su(C);
  constexpr int ZROW = c2f_zrow(C);
  constexpr int KD = (3 * C + 63) / 64;  // cv2's k-steps
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const IgemmArgs& a0 = p.a0;
  const IgemmArgs& a1 = p.a1;
  const IgemmArgs& a2 = p.a2;
  const IgemmArgs& a3 = p.a3;
  const int W = a1.w, H = a1.h, R = p.rows;
  const int TW = W + 2;
  const int KS1 = a1.ksteps;

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

  const C2fLayout L = c2f_layout(C, CBD * 16, KS0, KS1, KD, W, R);
  int* const s_tab = reinterpret_cast<int*>(smem + L.tab);
  uint8_t* const s_y1 = smem + L.y1;
  uint8_t* const s_t = smem + L.t;
  uint8_t* const s_y0 = smem + L.y0;

  // ---- the four weight sets (fragment order) and epilogue blocks, direct to LDS
  const int frag_lane = ((lane & 15) * 64 + (lane >> 4) * 16);
  auto load_weights = [&](const IgemmArgs& a, int cbs, int kss, uint8_t* dst) {
    const int nfr = kss * cbs;
    for (int f = wave; f < nfr; f += kC2fWaves) {
      const int sl = f / cbs, cb = f - sl * cbs;
      const uint8_t* src = a.wpk + (((uint32_t)sl * a.cout_pad + cb * 16) * 64u + frag_lane);
      __builtin_amdgcn_global_load_lds((const void*)src, (__attribute__((address_space(3))) void*)(dst + f * 1024), 16,
                                       0, 0);
    }
  };
  load_weights(a0, CBA, KS0, smem + L.w[0]);
  load_weights(a1, CB, KS1, smem + L.w[1]);
  load_weights(a2, CB, KS1, smem + L.w[2]);
  load_weights(a3, CBD, KD, smem + L.w[3]);
  // epilogue blocks: waves 0 .. 3 conv w's bias' and multipliers, waves
  // 4 .. 7 conv w - 4's table; each load from lane 0 up (an LDS-destination
  // load puts lane i's 16 bytes 16 i bytes past its destination)
  auto load_bm = [&](const IgemmArgs& a, uint8_t* e) {
    if (lane < a.cout / 4) {
      __builtin_amdgcn_global_load_lds((const void*)(a.bias_i + lane * 4), (__attribute__((address_space(3))) void*)(e + 256),
                                       16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(a.mscale + lane * 4),
                                       (__attribute__((address_space(3))) void*)(e + 256 + 4 * a.cout), 16, 0, 0);
    }
  };
  auto load_lut = [&](const IgemmArgs& a, uint8_t* e) {
    if (lane < 16)
      __builtin_amdgcn_global_load_lds((const void*)(a.lut + lane * 16), (__attribute__((address_space(3))) void*)e, 16,
                                       0, 0);
  };
  if (wave == 0) load_bm(a0, smem + L.epi[0]);
  if (wave == 1) load_bm(a1, smem + L.epi[1]);
  if (wave == 2) load_bm(a2, smem + L.epi[2]);
  if (wave == 3) load_bm(a3, smem + L.epi[3]);
  if (wave == 4) load_lut(a0, smem + L.epi[0]);
  if (wave == 5) load_lut(a1, smem + L.epi[1]);
  if (wave == 6) load_lut(a2, smem + L.epi[2]);
  if (wave == 7) load_lut(a3, smem + L.epi[3]);
  // the QLinearAdd tables: 2 KB, two loads of 64 lanes from lane 0 up
  if (RES && a2.rtab && wave == 8) {
    __builtin_amdgcn_global_load_lds((const void*)(a2.rtab + lane * 4),
                                     (__attribute__((address_space(3))) void*)(smem + L.rt), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((const void*)(a2.rtab + 256 + lane * 4),
                                     (__attribute__((address_space(3))) void*)(smem + L.rt + 1024), 16, 0, 0);
  }

  // ---- the 3x3 convs' k-slice offsets (same tile geometry and channels)
  for (int e = tid; e < KS1 * 4; e += kC2fThreads) {
    const int k = e * 16;
    int off = 0;
    if (k < 9 * C) {
      const int tap = k / C, ci = k - (k / C) * C;
      const int kh = tap / 3, kw = tap - (tap / 3) * 3;
      off = ((kh * TW + kw) * SU + ci / 16) * 16;
    }
    s_tab[e] = off;
  }

  // ---- padding of Y1 and T: the columns beside the image and the rows
  // outside it hold the next conv's padding pattern
  const float r_tw = 1.0f / (float)TW;
  {
    const u32x4 pad1 = u32x4{a1.xpad, a1.xpad, a1.xpad, a1.xpad};
    const u32x4 pad2 = u32x4{a2.xpad, a2.xpad, a2.xpad, a2.xpad};
    const int un1 = (R + 4) * TW * CU, un2 = (R + 2) * TW * CU;
    for (int u = tid; u < un1 + un2; u += kC2fThreads) {
      const bool second = u >= un1;
      const int uu = second ? u - un1 : u;
      const int ip = uu / CU;  // CU is 1 or 2
      const int cu = uu - ip * CU;
      const int tr = div_small(ip, TW, r_tw), tc = ip - tr * TW;
      const int ih = r0 - (second ? 1 : 2) + tr;
      if (tc == 0 || tc == TW - 1 || (unsigned)ih >= (unsigned)H)
        *reinterpret_cast<u32x4*>((second ? s_t : s_y1) + (ip * SU + cu) * 16) = second ? pad2 : pad1;
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const int cq = 4 * (lane >> 4);

  // ================= phase 0: cv1 over the in-image rows of Y1's range
  {
    const uint8_t* const e0 = smem + L.epi[0];
    const int qbase = 0x4B400000 - a0.y_zp;
    const float qlo = 12582912.0f - (float)a0.y_zp, qhi = qlo + 255.0f;
    const __attribute__((address_space(3))) uint8_t* lut3 = (const __attribute__((address_space(3))) uint8_t*)e0;
    const __amdgpu_buffer_rsrc_t xrsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)a0.x, (short)0, a0.x_bytes, 0x00020000);
    const int rlo = max(0, 2 - r0), rhi = min(R + 4, H - r0 + 2);  // Y1 rows inside the image
    const int np = (rhi - rlo) * W;
    const int nb = (np + 15) / 16;
    const uint8_t* const wl = smem + L.w[0] + lane * 16;
    // a chunk's pixels: x offset, and the byte offsets of their y1 in Y1
    // and (rows of the band only) y0 in Y0 (-1: none)
    auto setup = [&](int b0, int (&goff)[PBC0], int (&o1)[PBC0], int (&o0)[PBC0]) {
#pragma unroll
      for (int pb = 0; pb < PBC0; ++pb) {
        const int pl = (b0 + pb) * 16 + (lane & 15);
        const bool v = pl < np;
        const int q = v ? pl : 0;
        const int r = div_small(q, W, a1.r_wo), c = q - r * W;
        const int tr = rlo + r;
        const int ih = r0 - 2 + tr;
        goff[pb] = v ? ((n * H + ih) * W + c) * a0.x_pix_stride + a0.x_c_off : -1;
        o1[pb] = v ? (tr * TW + c + 1) * SU * 16 + cq : -1;
        o0[pb] = (v && (unsigned)(tr - 2) < (unsigned)R) ? ((tr - 2) * W + c) * C + cq : -1;
      }
    };
    // its operand rows: this lane's 16 bytes of every k-step (none past c1
    // or for pixels past the end: out-of-range loads)
    auto issue = [&](const int (&goff)[PBC0], u32x4 (&bq)[KS0][PBC0]) {
#pragma unroll
      for (int q = 0; q < KS0; ++q) {
        const int kb = q * 64 + (lane >> 4) * 16;
#pragma unroll
        for (int pb = 0; pb < PBC0; ++pb) {
          const int off = (goff[pb] >= 0 && kb < a0.cin) ? goff[pb] + kb : (int)0x80000000;
          bq[q][pb] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrsrc, off, 0, 0));
        }
      }
    };
    const int stride = kC2fWaves * PBC0;
    int goff[PBC0], o1[PBC0], o0[PBC0];
    u32x4 bq[KS0][PBC0];
    setup(wave * PBC0, goff, o1, o0);
    issue(goff, bq);
    for (int b0 = wave * PBC0; b0 < nb; b0 += stride) {
      // the next chunk's loads, in flight during this chunk's work
      int goff_n[PBC0], o1_n[PBC0], o0_n[PBC0];
      u32x4 bq_n[KS0][PBC0];
      setup(b0 + stride, goff_n, o1_n, o0_n);
      issue(goff_n, bq_n);
      v4i acc[CBA][PBC0];
#pragma unroll
      for (int cb = 0; cb < CBA; ++cb) {
        const v4i init = *reinterpret_cast<const v4i*>(e0 + 256 + 4 * (cb * 16 + cq));
#pragma unroll
        for (int pb = 0; pb < PBC0; ++pb) acc[cb][pb] = init;
      }
#pragma unroll
      for (int q = 0; q < KS0; ++q) {
        v4i bfr[PBC0];
#pragma unroll
        for (int pb = 0; pb < PBC0; ++pb) bfr[pb] = __builtin_bit_cast(v4i, bq[q][pb] ^ a0.xxor);
#pragma unroll
        for (int cb = 0; cb < CBA; ++cb) {
          const v4i af = *reinterpret_cast<const v4i*>(wl + (q * CBA + cb) * 1024);
#pragma unroll
          for (int pb = 0; pb < PBC0; ++pb)
            acc[cb][pb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bfr[pb], acc[cb][pb], 0, 0, 0);
        }
      }
      // epilogue: requantize, table; y0 (channels < c) to Y0 for the band's
      // own rows, y1 to Y1, each in its consumer's operand form
#pragma unroll
      for (int cb = 0; cb < CBA; ++cb) {
        const float4 m4 = *reinterpret_cast<const float4*>(e0 + 256 + 4 * 2 * C + 4 * (cb * 16 + cq));
        const float ms4[4] = {m4.x, m4.y, m4.z, m4.w};
#pragma unroll
        for (int pb = 0; pb < PBC0; ++pb) {
          const int o = cb < CB ? o0[pb] : o1[pb];  // y0 only for the band's own rows
          if (o < 0) continue;
          uint32_t out = 0;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int qb = requant_bits(acc[cb][pb][r], ms4[r], qlo, qhi);
            out |= (uint32_t)lut3[(uint32_t)qb - (uint32_t)qbase] << (8 * r);
          }
          if (cb < CB)
            *reinterpret_cast<uint32_t*>(s_y0 + o + cb * 16) = out ^ a3.xxor;
          else
            *reinterpret_cast<uint32_t*>(s_y1 + o + (cb - CB) * 16) = out ^ a1.xxor;
        }
      }
#pragma unroll
      for (int pb = 0; pb < PBC0; ++pb) {
        goff[pb] = goff_n[pb];
        o1[pb] = o1_n[pb];
        o0[pb] = o0_n[pb];
#pragma unroll
        for (int q = 0; q < KS0; ++q) bq[q][pb] = bq_n[q][pb];
      }
    }
  }
  __syncthreads();

  const int* const my_tab = s_tab + (lane >> 4);
  // One chunk of PBC blocks of a 3x3 conv, both operands in LDS (the next
  // k-step's fragments read while this one's MFMAs run).
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
    for (int q0 = 0; q0 < KS1; q0 += 2) {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int q = q0 + r;
        if (q < KS1) {
          if (q + 1 < KS1) DW_READ_K(q + 1, (r + 1) & 1);
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

  // ================= phase 1: t over the R + 2 rows of T
  {
    const uint8_t* const e1 = smem + L.epi[1];
    const int np = (R + 2) * W;
    const int nb = (np + 15) / 16;
    const int qbase = 0x4B400000 - a1.y_zp;
    const float qlo = 12582912.0f - (float)a1.y_zp, qhi = qlo + 255.0f;
    const __attribute__((address_space(3))) uint8_t* lut3 = (const __attribute__((address_space(3))) uint8_t*)e1;
    for (int b0 = wave * PBC; b0 < nb; b0 += kC2fWaves * PBC) {
      int pbase[PBC], poff[PBC];
#pragma unroll
      for (int pb = 0; pb < PBC; ++pb) {
        const int pl = (b0 + pb) * 16 + (lane & 15);
        const int q = pl < np ? pl : 0;
        const int r = div_small(q, W, a1.r_wo), c = q - r * W;
        pbase[pb] = (r * TW + c) * SU * 16;  // Y1 rows r .. r + 2 feed T row r
        const int ih = r0 - 1 + r;
        poff[pb] = (pl < np && (unsigned)ih < (unsigned)H) ? ((r * TW + c + 1) * SU * 16 + cq) : -1;
      }
      v4i acc[CB][PBC];
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const v4i init = *reinterpret_cast<const v4i*>(e1 + 256 + 4 * (cb * 16 + cq));
#pragma unroll
        for (int pb = 0; pb < PBC; ++pb) acc[cb][pb] = init;
      }
      chunk_gemm(acc, s_y1, smem + L.w[1] + lane * 16, pbase);
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const float4 m4 = *reinterpret_cast<const float4*>(e1 + 256 + 4 * C + 4 * (cb * 16 + cq));
        const float ms4[4] = {m4.x, m4.y, m4.z, m4.w};
#pragma unroll
        for (int pb = 0; pb < PBC; ++pb) {
          if (poff[pb] < 0) continue;
          uint32_t out = 0;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int qb = requant_bits(acc[cb][pb][r], ms4[r], qlo, qhi);
            out |= (uint32_t)lut3[(uint32_t)qb - (uint32_t)qbase] << (8 * r);
          }
          *reinterpret_cast<uint32_t*>(s_t + poff[pb] + cb * 16) = out ^ a2.xxor;
        }
      }
    }
  }
  __syncthreads();

  // ================= phase 2: z over the R rows, then cv2 block by block
  {
    const uint8_t* const e2 = smem + L.epi[2];
    const uint8_t* const e3 = smem + L.epi[3];
    const int np = R * W;
    const int nb = (np + 15) / 16;
    const int qbase2 = 0x4B400000 - a2.y_zp;
    const float qlo2 = 12582912.0f - (float)a2.y_zp, qhi2 = qlo2 + 255.0f;
    const int qbase3 = 0x4B400000 - a3.y_zp;
    const float qlo3 = 12582912.0f - (float)a3.y_zp, qhi3 = qlo3 + 255.0f;
    const __attribute__((address_space(3))) uint8_t* lut2 = (const __attribute__((address_space(3))) uint8_t*)e2;
    const __attribute__((address_space(3))) uint8_t* lut3 = (const __attribute__((address_space(3))) uint8_t*)e3;
    uint8_t* const zrow = smem + L.zr + (wave * 16 + (lane & 15)) * ZROW;
    const uint8_t* const wdl = smem + L.w[3] + lane * 16;  // cv2's weight fragments
    for (int b0 = wave * PBC; b0 < nb; b0 += kC2fWaves * PBC) {
      // per block: the window in T, the pixel in Y1 and in Y0, the output
      // pixel (-1: none)
      int pbase[PBC], y1c[PBC], y0c[PBC], pix[PBC];
#pragma unroll
      for (int pb = 0; pb < PBC; ++pb) {
        const int pl = (b0 + pb) * 16 + (lane & 15);
        const int q = pl < np ? pl : 0;
        const int r = div_small(q, W, a1.r_wo), c = q - r * W;
        pbase[pb] = (r * TW + c) * SU * 16;
        y1c[pb] = ((r + 2) * TW + c + 1) * SU * 16;
        y0c[pb] = (r * W + c) * C;
        pix[pb] = pl < np ? (n * H + r0 + r) * W + c : -1;
      }
      v4i acc[CB][PBC];
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const v4i init = *reinterpret_cast<const v4i*>(e2 + 256 + 4 * (cb * 16 + cq));
#pragma unroll
        for (int pb = 0; pb < PBC; ++pb) acc[cb][pb] = init;
      }
      chunk_gemm(acc, s_t, smem + L.w[2] + lane * 16, pbase);
#pragma unroll
      for (int pb = 0; pb < PBC; ++pb) {
        if (b0 + pb >= nb) break;  // wave-uniform
        asm volatile("" ::: "memory");  // the previous block's reads of the z rows are issued
        // z: requantize, table, the shortcut's QLinearAdd of y1; to this
        // wave's rows in cv2's operand form
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          const float4 m4 = *reinterpret_cast<const float4*>(e2 + 256 + 4 * C + 4 * (cb * 16 + cq));
          const float ms4[4] = {m4.x, m4.y, m4.z, m4.w};
          uint32_t rres = 0;
          if constexpr (RES) rres = *reinterpret_cast<const uint32_t*>(s_y1 + y1c[pb] + cb * 16 + cq) ^ a1.xxor;
          uint32_t out = 0;
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const int qb = requant_bits(acc[cb][pb][rr], ms4[rr], qlo2, qhi2);
            int qi;
            if (RES && a2.rtab) {
              qi = qadd_u8_tab((lds_f32p)(smem + L.rt), qb - qbase2, (rres >> (8 * rr)) & 0xff, a2.zy);
            } else {
              qi = lut2[(uint32_t)qb - (uint32_t)qbase2];
              if constexpr (RES) qi = qadd_u8(qi, (rres >> (8 * rr)) & 0xff, a2);
            }
            out |= (uint32_t)qi << (8 * rr);
          }
          *reinterpret_cast<uint32_t*>(zrow + cb * 16 + cq) = out ^ a3.xxor;
        }
        asm volatile("" ::: "memory");  // one wave's LDS operations run in order
        // cv2's operand: 16 bytes of concat(y0, y1, z) per lane and k-step,
        // one read from whichever holds them (past 3c: any bytes, their
        // weights are zero)
        v4i xd[KD];
#pragma unroll
        for (int q2 = 0; q2 < KD; ++q2) {
          const int kb = q2 * 64 + (lane >> 4) * 16;
          const uint8_t* src = kb < C ? s_y0 + y0c[pb] + kb
                               : kb < 2 * C ? s_y1 + y1c[pb] + (kb - C)
                                            : zrow + (kb < 3 * C ? kb - 2 * C : 0);
          xd[q2] = *reinterpret_cast<const v4i*>(src);
        }
        const bool pv = pix[pb] >= 0;
        uint8_t* const yrow = (uint8_t*)a3.y + (size_t)(pv ? pix[pb] : 0) * a3.y_pix_stride + a3.y_c_off;
#pragma unroll
        for (int cb = 0; cb < CBD; ++cb) {
          v4i acc2 = *reinterpret_cast<const v4i*>(e3 + 256 + 4 * (cb * 16 + cq));
#pragma unroll
          for (int q2 = 0; q2 < KD; ++q2)
            acc2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(*reinterpret_cast<const v4i*>(wdl + (q2 * CBD + cb) * 1024),
                                                         xd[q2], acc2, 0, 0, 0);
          const float4 m4 = *reinterpret_cast<const float4*>(e3 + 256 + 4 * CBD * 16 + 4 * (cb * 16 + cq));
          const float ms4[4] = {m4.x, m4.y, m4.z, m4.w};
          uint32_t out = 0;
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const int qb = requant_bits(acc2[rr], ms4[rr], qlo3, qhi3);
            out |= (uint32_t)lut3[(uint32_t)qb - (uint32_t)qbase3] << (8 * rr);
          }
          if (pv) *reinterpret_cast<uint32_t*>(yrow + cb * 16 + cq) = out;
        }
      }
    }
  }
}

}  // namespace ig
}  // namespace dw
