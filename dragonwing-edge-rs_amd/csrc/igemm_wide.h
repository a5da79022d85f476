// Wide-tile implicit GEMM (int8, or fp16 with ESZ = 2) for convolutions
// whose input rows are multiples of 128 bytes (c_in % 128 == 0 int8, c_in %
// 64 == 0 fp16): the variant for layers where igemm_kernel is bound by its
// im2col loads.  A k-step is 64 bytes of K either way (v_mfma_i32_16x16x64_i8
// or v_mfma_f32_16x16x32_f16, the same fragment bytes), so the staging and
// the fragment reads below are the element size's only in the MFMA, the
// operand conversion (none for fp16: padding reads as +0) and the epilogue.
//
// igemm_kernel loads each im2col k-step straight into the MFMA registers:
// one wave instruction fetches 64 bytes of 16 pixels, which for c_in >= 128
// (or any strided layer) are half-used 128-byte lines, and the per-CU
// vector-memory path serves those at half the rate of whole lines.  It also
// streams its BC-channel weight slice once per 256-pixel workgroup, so the
// bytes per operation grow as the channel tile shrinks.  Here:
//
//  * a workgroup of 8 waves owns 256 output pixels x BC output channels
//    (BC up to 256, i.e. the whole layer for c_out <= 256): wave w computes
//    64 pixels (w / 2) x BC / 2 channels (w % 2);
//  * K is walked in pairs of k-steps: 128 consecutive input channels of one
//    filter tap.  For each pair the workgroup copies the 256 pixels' 128
//    bytes into LDS with buffer loads that write LDS directly: 8 lanes per
//    pixel, so every wave instruction reads 8 whole lines.  Out-of-image
//    taps use an out-of-range offset, which writes zeros;
//  * the 16-byte chunks of a pixel's row are stored xor-swizzled (chunk c of
//    pixel p in slot c ^ (p & 7)), so the MFMA reads, 16 consecutive pixels
//    x one chunk, hit 8 distinct bank groups per LDS cycle;
//  * the pair's weight fragments (2 k-steps x BC channels, fragment order)
//    arrive the same way; both go to double buffers, so the next pair's
//    loads are in flight while this pair's MFMAs run, with one barrier per
//    pair.  The last two MFMA groups of a pair run after that barrier, from
//    registers, to cover the latency of the next pair's first LDS reads;
//  * LDS carries 128 bytes per cycle per CU; a pair costs 8 waves x 24 KB
//    of fragment reads plus 64 KB of copies against 2 x 64 MFMAs per SIMD
//    (2048 cycles), so the loop is bound by LDS as much as by the MFMAs;
//  * the u8 -> s8 xor (or the padding pattern) is applied to the operands
//    read from LDS, per pixel and tap, as in igemm_kernel; the epilogues are
//    igemm_kernel's.
// Integer sums do not depend on the order of K, so the results are those of
// every other tile shape.
#pragma once

#include "igemm_kernel.h"

namespace dw {

bool igemm_launch_wide_i8_a(hipStream_t st, const IgemmArgs& a, const TileCfg& t, int epv);  // generic, QU8
bool igemm_launch_wide_i8_b(hipStream_t st, const IgemmArgs& a, const TileCfg& t, int epv);  // LUT variants
bool igemm_launch_wide_f16(hipStream_t st, const IgemmArgs& a, const TileCfg& t);

namespace ig {

constexpr int kWidePix = 256;      // output pixels per workgroup
constexpr int kWideThreads = 512;  // 8 waves

// Static LDS of one instantiation (two im2col stages, two weight stages,
// epilogue data) and the dynamic k-pair table.
__host__ __device__ constexpr int wide_static_lds(int bc) { return 2 * kWidePix * 128 + 2 * (2 * bc * 64) + 256 + 8 * bc; }
inline size_t wide_lds_bytes(int bc, int ksteps) { return (size_t)wide_static_lds(bc) + (size_t)(ksteps / 2 + 1) * 8; }

// Element offset of pixel p's top-left tap (times ESZ: bytes) and the
// in-image bit of every tap (no bits for pixels past the end).
template <int ESZ>
__device__ __forceinline__ void wide_pixel(const IgemmArgs& a, int p, int& base, uint32_t& mask) {
  const bool pv = p < a.m;
  const int pp = pv ? p : 0;
  const int hw_o = a.ho * a.wo;
  const int nn = div_small(pp, hw_o, a.r_hwo);
  const int r = pp - nn * hw_o;
  const int oh = div_small(r, a.wo, a.r_wo);
  const int ow = r - oh * a.wo;
  const int ih0 = oh * a.sh - a.pt, iw0 = ow * a.sw - a.pl;
  base = (((nn * a.h + ih0) * a.w + iw0) * a.x_pix_stride + a.x_c_off) * ESZ;
  const int rlo = max(0, -ih0), rhi = min(a.kh, a.h - ih0);
  const int clo = max(0, -iw0), chi = min(a.kw, a.w - iw0);
  const uint32_t cols = chi > clo ? (1u << chi) - (1u << clo) : 0u;
  uint32_t m = 0;
  for (int kh = 0; kh < a.kh; ++kh) m |= (kh >= rlo && kh < rhi) ? cols << (kh * a.kw) : 0u;
  mask = pv ? m : 0u;
}

template <int ESZ, int BC, int EPV>
__global__ __launch_bounds__(kWideThreads) void igemm_wide_kernel(const IgemmArgs a) {
  using acc_t = typename std::conditional<ESZ == 1, v4i, v4f>::type;
  static_assert(ESZ == 1 || EPV == EPV_GENERIC, "specialised epilogues are int8");
  constexpr int CBT = BC / 16;  // 16-channel blocks of the tile
  constexpr int CB = CBT / 2;   // per wave
  constexpr int PB = 4;         // 16-pixel blocks per wave
  constexpr int HC = BC / 2;    // channels per wave
  constexpr bool FAST = EPV != EPV_GENERIC;
  constexpr int WPAIR = 2 * CBT * 1024;
  static_assert(BC == 256 || BC == 128 || BC == 64, "wide tile");
  __shared__ __attribute__((aligned(16))) uint8_t s_x0[kWidePix * 128];
  __shared__ __attribute__((aligned(16))) uint8_t s_x1[kWidePix * 128];
  __shared__ __attribute__((aligned(16))) uint8_t s_w0[WPAIR];
  __shared__ __attribute__((aligned(16))) uint8_t s_w1[WPAIR];
  __shared__ __attribute__((aligned(16))) uint8_t s_epi[256 + 8 * BC];
  extern __shared__ __attribute__((aligned(16))) int2 ktab[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int NP = a.ksteps / 2;

  // XCD-aware tile order, as igemm_kernel
  const int nwg = gridDim.x;
  const int bid = blockIdx.x;
  const int xcd = bid & 7, idx = bid >> 3;
  const int base = nwg >> 3, rem = nwg & 7;
  const int tile = xcd * base + min(xcd, rem) + idx;
  const int ctiles = a.cout_pad / BC;
  const int ptile = tile / ctiles;
  const int c0 = (tile - ptile * ctiles) * BC;
  const int tp0 = ptile * kWidePix;
  const int chh = wave & 1, pq = wave >> 1;

  uint8_t* const s_lut = s_epi;
  uint8_t* const s_bias = s_epi + 256;
  uint8_t* const s_ms = s_epi + 256 + 4 * BC;

  // ---- the pixels this thread loads (i * 64 + tid / 8, chunk slot tid % 8)
  int lbase[4];
  uint32_t lmask[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) wide_pixel<ESZ>(a, tp0 + i * 64 + (tid >> 3), lbase[i], lmask[i]);
  const int lchunk = (tid & 7) ^ ((tid >> 3) & 7);  // chunk this lane loads into slot tid % 8
  // ---- this lane's MFMA pixels: in-image bits (tp0 + pq * 64 + pb * 16 + lane % 16)
  int mbase[PB];
  uint32_t mmask[PB];
  pixel_setup<PB>(a, tp0 + pq * 64, lane, true, mbase, mmask);

  const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, a.x_bytes, 0x00020000);
  const int frag_lane = ((lane & 15) * 64 + (lane >> 4) * 16);
  // pair q's im2col rows and weight fragments (t: its ktab entry), straight
  // into LDS
  auto issue_t = [&](int q, int2 t, uint8_t* sx, uint8_t* sw) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool ok = (lmask[i] >> t.y) & 1u;
      const int off = ok ? lbase[i] + t.x + lchunk * 16 : (int)0x80000000;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xrsrc, (__attribute__((address_space(3))) void*)(sx + (i * 64 + wave * 8) * 128), 16, off, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < (2 * CBT + 7) / 8; ++j) {
      const int f = wave + 8 * j;
      if (f < 2 * CBT) {
        const int ks = f / CBT, cb = f - (f / CBT) * CBT;
        const uint8_t* src = a.wpk + (((uint32_t)(2 * q + ks) * a.cout_pad + c0 + cb * 16) * 64u + frag_lane);
        __builtin_amdgcn_global_load_lds((const void*)src, (__attribute__((address_space(3))) void*)(sw + f * 1024),
                                         16, 0, 0);
      }
    }
  };

  auto issue = [&](int q, uint8_t* sx, uint8_t* sw) { issue_t(q, ktab[q], sx, sw); };

  // pair 0 (tap 0, channels 0..127) is in flight while the tables are built
  issue_t(0, make_int2(0, 0), s_x0, s_w0);
  // ---- k-pair table: pair q is 128 bytes (128 / ESZ input channels) of
  // one tap: its byte offset from the pixel's top-left tap, and the tap
  for (int q = tid; q < NP; q += kWideThreads) {
    const int e = q * (128 / ESZ);
    const int tap = div_small(e, a.cin, a.r_cin);
    const int ci = e - tap * a.cin;
    const int kh = div_small(tap, a.kw, a.r_kw);
    const int kw = tap - kh * a.kw;
    ktab[q] = make_int2(((kh * a.w + kw) * a.x_pix_stride + ci) * ESZ, tap);
  }
  // ---- epilogue data of the channel tile
  const int nvalid = min(BC, a.cout - c0);
  if (a.epi == EPI_QU8) {
    if (tid < nvalid) {
      reinterpret_cast<int*>(s_bias)[tid] = a.bias_i ? a.bias_i[c0 + tid] : 0;
      reinterpret_cast<float*>(s_ms)[tid] = a.mscale[c0 + tid];
    }
    if (a.lut && tid < 256) s_lut[tid] = a.lut[tid];
  } else if (a.epi == EPI_F16 && a.bias_h && tid < nvalid) {
    reinterpret_cast<uint16_t*>(s_bias)[tid] = a.bias_h[c0 + tid];
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();  // pair 0, the k-pair table and the epilogue data

  const int cq = 4 * (lane >> 4);
  acc_t acc[CB][PB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    acc_t init = acc_t{0, 0, 0, 0};
    if constexpr (FAST) {
      if (a.bias_i) init = *reinterpret_cast<const v4i*>(s_bias + 4 * (chh * HC + cb * 16 + cq));
    }
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) acc[cb][pb] = init;
  }

  // pair q from stage (sx, sw): two k-steps of CB x PB MFMAs, one group
  // (one weight fragment x PB pixel fragments) at a time.  The pixel
  // fragments and the first two weight fragments are read up front; each
  // later weight fragment two groups ahead of its use.  The last kDefer
  // groups are held back in registers (weight fragments pa, pixel fragments
  // pbf) and run after the barrier, at the start of the next pair, while
  // that pair's first reads are in flight.  sched_barrier keeps the reads
  // where they are placed.
  constexpr int kDefer = 2;
  constexpr int NG = 2 * CB - kDefer;  // groups run within their own pair
  static_assert(kDefer <= CB, "the held-back groups are second k-step groups");
  v4i pa[kDefer];
  u32x4 pbf[PB];
  // one MFMA: weight fragment x pixel fragment (int8 or fp16 operand bytes)
  auto mma = [](const v4i& w, const u32x4& x, const acc_t& c) -> acc_t {
    if constexpr (ESZ == 1)
      return __builtin_amdgcn_mfma_i32_16x16x64_i8(w, __builtin_bit_cast(v4i, x), c, 0, 0, 0);
    else
      return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, w), __builtin_bit_cast(v8h, x), c, 0, 0,
                                                    0);
  };
  auto held_back = [&]() {
#pragma unroll
    for (int d = 0; d < kDefer; ++d)
#pragma unroll
      for (int pb = 0; pb < PB; ++pb)
        acc[CB - kDefer + d][pb] = mma(pa[d], pbf[pb], acc[CB - kDefer + d][pb]);
  };
  auto compute = [&](int q, const uint8_t* sx, const uint8_t* sw, bool pend) {
    const int tap = ktab[q].y;
    const uint8_t* const wl = sw + chh * CB * 1024 + lane * 16;
    u32x4 bf[2][PB];
    v4i ar[3];
    auto read_pix = [&](int h) {
      const int slot = ((4 * h) + (lane >> 4)) ^ (lane & 7);
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) {
        const int pl = pq * 64 + pb * 16 + (lane & 15);
        bf[h][pb] = *reinterpret_cast<const u32x4*>(sx + pl * 128 + slot * 16);
      }
    };
    auto read_w = [&](int i) {  // group i's weight fragment: k-step i / CB, block i % CB
      const int h = i / CB, cb = i - (i / CB) * CB;
      const v4i v = *reinterpret_cast<const v4i*>(wl + (h * CBT + cb) * 1024);
      if (i >= NG)
        pa[i - NG] = v;
      else
        ar[i % 3] = v;
    };
    read_pix(0);
    read_w(0);
    read_w(1);
    read_pix(1);
    __builtin_amdgcn_sched_barrier(0);
    if (pend) held_back();
    __builtin_amdgcn_sched_barrier(0);
    // int8: u8 -> s8 for in-image taps, the padding pattern for the others
    // (fp16 operands are used as they are: padding reads as +0)
    uint32_t key[PB];
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) key[pb] = ((mmask[pb] >> tap) & 1u) ? a.xxor : a.xpad;
    if constexpr (ESZ == 1) {
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) bf[0][pb] ^= key[pb];
    }
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const int h = i / CB, cb = i - (i / CB) * CB;
      if (i + 2 < 2 * CB) read_w(i + 2);
      __builtin_amdgcn_sched_barrier(0);
      if (ESZ == 1 && i == CB) {
#pragma unroll
        for (int pb = 0; pb < PB; ++pb) bf[1][pb] ^= key[pb];
      }
      const v4i af = ar[i % 3];
#pragma unroll
      for (int pb = 0; pb < PB; ++pb)
        acc[cb][pb] = mma(af, bf[h][pb], acc[cb][pb]);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (ESZ == 1 && NG <= CB) {
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) bf[1][pb] ^= key[pb];
    }
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) pbf[pb] = bf[1][pb];
  };

  // the waitcnt also covers this pair's LDS reads (pa, pbf included), so the
  // stage may be overwritten after the barrier
  for (int q = 0; q < NP; q += 2) {
    if (q + 1 < NP) issue(q + 1, s_x1, s_w1);
    compute(q, s_x0, s_w0, q > 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (q + 1 < NP) {
      if (q + 2 < NP) issue(q + 2, s_x0, s_w0);
      compute(q + 1, s_x1, s_w1, true);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
  }
  held_back();

  // epilogue: this wave's 64 pixels x HC channels; the first im2col stage
  // regroups the u8 results (every wave is past its last read of it)
  EpiLds ep{nullptr, nullptr, nullptr, nullptr};
  if (a.epi == EPI_QU8) {
    ep.bias = a.bias_i ? reinterpret_cast<const int*>(s_bias) + chh * HC : nullptr;
    ep.ms = reinterpret_cast<const float*>(s_ms) + chh * HC;
    ep.lut = a.lut ? s_lut : nullptr;
  } else if (a.epi == EPI_F16 && a.bias_h) {
    ep.bias_h = reinterpret_cast<const uint16_t*>(s_bias) + chh * HC;
  }
  uint8_t* xp = nullptr;
  if constexpr (FAST && HC >= 32) xp = s_x0 + wave * 16 * xpose_row(HC);
  igemm_store<ESZ, HC, PB, EPV>(a, ep, acc, c0 + chh * HC, tp0 + pq * 64, lane, s_ms + 4 * chh * HC, s_lut, xp);
}

template <int ESZ, int EPV>
bool launch_wide_tiles(hipStream_t st, const IgemmArgs& a, const TileCfg& t) {
  const dim3 grid((unsigned)(((a.m + kWidePix - 1) / kWidePix) * (a.cout_pad / t.bc)));
  const size_t dyn = (size_t)(a.ksteps / 2 + 1) * 8;
#define DW_B(BC_)                                                                                   \
  case BC_:                                                                                         \
    hipLaunchKernelGGL((igemm_wide_kernel<ESZ, BC_, EPV>), grid, dim3(kWideThreads), dyn, st, a); \
    return true;
  switch (t.bc) {
    DW_B(256)
    DW_B(128)
    DW_B(64)
  }
#undef DW_B
  return false;
}

}  // namespace ig
}  // namespace dw
