// Implicit-GEMM convolution on CDNA4 matrix cores (gfx950).
//
// The convolution is the GEMM  Y[c][p] = sum_k W[k][c] * X[p][k]  with
//   c = output channel, p = output pixel (n, oh, ow), k = (kh, kw, ci).
// Both operands are consumed as 64-byte rows per k-step (64 int8 or 32 fp16
// values): one wavefront instruction is v_mfma_i32_16x16x64_i8 (int8) or
// v_mfma_f32_16x16x32_f16 (fp16), and each lane supplies a 16-byte slice of
// one row of each operand (row = lane % 16, slice = lane / 16).
//
// Data movement, per 256-thread workgroup:
//  * weights (operand A) are pre-packed on the host side into
//    [k-step][c_out][64 B] rows; the workgroup stages them in LDS in chunks
//    of several k-steps (double-buffered, one barrier per chunk) and every
//    wave reads its fragments from there;
//  * im2col rows (operand B) are never staged: each lane loads its 16-byte
//    slice straight from NHWC memory into the MFMA source registers (a
//    16-byte slice is 16 int8 / 8 fp16 consecutive input channels of one
//    filter tap, so c_in * esize must be a multiple of 16), one k-step
//    ahead of use.  Out-of-image taps read the zero-point pattern.
//  * a wave owns 16*PB output pixels and all BC channels of the tile; with
//    KS > 1 the four waves split the k-steps of the same pixels and add
//    their partial sums through LDS at the end (used when the layer has too
//    few pixels to fill 256 CUs).
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
#include "dw_common.h"
#include "dw_device.h"

#include <stdio.h>
#include <stdlib.h>

#include <type_traits>

namespace dw {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// LDS address of 16-byte slice `chunk` (0..3) of 64-byte row `row`, xor
// swizzled so that the 16 rows read by one MFMA fragment spread over banks.
__device__ __forceinline__ int swz(int row, int chunk) {
  return row * 64 + ((chunk ^ ((row >> 1) & 3)) << 4);
}

// f16 epilogue chain of CpuGraphRuntime: conv result rounded to f16, then
// the bias pass, the activation and the residual add, each on stored f16.
__device__ __forceinline__ uint16_t f16_chain(float acc, const uint16_t* bias_h, int ch, int act,
                                              bool has_res, uint16_t resv) {
  uint16_t hb = f2h(acc);
  if (bias_h) hb = f16_add_bits(hb, bias_h[ch]);
  hb = f16_act_bits(hb, act);
  if (has_res) hb = f16_add_bits(hb, resv);
  return hb;
}

// Epilogue for one 16x16 block: this lane holds channels ch..ch+3 of pixel p.
template <int ESZ, typename AccT>
__device__ __forceinline__ void epilogue4(const IgemmArgs& a, const AccT& v, int ch, int p) {
  const size_t yo = (size_t)p * a.y_pix_stride + a.y_c_off + ch;
  if constexpr (ESZ == 1) {
    if (a.epi == EPI_QU8) {
      const int4 bi = a.bias_i ? *reinterpret_cast<const int4*>(a.bias_i + ch) : make_int4(0, 0, 0, 0);
      const float4 ms = *reinterpret_cast<const float4*>(a.mscale + ch);
      uint32_t rres = 0;
      if (a.res)
        rres = *reinterpret_cast<const uint32_t*>((const uint8_t*)a.res + (size_t)p * a.r_pix_stride +
                                                  a.r_c_off + ch);
      const int accs[4] = {v[0] + bi.x, v[1] + bi.y, v[2] + bi.z, v[3] + bi.w};
      const float mss[4] = {ms.x, ms.y, ms.z, ms.w};
      uint32_t out = 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float q = rintf((float)accs[r] * mss[r]) + (float)a.y_zp;
        q = fminf(fmaxf(q, 0.0f), 255.0f);
        int qi = (int)q;
        if (a.lut) qi = a.lut[qi];
        if (a.res) {
          const int rb = (rres >> (8 * r)) & 0xff;
          const float f = (float)(qi - a.za) * a.ra + (float)(rb - a.zb) * a.rb;
          float g = rintf(f) + (float)a.zy;
          g = fminf(fmaxf(g, 0.0f), 255.0f);
          qi = (int)g;
        }
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
    const bool hr = a.res != nullptr;
    const uint32_t lo = (uint32_t)f16_chain(v[0], a.bias_h, ch + 0, a.act, hr, rres.x & 0xffff) |
                        ((uint32_t)f16_chain(v[1], a.bias_h, ch + 1, a.act, hr, rres.x >> 16) << 16);
    const uint32_t hi = (uint32_t)f16_chain(v[2], a.bias_h, ch + 2, a.act, hr, rres.y & 0xffff) |
                        ((uint32_t)f16_chain(v[3], a.bias_h, ch + 3, a.act, hr, rres.y >> 16) << 16);
    *reinterpret_cast<uint2*>((uint16_t*)a.y + yo) = make_uint2(lo, hi);
  }
}

// Number of k-steps per LDS weight chunk (16 KB per buffer).
template <int BC>
constexpr int chunk_steps() {
  return (16384 / (BC * 64)) > 0 ? (16384 / (BC * 64)) : 1;
}

// Bytes of LDS: two weight-chunk buffers, or the split-K partial sums.
template <int BC, int PB, int KS>
constexpr int smem_bytes() {
  return (2 * chunk_steps<BC>() * BC * 64) > ((KS - 1) * (4 / KS) * 64 * (BC / 16) * PB * 16)
             ? (2 * chunk_steps<BC>() * BC * 64)
             : ((KS - 1) * (4 / KS) * 64 * (BC / 16) * PB * 16);
}

template <int ESZ, int BC, int PB, int KS>
__global__ __launch_bounds__(256) void igemm_kernel(const IgemmArgs a) {
  constexpr int CB = BC / 16;       // 16-channel blocks (all channels of the tile per wave)
  constexpr int KE = 64 / ESZ;      // elements per row per k-step
  constexpr int CE = 16 / ESZ;      // elements per 16-byte slice
  constexpr int PG = 4 / KS;        // waves along pixels
  constexpr int WPIX = 16 * PB;     // pixels per wave
  constexpr int WGPIX = PG * WPIX;  // pixels per workgroup
  constexpr int KC = chunk_steps<BC>();
  constexpr int ABYTES = KC * BC * 64;
  constexpr int AQ = ABYTES / 16;         // 16-byte slices per chunk
  constexpr int AREG = (AQ + 255) / 256;  // slices per thread
  using acc_t = typename std::conditional<ESZ == 1, v4i, v4f>::type;
  static_assert(BC % 16 == 0 && (KS == 1 || KS == 2 || KS == 4), "tile");
  __shared__ __attribute__((aligned(16))) uint8_t smem[smem_bytes<BC, PB, KS>()];

  // scalars used in the k loop (kept in SGPRs)
  const uint8_t* __restrict__ X = a.x;
  const uint8_t* __restrict__ WPK = a.wpk;
  const int H = a.h, W = a.w, CIN = a.cin, KH = a.kh, KW = a.kw;
  const int XPS = a.x_pix_stride, XCO = a.x_c_off, KSTEPS = a.ksteps, COUTP = a.cout_pad;
  const uint32_t XXOR = a.xxor;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int pg = wave % PG;
  const int ks = wave / PG;

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
  const int p0 = ptile * WGPIX + pg * WPIX;

  // ---- im2col state of this lane: pixels p0 + pb*16 + (lane & 15), slice lane >> 4
  const int hw_o = a.ho * a.wo;
  int ih0[PB], iw0[PB], nb[PB];
  bool pv[PB];
#pragma unroll
  for (int pb = 0; pb < PB; ++pb) {
    const int p = p0 + pb * 16 + (lane & 15);
    pv[pb] = p < a.m;
    const int pp = pv[pb] ? p : 0;
    const int nn = pp / hw_o;
    const int r = pp - nn * hw_o;
    const int oh = r / a.wo;
    const int ow = r - oh * a.wo;
    ih0[pb] = oh * a.sh - a.pt;
    iw0[pb] = ow * a.sw - a.pl;
    nb[pb] = nn * H;
  }
  int e_c = ks * KE + (lane >> 4) * CE;  // first k-step of this wave is `ks`
  int e_kh = 0, e_kw = 0;
#define DW_NORMALIZE()                      \
  while (e_c >= CIN) {                      \
    e_c -= CIN;                             \
    if (++e_kw == KW) { e_kw = 0; ++e_kh; } \
  }
  DW_NORMALIZE();

  const u32x4 padv = {a.xpad, a.xpad, a.xpad, a.xpad};
#define DW_LOAD_B(dst)                                                                                  \
  _Pragma("unroll") for (int pb = 0; pb < PB; ++pb) {                                                   \
    const int ih = ih0[pb] + e_kh;                                                                      \
    const int iw = iw0[pb] + e_kw;                                                                      \
    const bool ok = pv[pb] && e_kh < KH && (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W;    \
    /* branch-free: out-of-image taps read the tensor base, then take the pad */                        \
    const int off = ok ? ((nb[pb] + ih) * W + iw) * XPS + XCO + e_c : 0;                                \
    u32x4 v = *reinterpret_cast<const u32x4*>(X + (size_t)off * ESZ);                                   \
    if (ESZ == 1) v ^= XXOR;                                                                            \
    dst[pb] = ok ? v : padv;                                                                            \
  }

  // ---- weight chunks: thread-strided 16-byte slices of [KC][BC][64 B]
  const int nchunks = (KSTEPS + KC - 1) / KC;
  u32x4 areg[AREG];
#define DW_FETCH_CHUNK(c)                                                                              \
  {                                                                                                    \
    const int s0_ = (c) * KC;                                                                          \
    const int nq_ = min(KC, KSTEPS - s0_) * BC * 4;                                                    \
    _Pragma("unroll") for (int t = 0; t < AREG; ++t) {                                                 \
      /* clamped index: every load is valid, so areg stays in registers */                            \
      const int q = min(tid + 256 * t, nq_ - 1);                                                       \
      const int sl = q / (BC * 4), r = q - sl * (BC * 4);                                              \
      areg[t] = *reinterpret_cast<const u32x4*>(WPK + ((size_t)(s0_ + sl) * COUTP + c0 + (r >> 2)) * 64 + \
                                                (r & 3) * 16);                                         \
    }                                                                                                  \
  }
#define DW_STORE_CHUNK(c, buf)                                                                       \
  {                                                                                                    \
    const int s0_ = (c) * KC;                                                                          \
    const int nq_ = min(KC, KSTEPS - s0_) * BC * 4;                                                    \
    uint8_t* As_ = smem + (buf) * ABYTES;                                                              \
    _Pragma("unroll") for (int t = 0; t < AREG; ++t) {                                                 \
      /* same clamp as the fetch: surplus threads rewrite the last slice with its own value */         \
      const int q = min(tid + 256 * t, nq_ - 1);                                                       \
      const int sl = q / (BC * 4), r = q - sl * (BC * 4);                                              \
      *reinterpret_cast<u32x4*>(As_ + sl * (BC * 64) + swz(r >> 2, r & 3)) = areg[t];                  \
    }                                                                                                  \
  }

  acc_t acc[CB][PB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) acc[cb][pb] = acc_t{0, 0, 0, 0};

  DW_FETCH_CHUNK(0);
  DW_STORE_CHUNK(0, 0);
  int my_s = ks;  // next k-step this wave computes
  u32x4 bcur[PB], bnext[PB];
  if (my_s < KSTEPS) {
    DW_LOAD_B(bcur);
  }
  __syncthreads();

  const int arow = lane & 15;
  const int kslice = lane >> 4;
  for (int c = 0; c < nchunks; ++c) {
    const bool more = c + 1 < nchunks;
    if (more) DW_FETCH_CHUNK(c + 1);
    const uint8_t* As = smem + (c & 1) * ABYTES;
    const int s1 = min(KSTEPS, (c + 1) * KC);
    while (my_s < s1) {
      const int nxt = my_s + KS;
      if (nxt < KSTEPS) {
        e_c += KS * KE;
        DW_NORMALIZE();
        DW_LOAD_B(bnext);
      }
      const uint8_t* Arow = As + (my_s - c * KC) * (BC * 64);
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const v4i af = *reinterpret_cast<const v4i*>(Arow + swz(cb * 16 + arow, kslice));
#pragma unroll
        for (int pb = 0; pb < PB; ++pb) {
          if constexpr (ESZ == 1) {
            acc[cb][pb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, __builtin_bit_cast(v4i, bcur[pb]),
                                                                acc[cb][pb], 0, 0, 0);
          } else {
            acc[cb][pb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                __builtin_bit_cast(v8h, af), __builtin_bit_cast(v8h, bcur[pb]), acc[cb][pb], 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) bcur[pb] = bnext[pb];
      my_s = nxt;
    }
    if (more) DW_STORE_CHUNK(c + 1, (c + 1) & 1);
    __syncthreads();
  }
#undef DW_NORMALIZE
#undef DW_LOAD_B
#undef DW_FETCH_CHUNK
#undef DW_STORE_CHUNK

  // ---- split-K: waves ks > 0 hand their partial sums to wave ks == 0
  if constexpr (KS > 1) {
    // (the final barrier of the k loop guarantees smem is free)
    acc_t* red = reinterpret_cast<acc_t*>(smem);
    if (ks > 0) {
      acc_t* dst = red + (((ks - 1) * PG + pg) * 64 + lane) * (CB * PB);
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
#pragma unroll
        for (int pb = 0; pb < PB; ++pb) dst[cb * PB + pb] = acc[cb][pb];
    }
    __syncthreads();
    if (ks > 0) return;
#pragma unroll
    for (int k2 = 1; k2 < KS; ++k2) {
      const acc_t* src = red + (((k2 - 1) * PG + pg) * 64 + lane) * (CB * PB);
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
#pragma unroll
        for (int pb = 0; pb < PB; ++pb) acc[cb][pb] += src[cb * PB + pb];
    }
  }

  // ---- epilogue: lane holds channels ch..ch+3 of pixel p for every block
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const int ch = c0 + cb * 16 + 4 * (lane >> 4);
    if (ch >= a.cout) continue;
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) {
      const int p = p0 + pb * 16 + (lane & 15);
      if (p < a.m) epilogue4<ESZ>(a, acc[cb][pb], ch, p);
    }
  }
}

// ---------------------------------------------------------------------------
// Weight packing: HWIO [K][cout] -> [ksteps][cout_pad][64 bytes], zero filled.
// ---------------------------------------------------------------------------
__global__ void pack_weights_kernel(const uint8_t* __restrict__ w, uint8_t* __restrict__ out, int K,
                                    int cout, int cout_pad, int ksteps, int esize) {
  const size_t total = (size_t)ksteps * cout_pad * 64;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const int b = (int)(i & 63);
    const size_t row = i >> 6;
    const int c = (int)(row % cout_pad);
    const int s = (int)(row / cout_pad);
    const int k = s * (64 / esize) + b / esize;
    uint8_t v = 0;
    if (k < K && c < cout) v = w[((size_t)k * cout + c) * esize + (b % esize)];
    out[i] = v;
  }
}

__global__ void qconv_bias_kernel(const int8_t* __restrict__ w, const int* __restrict__ bias,
                                  int* __restrict__ out, int K, int cout, int corr) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= cout) return;
  int s = 0;
  for (int k = 0; k < K; ++k) s += w[(size_t)k * cout + c];
  out[c] = (bias ? bias[c] : 0) + corr * s;
}

struct TileCfg {
  int bc, pb, ks;
};

int channel_tile(int cout) {
  if (cout > 96) return 128;
  if (cout > 80) return 96;
  if (cout > 64) return 80;
  if (cout > 48) return 64;
  if (cout > 32) return 48;
  if (cout > 16) return 32;
  return 16;
}

// Split-K partial sums must fit the 64 KB of LDS a workgroup may use.
bool splitk_fits(int bc, int pb, int ks) {
  if (ks == 1) return true;
  return (ks - 1) * (4 / ks) * 64 * (bc / 16) * pb * 16 <= 65536;
}

// Tile shape for a problem: the widest pixel tile that still yields at
// least two workgroups per CU; otherwise split the k-steps across the four
// waves (the deep, small-spatial layers).
TileCfg pick(const IgemmArgs& a) {
  const int bc = channel_tile(a.cout);
  // Tuning override "PB,KS" (pixel blocks per wave, k-split), e.g. "2,2".
  static const char* env = getenv("DW_IGEMM_TILE");
  if (env) {
    int pb = 0, ks = 0;
    if (sscanf(env, "%d,%d", &pb, &ks) == 2 && (pb == 1 || pb == 2 || pb == 4) &&
        (ks == 1 || ks == 2 || ks == 4) && splitk_fits(bc, pb, ks))
      return {bc, pb, ks};
  }
  const int ctiles = (a.cout_pad + bc - 1) / bc;
  const TileCfg opts[] = {{bc, 4, 1}, {bc, 4, 2}, {bc, 2, 2}, {bc, 4, 4}, {bc, 2, 4}, {bc, 1, 4}};
  TileCfg best = {bc, 1, 1};
  long best_wgs = 0;
  for (const TileCfg& t : opts) {
    if (!splitk_fits(t.bc, t.pb, t.ks)) continue;
    if (t.ks > 1 && a.ksteps < 2 * t.ks) continue;
    const int wgpix = (4 / t.ks) * 16 * t.pb;
    const long wgs = (long)((a.m + wgpix - 1) / wgpix) * ctiles;
    if (wgs >= 512) return t;
    if (wgs > best_wgs) {
      best_wgs = wgs;
      best = t;
    }
  }
  return best;
}

template <int ESZ, int BC>
bool launch_bc(hipStream_t st, const IgemmArgs& a, const TileCfg& t, dim3 grid) {
#define DW_T(PB, KS)                                                                       \
  if (t.pb == PB && t.ks == KS) {                                                          \
    hipLaunchKernelGGL((igemm_kernel<ESZ, BC, PB, KS>), grid, dim3(256), 0, st, a);        \
    return true;                                                                           \
  }
  DW_T(4, 1)
  DW_T(4, 2)
  DW_T(2, 2)
  DW_T(4, 4)
  DW_T(2, 4)
  DW_T(1, 4)
  DW_T(1, 1)
#undef DW_T
  return false;
}

template <int ESZ>
void launch_cfg(hipStream_t st, const IgemmArgs& a, const TileCfg& t) {
  const int wgpix = (4 / t.ks) * 16 * t.pb;
  const dim3 grid((unsigned)(((a.m + wgpix - 1) / wgpix) * (a.cout_pad / t.bc)));
  bool ok = false;
  switch (t.bc) {
    case 128: ok = launch_bc<ESZ, 128>(st, a, t, grid); break;
    case 96: ok = launch_bc<ESZ, 96>(st, a, t, grid); break;
    case 80: ok = launch_bc<ESZ, 80>(st, a, t, grid); break;
    case 64: ok = launch_bc<ESZ, 64>(st, a, t, grid); break;
    case 48: ok = launch_bc<ESZ, 48>(st, a, t, grid); break;
    case 32: ok = launch_bc<ESZ, 32>(st, a, t, grid); break;
    case 16: ok = launch_bc<ESZ, 16>(st, a, t, grid); break;
  }
  if (!ok) fail(-2, "igemm: no kernel for tile");
}

}  // namespace

int igemm_channel_tile(int cout) { return channel_tile(cout); }

const char* igemm_tile_name(const IgemmArgs& a, int esize) {
  static thread_local char buf[64];
  const TileCfg t = pick(a);
  snprintf(buf, sizeof buf, "igemm_%s_c%d_p%d_k%d", esize == 1 ? "i8" : "f16", t.bc, 16 * t.pb * (4 / t.ks),
           t.ks);
  return buf;
}

void launch_igemm(hipStream_t st, const IgemmArgs& a, int esize) {
  const TileCfg t = pick(a);
  if (a.cout_pad % t.bc != 0) fail(-4, "igemm: cout_pad not a multiple of the channel tile");
  if (esize == 1)
    launch_cfg<1>(st, a, t);
  else
    launch_cfg<2>(st, a, t);
  DW_HIP(hipGetLastError());
}

void launch_pack_weights(hipStream_t st, const void* w_hwio, void* wpk, int K, int cout,
                         int cout_pad, int ksteps, int esize) {
  const size_t total = (size_t)ksteps * cout_pad * 64;
  int blocks = (int)((total + 255) / 256);
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(pack_weights_kernel, dim3(blocks), dim3(256), 0, st,
                     (const uint8_t*)w_hwio, (uint8_t*)wpk, K, cout, cout_pad, ksteps, esize);
  DW_HIP(hipGetLastError());
}

void launch_qconv_bias(hipStream_t st, const int8_t* w_hwio, const int* bias, int* bias_out, int K,
                       int cout, int corr) {
  hipLaunchKernelGGL(qconv_bias_kernel, dim3((cout + 63) / 64), dim3(64), 0, st, w_hwio, bias,
                     bias_out, K, cout, corr);
  DW_HIP(hipGetLastError());
}

}  // namespace dw
