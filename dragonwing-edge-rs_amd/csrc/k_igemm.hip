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

#include <algorithm>
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

// Per-channel epilogue parameters of the workgroup's channel tile, staged
// in LDS at the start (indexed by the channel's position in the tile).
struct EpiLds {
  const int* bias;         // EPI_QU8 bias' or null
  const float* ms;         // EPI_QU8 multipliers
  const uint8_t* lut;      // EPI_QU8 table (256 entries) or null
  const uint16_t* bias_h;  // EPI_F16 bias or null
};

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

// Epilogue for one 16x16 block: this lane holds channels ch..ch+3 of pixel
// p (channel cl..cl+3 of the tile).
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
        float q = rintf((float)accs[r] * mss[r]) + (float)a.y_zp;
        q = fminf(fmaxf(q, 0.0f), 255.0f);
        int qi = (int)q;
        if (e.lut) qi = e.lut[qi];
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
    const uint32_t lo = (uint32_t)f16_chain(v[0], e.bias_h, cl + 0, a.act, hr, rres.x & 0xffff) |
                        ((uint32_t)f16_chain(v[1], e.bias_h, cl + 1, a.act, hr, rres.x >> 16) << 16);
    const uint32_t hi = (uint32_t)f16_chain(v[2], e.bias_h, cl + 2, a.act, hr, rres.y & 0xffff) |
                        ((uint32_t)f16_chain(v[3], e.bias_h, cl + 3, a.act, hr, rres.y >> 16) << 16);
    *reinterpret_cast<uint2*>((uint16_t*)a.y + yo) = make_uint2(lo, hi);
  }
}

template <int ESZ, int BC, int PB, int PD>
__global__ __launch_bounds__(256) void igemm_kernel(const IgemmArgs a) {
  constexpr int CB = BC / 16;       // 16-channel blocks (all channels of the tile per wave)
  constexpr int CE = 16 / ESZ;      // elements per 16-byte slice
  constexpr int WPIX = 16 * PB;     // pixels per wave
  constexpr int WGPIX = 4 * WPIX;   // pixels per workgroup
  using acc_t = typename std::conditional<ESZ == 1, v4i, v4f>::type;
  static_assert(BC % 16 == 0 && PD >= 2, "tile");
  // LDS: the weight chunk, fragment-major [k-step][channel block][lane][16 B],
  // then the k-slice table (one int2 per 16-byte slice along K).
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const uint8_t* __restrict__ X = a.x;
  const uint8_t* __restrict__ WPK = a.wpk;
  const int H = a.h, W = a.w, CIN = a.cin, KH = a.kh, KW = a.kw;
  const int XPS = a.x_pix_stride, XCO = a.x_c_off, KSTEPS = a.ksteps, COUTP = a.cout_pad;
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

  // ---- k-slice table: slice q of K (16 bytes, one filter tap) is at element
  // offset koff from the pixel's top-left tap and belongs to tap `tap`
  // (31 = past the end of K: always padding).  It does not depend on the
  // pixel, so the workgroup builds it once.
  // (the ring reads up to k-step KSTEPS + 2 * PD - 3, see the main loop)
  int2* ktab = reinterpret_cast<int2*>(smem + KCH * (BC * 64));
  const int nq = (KSTEPS + 2 * PD) * 4;
  const int kelems = KH * KW * CIN;
  for (int q = tid; q < nq; q += 256) {
    const int e = q * CE;
    int2 t = make_int2(0, 31);
    if (e < kelems) {
      const int tap = e / CIN, ci = e - (e / CIN) * CIN;
      const int kh = tap / KW, kw = tap - (tap / KW) * KW;
      t = make_int2((kh * W + kw) * XPS + ci, tap);
    }
    ktab[q] = t;
  }

  // ---- this lane's pixels p0 + pb*16 + (lane & 15): element offset of the
  // top-left tap and the in-image bit of every tap
  const int hw_o = a.ho * a.wo;
  int pbase[PB];
  uint32_t tmask[PB];
#pragma unroll
  for (int pb = 0; pb < PB; ++pb) {
    const int p = p0 + pb * 16 + (lane & 15);
    const bool pv = p < a.m;
    const int pp = pv ? p : 0;
    const int nn = pp / hw_o;
    const int r = pp - nn * hw_o;
    const int oh = r / a.wo;
    const int ow = r - oh * a.wo;
    const int ih0 = oh * a.sh - a.pt, iw0 = ow * a.sw - a.pl;
    pbase[pb] = ((nn * H + ih0) * W + iw0) * XPS + XCO;
    uint32_t m = 0;
    for (int kh = 0; kh < KH; ++kh)
      for (int kw = 0; kw < KW; ++kw)
        if ((unsigned)(ih0 + kh) < (unsigned)H && (unsigned)(iw0 + kw) < (unsigned)W) m |= 1u << (kh * KW + kw);
    tmask[pb] = pv ? m : 0u;
  }

  // Weight chunks go to LDS with direct global->LDS loads: one 1 KB
  // fragment per wave instruction, lane l writing bytes [16 l, 16 l + 16).
  const int frag_lane = ((lane & 15) * 64 + (lane >> 4) * 16);  // this lane's slice in a 16-row block
#define DW_ISSUE_A(s_first)                                                                         \
  {                                                                                                 \
    const int nfr_ = (min(KSTEPS, (s_first) + KCH) - (s_first)) * CB;                               \
    for (int f = wave; f < nfr_; f += 4) {                                                          \
      const int sl = f / CB, cb = f - (f / CB) * CB;                                                \
      const uint8_t* src = WPK + ((size_t)((s_first) + sl) * COUTP + c0 + cb * 16) * 64 + frag_lane; \
      __builtin_amdgcn_global_load_lds((const void*)src,                                            \
                                       (__attribute__((address_space(3))) void*)(smem + f * 1024), \
                                       16, 0, 0);                                                   \
    }                                                                                               \
  }
  // this wave's LDS writes (and loads) have landed, then everyone's have
#define DW_LDS_FENCE()              \
  __builtin_amdgcn_s_waitcnt(0);    \
  __syncthreads();

  // Epilogue parameters of the channel tile, also copied to LDS (one wave
  // each): bias' and multipliers, the activation table, or the f16 bias.
  uint8_t* sx = smem + KCH * (BC * 64) + nq * sizeof(int2);
  const int nvalid = min(BC, a.cout - c0);  // a multiple of 4
  EpiLds ep{nullptr, nullptr, nullptr, nullptr};
  if (a.epi == EPI_QU8) {
    ep.bias = a.bias_i ? reinterpret_cast<const int*>(sx) : nullptr;
    ep.ms = reinterpret_cast<const float*>(sx + BC * 4);
    ep.lut = a.lut ? sx + BC * 8 : nullptr;
  } else if (a.epi == EPI_F16 && a.bias_h) {
    ep.bias_h = reinterpret_cast<const uint16_t*>(sx);
  }

  __syncthreads();  // the k-slice table is complete
  // ---- im2col ring: k-step s lives in bq[s % PD], loaded PD - 1 steps
  // ahead.  The ring holds the raw loads and their in-image flags; the xor
  // and the pad select happen when the k-step is consumed, so nothing waits
  // for a load before its k-step comes up.  Every k-step issues exactly PB
  // loads, also past the last k-step (those read the pad), so the compiler's
  // load counters stay exact and a k-step waits only for its own loads.
  const u32x4 padv = {a.xpad, a.xpad, a.xpad, a.xpad};
  const int2* my_tab = ktab + (lane >> 4);
#define DW_LOAD_B(s_, dst, dok)                                                      \
  {                                                                                  \
    const int2 t_ = my_tab[(s_) * 4];                                                \
    _Pragma("unroll") for (int pb = 0; pb < PB; ++pb) {                              \
      const bool ok = (tmask[pb] >> t_.y) & 1u;                                      \
      /* out-of-image taps read the tensor base, then take the pad */              \
      const int off = ok ? pbase[pb] + t_.x : 0;                                     \
      dst[pb] = *reinterpret_cast<const u32x4*>(X + (size_t)(unsigned)off * ESZ);    \
      dok[pb] = ok;                                                                  \
    }                                                                                \
  }

  acc_t acc[CB][PB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) acc[cb][pb] = acc_t{0, 0, 0, 0};

  u32x4 bq[PD][PB];
  bool bok[PD][PB];
#pragma unroll
  for (int r = 0; r < PD - 1; ++r) DW_LOAD_B(r, bq[r], bok[r]);

  // All of the workgroup's start-up loads are in flight together: the first
  // PD - 1 im2col k-steps, the first weight chunk and the epilogue data.
  DW_ISSUE_A(0);
  if (a.epi == EPI_QU8) {
    if (wave == 0 && a.bias_i && lane < nvalid / 4)
      __builtin_amdgcn_global_load_lds((const void*)(a.bias_i + c0 + lane * 4),
                                       (__attribute__((address_space(3))) void*)sx, 16, 0, 0);
    if (wave == 1 && lane < nvalid / 4)
      __builtin_amdgcn_global_load_lds((const void*)(a.mscale + c0 + lane * 4),
                                       (__attribute__((address_space(3))) void*)(sx + BC * 4), 16, 0, 0);
    if (wave == 2 && a.lut && lane < 16)
      __builtin_amdgcn_global_load_lds((const void*)(a.lut + lane * 16),
                                       (__attribute__((address_space(3))) void*)(sx + BC * 8), 16, 0, 0);
  } else if (a.epi == EPI_F16 && a.bias_h) {
    if (wave == 0 && lane < nvalid / 2)
      __builtin_amdgcn_global_load_lds((const void*)(a.bias_h + c0 + lane * 2),
                                       (__attribute__((address_space(3))) void*)sx, 4, 0, 0);
  }
  DW_LDS_FENCE();

  int next_chunk = KCH, chunk0 = 0;
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
      }
      DW_LOAD_B(s + PD - 1, bq[(r + PD - 1) % PD], bok[(r + PD - 1) % PD]);
      if (s < KSTEPS) {
        u32x4 bcur[PB];
#pragma unroll
        for (int pb = 0; pb < PB; ++pb) bcur[pb] = bok[r][pb] ? (bq[r][pb] ^ XXOR) : padv;
        const uint8_t* Af = smem + (s - chunk0) * (CB * 1024) + lane * 16;
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          const v4i af = *reinterpret_cast<const v4i*>(Af + cb * 1024);
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
      }
    }
  }
#undef DW_ISSUE_A
#undef DW_LDS_FENCE
#undef DW_LOAD_B

  // ---- epilogue: lane holds channels ch..ch+3 of pixel p for every block
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const int ch = c0 + cb * 16 + 4 * (lane >> 4);
    if (ch >= a.cout) continue;
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) {
      const int p = p0 + pb * 16 + (lane & 15);
      if (p < a.m) epilogue4<ESZ>(a, ep, acc[cb][pb], ch, ch - c0, p);
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
  int bc, pb, pd, kchunk;
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

// LDS for the weight chunk of one workgroup: two workgroups fit a CU.
constexpr int kWeightLds = 65536;

// Prefetch depth of the im2col ring: deeper for narrow pixel tiles, whose
// k-steps are short, so about the same time's worth of loads is in flight.
int ring_depth(int pb) { return pb == 4 ? 4 : (pb == 2 ? 6 : 8); }

bool tile_ok(const IgemmArgs& a, int bc, int pb) {
  const int bcs[] = {128, 96, 80, 64, 48, 32, 16};
  bool known = false;
  for (int b : bcs) known |= b == bc;
  return known && (pb == 1 || pb == 2 || pb == 4) && bc <= channel_tile(a.cout) && a.cout_pad % bc == 0;
}

TileCfg make_tile(const IgemmArgs& a, int bc, int pb) {
  const int kchunk = std::max(1, std::min(a.ksteps, kWeightLds / (bc * 64)));
  return {bc, pb, ring_depth(pb), kchunk};
}

// Tile shape for a problem: an explicit choice (a.tile_bc / a.tile_pb, set
// by the graph runtime's tuner), else the widest channel tile and the widest
// pixel tile (16 * pb pixels per wave) that still gives about two
// workgroups per CU.  The weight slice of the channel tile is staged in
// chunks of at most kWeightLds bytes.
TileCfg pick(const IgemmArgs& a) {
  // Override for tests and tuning runs: "BC,PB" (or "PB" with the default
  // channel tile), applied where it is a valid shape for the problem.
  if (const char* env = getenv("DW_IGEMM_TILE")) {
    int v0 = 0, v1 = 0;
    const int nv = sscanf(env, "%d,%d", &v0, &v1);
    if (nv == 2 && tile_ok(a, v0, v1)) return make_tile(a, v0, v1);
    if (nv == 1 && tile_ok(a, channel_tile(a.cout), v0)) return make_tile(a, channel_tile(a.cout), v0);
  }
  if (a.tile_bc && tile_ok(a, a.tile_bc, a.tile_pb)) return make_tile(a, a.tile_bc, a.tile_pb);
  const int bc = channel_tile(a.cout);
  const int ctiles = a.cout_pad / bc;
  for (int pb : {4, 2, 1}) {
    const long wgs = (long)((a.m + 64 * pb - 1) / (64 * pb)) * ctiles;
    if (wgs >= 512) return make_tile(a, bc, pb);
  }
  return make_tile(a, bc, 1);
}

template <int ESZ, int BC>
bool launch_bc(hipStream_t st, const IgemmArgs& a, const TileCfg& t, dim3 grid) {
  // weight chunk + k-slice table
  // weight chunk + k-slice table + epilogue data (bias', multipliers, table)
  const size_t lds = (size_t)t.kchunk * BC * 64 + (size_t)(a.ksteps + 2 * t.pd) * 4 * sizeof(int2) + BC * 8 + 256;
#define DW_T(PB, PD)                                                                       \
  if (t.pb == PB && t.pd == PD) {                                                          \
    hipLaunchKernelGGL((igemm_kernel<ESZ, BC, PB, PD>), grid, dim3(256), lds, st, a);      \
    return true;                                                                           \
  }
  DW_T(4, 4)
  DW_T(2, 6)
  DW_T(1, 8)
#undef DW_T
  return false;
}

template <int ESZ>
void launch_cfg(hipStream_t st, const IgemmArgs& a, const TileCfg& t) {
  const int wgpix = 64 * t.pb;
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

int igemm_candidates(const IgemmArgs& a, int* bc, int* pb, int max) {
  int n = 0;
  for (int b : {128, 96, 80, 64, 48, 32, 16})
    for (int p : {4, 2, 1})
      if (n < max && tile_ok(a, b, p)) {
        bc[n] = b;
        pb[n] = p;
        ++n;
      }
  return n;
}

const char* igemm_tile_name(const IgemmArgs& a, int esize) {
  static thread_local char buf[64];
  const TileCfg t = pick(a);
  snprintf(buf, sizeof buf, "igemm_%s_c%d_p%d", esize == 1 ? "i8" : "f16", t.bc, 64 * t.pb);
  return buf;
}

void launch_igemm(hipStream_t st, const IgemmArgs& a_in, int esize) {
  const TileCfg t = pick(a_in);
  if (a_in.cout_pad % t.bc != 0) fail(-4, "igemm: cout_pad not a multiple of the channel tile");
  IgemmArgs a = a_in;
  a.kchunk = t.kchunk;
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
