// Implicit-GEMM convolution on CDNA4 matrix cores (gfx950).
//
// The convolution is the GEMM  Y[c][p] = sum_k W[k][c] * X[p][k]  with
//   c = output channel, p = output pixel (n, oh, ow), k = (kh, kw, ci).
// MFMA operand A holds weight rows (channels), operand B holds im2col rows
// (pixels); both are 64-byte rows per k-step (64 int8 or 32 fp16 values).
// One wavefront instruction is v_mfma_i32_16x16x64_i8 (int8) or
// v_mfma_f32_16x16x32_f16 (fp16); each lane owns a 16-byte slice of a row,
// so every global load, LDS store and LDS read is 16 bytes per lane.
//
// Work split: a 256-thread workgroup computes a BC x BP (channels x pixels)
// tile; its four waves form a WC x WP grid of (BC/WC) x (BP/WP) wave tiles.
// The k loop double-buffers both operand tiles in LDS (one barrier per
// k-step): the next step's global loads are issued before the current
// step's MFMAs so their latency hides behind matrix work.
//
// The im2col rows are gathered straight from NHWC memory: a 16-byte chunk
// is 16 (int8) or 8 (fp16) consecutive input channels of one filter tap, so
// c_in * esize must be a multiple of 16.  Out-of-image taps read the
// zero-point pattern (int8) or 0 (fp16).  u8 inputs are mapped to s8 by
// xor 0x80 (x - 128); the missing (128 - x_zp) * sum_k W is folded into the
// per-channel bias on the host side, so results are exact.
//
// Epilogues fuse what the reference runs as separate passes: bias, the
// requantization with its rounding rule, activations (f16 chain or a u8
// table) and the residual add; stores go to channel-strided views so concat
// outputs are written in place.
#include "dw_common.h"
#include "dw_device.h"

#include <stdio.h>

#include <type_traits>

namespace dw {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

// LDS address of 16-byte chunk `chunk` (0..3) of 64-byte row `row`, xor
// swizzled so that 8 consecutive rows at one chunk hit distinct banks.
__device__ __forceinline__ int swz(int row, int chunk) {
  return row * 64 + ((chunk ^ ((row >> 1) & 3)) << 4);
}


// f16 epilogue chain of CpuGraphRuntime: conv result rounded to f16, bias
// added in f32 and rounded, activation computed in f32 from f16 and rounded
// (SiLU = Sigmoid then Mul, each rounded), residual added and rounded.
__device__ __forceinline__ uint16_t f16_chain(float acc, const uint16_t* bias_h, int ch, int act,
                                              bool has_res, uint16_t resv) {
  uint16_t hb = f2h(acc);
  if (bias_h) hb = f16_add_bits(hb, bias_h[ch]);
  hb = f16_act_bits(hb, act);
  if (has_res) hb = f16_add_bits(hb, resv);
  return hb;
}

template <int ESZ, int BC, int BP, int WC, int WP>
__global__ __launch_bounds__(256) void igemm_conv_kernel(const IgemmArgs a) {
  constexpr int CB = BC / 16 / WC;  // 16-channel blocks per wave
  constexpr int PB = BP / 16 / WP;  // 16-pixel blocks per wave
  constexpr int KE = 64 / ESZ;      // elements per row per k-step
  constexpr int CE = 16 / ESZ;      // elements per 16-byte chunk
  constexpr int TILE = (BC + BP) * 64;
  constexpr int BROWS = BP / 64;    // B rows loaded per thread
  constexpr int ACHUNKS = BC * 4;   // 16-byte chunks of the A tile
  constexpr int AITER = (ACHUNKS + 255) / 256;
  static_assert(BC % (16 * WC) == 0 && BP % (16 * WP) == 0 && WC * WP == 4, "tile");
  static_assert(BP % 64 == 0, "BP");

  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * TILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wc = wave % WC;
  const int wp = wave / WC;
  const int p0 = blockIdx.x * BP;
  const int c0 = blockIdx.y * BC;

  // ---- per-thread im2col gather state: rows (tid>>2) + 64*i, chunk j.
  const int j = tid & 3;
  const int hw_o = a.ho * a.wo;
  int ih0[BROWS], iw0[BROWS], nb[BROWS];
  bool pv[BROWS];
#pragma unroll
  for (int i = 0; i < BROWS; ++i) {
    const int p = p0 + (tid >> 2) + 64 * i;
    pv[i] = p < a.m;
    const int pp = pv[i] ? p : 0;
    const int nn = pp / hw_o;
    const int rem = pp - nn * hw_o;
    const int oh = rem / a.wo;
    const int ow = rem - oh * a.wo;
    ih0[i] = oh * a.sh - a.pt;
    iw0[i] = ow * a.sw - a.pl;
    nb[i] = nn * a.h;
  }
  int e_c = j * CE;
  int e_kh = 0, e_kw = 0;
  while (e_c >= a.cin) {
    e_c -= a.cin;
    if (++e_kw == a.kw) { e_kw = 0; ++e_kh; }
  }

  const uint4 padv = make_uint4(a.xpad, a.xpad, a.xpad, a.xpad);
  uint4 breg[BROWS];
  uint4 areg[AITER];

  auto load_b = [&]() {
#pragma unroll
    for (int i = 0; i < BROWS; ++i) {
      const int ih = ih0[i] + e_kh;
      const int iw = iw0[i] + e_kw;
      const bool ok = pv[i] && e_kh < a.kh && (unsigned)ih < (unsigned)a.h &&
                      (unsigned)iw < (unsigned)a.w;
      if (ok) {
        const int off = ((nb[i] + ih) * a.w + iw) * a.x_pix_stride + a.x_c_off + e_c;
        uint4 v = *reinterpret_cast<const uint4*>(a.x + (size_t)off * ESZ);
        if (ESZ == 1) {
          v.x ^= a.xxor; v.y ^= a.xxor; v.z ^= a.xxor; v.w ^= a.xxor;
        }
        breg[i] = v;
      } else {
        breg[i] = padv;
      }
    }
  };
  auto advance_k = [&]() {
    e_c += KE;
    while (e_c >= a.cin) {
      e_c -= a.cin;
      if (++e_kw == a.kw) { e_kw = 0; ++e_kh; }
    }
  };
  auto load_a = [&](int s) {
    const uint8_t* src = a.wpk + ((size_t)s * a.cout_pad + c0) * 64;
#pragma unroll
    for (int t = 0; t < AITER; ++t) {
      const int q = tid + 256 * t;
      if (q < ACHUNKS) areg[t] = *reinterpret_cast<const uint4*>(src + q * 16);
    }
  };
  auto store_tiles = [&](int buf) {
    uint8_t* As = smem + buf * TILE;
    uint8_t* Bs = As + BC * 64;
#pragma unroll
    for (int t = 0; t < AITER; ++t) {
      const int q = tid + 256 * t;
      if (q < ACHUNKS) *reinterpret_cast<uint4*>(As + swz(q >> 2, q & 3)) = areg[t];
    }
#pragma unroll
    for (int i = 0; i < BROWS; ++i)
      *reinterpret_cast<uint4*>(Bs + swz((tid >> 2) + 64 * i, j)) = breg[i];
  };

  typedef typename std::conditional<ESZ == 1, v4i, v4f>::type acc_t;
  acc_t acc[CB][PB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) acc[cb][pb] = acc_t{0, 0, 0, 0};

  load_a(0);
  load_b();
  store_tiles(0);
  __syncthreads();

  const int arow0 = wc * CB * 16 + (lane & 15);
  const int brow0 = wp * PB * 16 + (lane & 15);
  const int kchunk = lane >> 4;

  for (int s = 0; s < a.ksteps; ++s) {
    const int cur = s & 1;
    const bool more = s + 1 < a.ksteps;
    if (more) {
      advance_k();
      load_a(s + 1);
      load_b();
    }
    const uint8_t* As = smem + cur * TILE;
    const uint8_t* Bs = As + BC * 64;
    v4i af[CB], bf[PB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
      af[cb] = *reinterpret_cast<const v4i*>(As + swz(arow0 + cb * 16, kchunk));
#pragma unroll
    for (int pb = 0; pb < PB; ++pb)
      bf[pb] = *reinterpret_cast<const v4i*>(Bs + swz(brow0 + pb * 16, kchunk));
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) {
        if constexpr (ESZ == 1) {
          acc[cb][pb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[cb], bf[pb], acc[cb][pb], 0, 0, 0);
        } else {
          acc[cb][pb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              __builtin_bit_cast(v8h, af[cb]), __builtin_bit_cast(v8h, bf[pb]), acc[cb][pb], 0, 0, 0);
        }
      }
    if (more) store_tiles(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane holds channels ch..ch+3 of pixel p for every block.
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const int ch = c0 + wc * CB * 16 + cb * 16 + 4 * (lane >> 4);
    if (ch >= a.cout) continue;
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) {
      const int p = p0 + wp * PB * 16 + pb * 16 + (lane & 15);
      if (p >= a.m) continue;
      const size_t yo = (size_t)p * a.y_pix_stride + a.y_c_off + ch;
      if constexpr (ESZ == 1) {
        const v4i v = acc[cb][pb];
        if (a.epi == EPI_QU8) {
          const int4 bi = a.bias_i ? *reinterpret_cast<const int4*>(a.bias_i + ch) : make_int4(0, 0, 0, 0);
          const float4 ms = *reinterpret_cast<const float4*>(a.mscale + ch);
          uint32_t rres = 0;
          if (a.res) {
            rres = *reinterpret_cast<const uint32_t*>(
                (const uint8_t*)a.res + (size_t)p * a.r_pix_stride + a.r_c_off + ch);
          }
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
              float f = (float)(qi - a.za) * a.ra + (float)(rb - a.zb) * a.rb;
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
        const v4f v = acc[cb][pb];
        uint2 rres = make_uint2(0, 0);
        if (a.res) {
          rres = *reinterpret_cast<const uint2*>(
              (const uint16_t*)a.res + (size_t)p * a.r_pix_stride + a.r_c_off + ch);
        }
        const uint16_t r0 = rres.x & 0xffff, r1 = rres.x >> 16, r2 = rres.y & 0xffff, r3 = rres.y >> 16;
        const bool hr = a.res != nullptr;
        const uint32_t lo = (uint32_t)f16_chain(v[0], a.bias_h, ch + 0, a.act, hr, r0) |
                            ((uint32_t)f16_chain(v[1], a.bias_h, ch + 1, a.act, hr, r1) << 16);
        const uint32_t hi = (uint32_t)f16_chain(v[2], a.bias_h, ch + 2, a.act, hr, r2) |
                            ((uint32_t)f16_chain(v[3], a.bias_h, ch + 3, a.act, hr, r3) << 16);
        *reinterpret_cast<uint2*>((uint16_t*)a.y + yo) = make_uint2(lo, hi);
      }
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
  int bc, bp, wc, wp;
};

TileCfg pick_tile(int cout) {
  if (cout > 128) return {128, 256, 2, 2};
  if (cout > 96) return {128, 256, 1, 4};
  if (cout > 80) return {96, 256, 1, 4};
  if (cout > 64) return {80, 256, 1, 4};
  if (cout > 48) return {64, 256, 1, 4};
  if (cout > 32) return {48, 256, 1, 4};
  if (cout > 16) return {32, 256, 1, 4};
  return {16, 256, 1, 4};
}

template <int ESZ>
void launch_cfg(hipStream_t st, const IgemmArgs& a, const TileCfg& t) {
  dim3 grid((a.m + t.bp - 1) / t.bp, a.cout_pad / t.bc);
  dim3 block(256);
#define DW_TILE(BC, BP, WC, WP)                                                     \
  if (t.bc == BC && t.bp == BP && t.wc == WC && t.wp == WP) {                      \
    hipLaunchKernelGGL((igemm_conv_kernel<ESZ, BC, BP, WC, WP>), grid, block, 0, st, a); \
    return;                                                                         \
  }
  DW_TILE(128, 256, 2, 2)
  DW_TILE(128, 256, 1, 4)
  DW_TILE(96, 256, 1, 4)
  DW_TILE(80, 256, 1, 4)
  DW_TILE(64, 256, 1, 4)
  DW_TILE(48, 256, 1, 4)
  DW_TILE(32, 256, 1, 4)
  DW_TILE(16, 256, 1, 4)
#undef DW_TILE
  fail(-2, "igemm: no kernel for tile");
}

}  // namespace

int igemm_channel_tile(int cout) { return pick_tile(cout).bc; }

const char* igemm_tile_name(const IgemmArgs& a, int esize) {
  static thread_local char buf[64];
  TileCfg t = pick_tile(a.cout);
  snprintf(buf, sizeof buf, "igemm_%s_%dx%d_w%dx%d", esize == 1 ? "i8" : "f16", t.bc, t.bp, t.wc, t.wp);
  return buf;
}

void launch_igemm(hipStream_t st, const IgemmArgs& a, int esize) {
  TileCfg t = pick_tile(a.cout);
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
