// Convolutions whose whole K (kh * kw * c_in, c_in <= 4) fits one fp16 MFMA
// k-step of 32: the three-channel stem of the fp16 graphs (3x3, stride 2), on the
// fp16 matrix cores, held to the fp16 tolerance as the other MFMA convs
// (the exact-order kernel in k_direct.hip stays for the INT8 graph's stem,
// whose u8 output must be bit-exact).
//
// The input rows (c_in = 3 values a pixel) are not 16-byte slices of one
// tap, so the implicit-GEMM loaders do not apply.  A workgroup (4 waves)
// owns two output rows of one image and every output channel (up to 64):
// it copies the input rows their windows reach (padding as zeros) into LDS
// with coalesced loads (from the f16 NHWC tensor, or from the graph input's
// NCHW f32 planes, rounding each value to f16 as F16::from_f32 does, so the
// tile holds the bytes the host conversion would have produced), then each
// lane gathers its own B operand from there, the 8 consecutive values of K
// (tap-major, channel-minor, as the HWIO weights flatten) that
// v_mfma_f32_16x16x32_f16 takes from it, for one output pixel: lane l supplies pixel l % 16 and K values 8 (l / 16) .. +7,
// zeros past K.  The (tap row, tap column, channel) of those 8 values depend
// only on l / 16, so they are worked out once.  The weight fragments (one
// per 16 channels) are read once per lane.  The epilogue is the fp16 chain
// of the other MFMA convs: round to f16, f16 bias, activation
// (conv1x1_f16_finish).
#include "dw_common.h"
#include "dw_device.h"

namespace dw {
namespace {

constexpr int kStemRows = 2;  // output rows per workgroup

__host__ __device__ inline int stem_tile_rows(const StemF16Args& a) { return (kStemRows - 1) * a.sh + a.kh; }
__host__ __device__ inline int stem_tile_cols(const StemF16Args& a) { return (a.wo - 1) * a.sw + a.kw; }

template <int CB, bool NCHW>
__global__ __launch_bounds__(256) void stem_f16_mfma_kernel(const StemF16Args a) {
  extern __shared__ uint16_t tile[];  // [tile rows][tile columns][c_in]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bands = (a.ho + kStemRows - 1) / kStemRows;
  const int n = blockIdx.x / bands;
  const int oh0 = (blockIdx.x - n * bands) * kStemRows;
  const int TR = stem_tile_rows(a), TC = stem_tile_cols(a);
  const int ih0 = oh0 * a.sh - a.pt;
  // ---- the input rows of the band, columns -pl .. , zeros outside the image:
  // kFill pixels a thread per round, all their loads in flight before the
  // first LDS store
  constexpr int kFill = 16;
  const int units = TR * TC;
  const float rtc = 1.0f / (float)TC;
  for (int u0 = 0; u0 < units; u0 += 256 * kFill) {
    uint16_t v[kFill][4];
    int dst[kFill];
#pragma unroll
    for (int i = 0; i < kFill; ++i) {
      const int t = u0 + i * 256 + tid;
      dst[i] = -1;
#pragma unroll
      for (int c = 0; c < 4; ++c) v[i][c] = 0;
      if (t < units) {
        int tr = (int)((float)t * rtc);  // t / TC, corrected once
        if (tr * TC > t) --tr;
        else if ((tr + 1) * TC <= t) ++tr;
        const int ih = ih0 + tr, iw = t - tr * TC - a.pl;
        dst[i] = t * a.cin;
        if ((unsigned)ih < (unsigned)a.h && (unsigned)iw < (unsigned)a.w) {
          if constexpr (NCHW) {
            const long long plane = (long long)a.h * a.w;
            const float* src = a.x_nchw + (long long)n * a.cin * plane + (long long)ih * a.w + iw;
#pragma unroll
            for (int c = 0; c < 4; ++c)
              if (c < a.cin) v[i][c] = f2h(src[c * plane]);
          } else {
            const uint16_t* src = a.x + ((long long)(n * a.h + ih) * a.w + iw) * a.x_pix_stride + a.x_c_off;
#pragma unroll
            for (int c = 0; c < 4; ++c)
              if (c < a.cin) v[i][c] = src[c];
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < kFill; ++i)
      if (dst[i] >= 0) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (c < a.cin) tile[dst[i] + c] = v[i][c];
      }
  }
  // this lane's 8 values of K: tile offsets from the window's top-left
  const int K = a.kh * a.kw * a.cin;
  int off[8];
  bool kin[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int k = 8 * (lane >> 4) + j;
    kin[j] = k < K;
    const int kk = kin[j] ? k : 0;
    const int tap = kk / a.cin, c = kk - (kk / a.cin) * a.cin;
    const int dh = tap / a.kw, dw = tap - (tap / a.kw) * a.kw;
    off[j] = (dh * TC + dw) * a.cin + c;
  }
  f16x8 wf[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) wf[cb] = *reinterpret_cast<const f16x8*>(a.wfrag + ((size_t)cb * 64 + lane) * 8);
  __syncthreads();
  const int np = min(kStemRows, a.ho - oh0) * a.wo;
  const int nb = (np + 15) / 16;
  // blocks of 16 pixels; when the output rows hold whole blocks, a block's
  // row is wave-uniform (scalar division), else each lane divides
  const int bpr = a.wo % 16 == 0 ? a.wo / 16 : 0;
  for (int b = wave; b < nb; b += 4) {
    const int pl = b * 16 + (lane & 15);
    const bool pv = pl < np;
    int orow, ow;
    if (bpr) {
      orow = b / bpr;
      ow = (b - orow * bpr) * 16 + (lane & 15);
    } else {
      const int q = pv ? pl : 0;
      orow = q / a.wo;
      ow = q - orow * a.wo;
    }
    const int base = ((orow * a.sh) * TC + ow * a.sw) * a.cin;
    f16x8 xv;
#pragma unroll
    for (int j = 0; j < 8; ++j) xv[j] = __builtin_bit_cast(_Float16, kin[j] ? tile[base + off[j]] : (uint16_t)0);
    const size_t p = ((size_t)n * a.ho + oh0 + orow) * a.wo + ow;
    uint16_t* yrow = a.y + p * a.y_pix_stride + a.y_c_off;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[cb], xv, acc, 0, 0, 0);
      const int ch = cb * 16 + 4 * (lane >> 4);
      if (pv) *reinterpret_cast<uint2*>(yrow + ch) = conv1x1_f16_finish(acc, a.bias ? a.bias + ch : nullptr, a.act);
    }
  }
}

}  // namespace

namespace {
size_t stem_lds(int cin, int kh, int kw, int wo, int sh, int sw) {
  return (size_t)((kStemRows - 1) * sh + kh) * ((wo - 1) * sw + kw) * cin * 2;
}
}  // namespace

bool stem_f16_supported(int cin, int kh, int kw, int cout, int wo, int sh, int sw) {
  return cin >= 1 && cin <= 4 && kh * kw * cin <= 32 && cout % 16 == 0 && cout >= 16 && cout <= 64 && wo >= 1 &&
         stem_lds(cin, kh, kw, wo, sh, sw) <= 64 * 1024;
}

void launch_stem_f16(hipStream_t st, const StemF16Args& a) {
  if (!stem_f16_supported(a.cin, a.kh, a.kw, a.cout, a.wo, a.sh, a.sw)) fail(-2, "fp16 stem: unsupported shape");
  if (a.m <= 0) return;
  if ((long long)a.n * a.h * a.w * a.x_pix_stride >= (1ll << 31) || (long long)a.m * a.y_pix_stride >= (1ll << 31))
    fail(-2, "fp16 stem: views larger than 2^31 elements");
  const size_t lds = stem_lds(a.cin, a.kh, a.kw, a.wo, a.sh, a.sw);
  const dim3 grid((unsigned)(a.n * ((a.ho + kStemRows - 1) / kStemRows)));
  if (a.in_kind != 1 && a.in_kind != 3) fail(-2, "fp16 stem: input kind must be 1 (f16 NHWC) or 3 (f32 NCHW)");
#define DW_STEM(CB_)                                                                              \
  if (a.in_kind == 3)                                                                             \
    hipLaunchKernelGGL((stem_f16_mfma_kernel<CB_, true>), grid, dim3(256), lds, st, a);          \
  else                                                                                            \
    hipLaunchKernelGGL((stem_f16_mfma_kernel<CB_, false>), grid, dim3(256), lds, st, a);
  switch (a.cout / 16) {
    case 1: DW_STEM(1) break;
    case 2: DW_STEM(2) break;
    case 3: DW_STEM(3) break;
    default: DW_STEM(4) break;
  }
#undef DW_STEM
  DW_HIP(hipGetLastError());
}

}  // namespace dw
