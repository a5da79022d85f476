// Implicit-GEMM convolution on CDNA4 matrix cores: tile selection, launch
// dispatch and weight packing.  The kernels are igemm_kernel.h, the
// persistent igemm_sk.h for small K, the streamed-weight igemm_stream.h for
// long K, the row-, band- and wide-tile kernels (igemm_rows.h, igemm_band.h,
// igemm_wide.h); their instantiations live in the k_igemm_*.hip files so
// that they compile in parallel.
#include "igemm_band.h"
#include "igemm_rows.h"
#include "igemm_sk.h"
#include "igemm_stream.h"
#include "igemm_wide.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>

namespace dw {
namespace {

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
  return {bc, pb, ring_depth(pb), kchunk, 0};
}

// The persistent small-K kernel: all of K in at most 4 k-steps, instantiated
// for these channel and pixel tiles.
bool sk_ok(const IgemmArgs& a, int bc, int pb, int tpw) {
  return tpw > 0 && a.ksteps >= 1 && a.ksteps <= 4 && (pb == 2 || pb == 4) &&
         (bc == 128 || bc == 64 || bc == 32 || bc == 16) && tile_ok(a, bc, pb);
}

TileCfg make_sk_tile(const IgemmArgs& a, int bc, int pb, int tpw) {
  TileCfg t = make_tile(a, bc, pb);
  t.kchunk = a.ksteps;
  t.tpw = tpw;
  return t;
}

// The streamed-weight kernel (tpw = -1): two or more k-steps, and its
// weight ring and k-slice table fit LDS.
bool st_ok(const IgemmArgs& a, int bc, int pb) {
  return tile_ok(a, bc, pb) && a.ksteps >= 2 && ig::st_lds_bytes(bc, a.ksteps, ring_depth(pb)) <= 160 * 1024;
}

TileCfg make_st_tile(const IgemmArgs& a, int bc, int pb) {
  TileCfg t = make_tile(a, bc, pb);
  t.tpw = -1;
  return t;
}

// The row-tile kernel (tpw = -2): int8 3x3, stride 1, padding 1 (same-size
// output), whole rows of 320 output pixels per workgroup (W divides 320, and
// the row count per tile divides H), channel tiles up to 96 (register
// budget), the input tile within the start-up loads and LDS.
bool rows_ok(const IgemmArgs& a, int bc) {
  const int es = a.epi == EPI_F16 ? 2 : 1;
  if (a.kh != 3 || a.kw != 3 || a.sh != 1 || a.sw != 1 || a.pt != 1 || a.pl != 1) return false;
  if (a.ho != a.h || a.wo != a.w || (a.cin * es) % 16 != 0 || a.w <= 0 || ig::kRowsPix % a.w != 0) return false;
  const int r = ig::kRowsPix / a.w;
  if (a.h % r != 0 || bc > 96 || !tile_ok(a, bc, 4)) return false;
  if ((r + 2) * (a.w + 2) * (a.cin * es / 16) > ig::kRowsFill * 256) return false;
  return ig::rows_lds_bytes(bc, a.ksteps, a.w, a.cin, es) <= 160 * 1024;
}

TileCfg make_rows_tile(const IgemmArgs& a, int bc) {
  TileCfg t = make_tile(a, bc, 4);
  t.kchunk = a.ksteps;
  t.tpw = -2;
  return t;
}

// The wide-tile kernel (tpw = -3): input rows of whole 128-byte units
// (c_in % 128 == 0 int8, % 64 == 0 fp16; 16-byte aligned views), 256-pixel
// workgroups of 64, 128 or 256 channels.
bool wide_ok(const IgemmArgs& a, int bc) {
  const int es = a.epi == EPI_F16 ? 2 : 1;
  if ((a.cin * es) % 128 != 0 || (a.x_pix_stride * es) % 16 != 0 || (a.x_c_off * es) % 16 != 0) return false;
  if (!(bc == 256 || bc == 128 || bc == 64) || a.cout_pad % bc != 0 || a.ksteps % 2 != 0) return false;
  if (bc > 64 && a.cout <= bc / 2) return false;  // half the tile would be padding
  return ig::wide_lds_bytes(bc, a.ksteps) <= 160 * 1024;
}

TileCfg make_wide_tile(const IgemmArgs& a, int bc) {
  TileCfg t = make_tile(a, std::min(bc, 128), 4);
  t.bc = bc;
  t.kchunk = a.ksteps;
  t.tpw = -3;
  return t;
}

// The band-tile kernel (tpw = -4: 8 waves, -5: 16 waves; pb = its band
// height R): 3x3, stride 1 or 2 on both axes, padding 1 (the output map
// (h - 1) / s + 1 by (w - 1) / s + 1), R whole output rows (R divides the
// output height) of at least one 16-pixel block per wave, the input tile
// within the start-up loads, everything within LDS.
int band_waves(int tpw) { return tpw == -5 ? 16 : 8; }

bool band_ok(const IgemmArgs& a, int bc, int rows, int tpw = -4) {
  const int es = a.epi == EPI_F16 ? 2 : 1;
  const int nw = band_waves(tpw);
  const int s = a.sh;
  // DW_BAND_S2=0: no stride-2 band tiles (plan comparisons)
  static const bool s2_on = !(getenv("DW_BAND_S2") && atoi(getenv("DW_BAND_S2")) == 0);
  if (a.kh != 3 || a.kw != 3 || !(s == 1 || (s == 2 && s2_on)) || a.sw != s || a.pt != 1 || a.pl != 1) return false;
  if (a.h <= 0 || a.w <= 0 || a.ho != (a.h - 1) / s + 1 || a.wo != (a.w - 1) / s + 1) return false;
  if ((a.cin * es) % 16 != 0) return false;
  if (!(bc == 128 || bc == 80 || bc == 64 || bc == 32 || bc == 16) || a.cout_pad % bc != 0) return false;
  // 16 waves over 64 channels: only the u8 requantize and table epilogues
  // without a residual fit 128 VGPRs
  if (nw == 16 && bc > 64 && !(es == 1 && a.epi == EPI_QU8 && !a.res && !a.h_wfrag)) return false;
  if (rows < 1 || a.ho % rows != 0 || rows * a.wo < 16 * nw) return false;
  const int cu = a.cin * es / 16;
  if ((long)ig::band_tile_rows(rows, s) * ig::band_tile_w(a.wo, s) * cu > ig::kBandFill * 512) return false;
  return ig::band_lds_bytes(bc, a.ksteps, rows, a.wo, cu, nw, s) <= 160 * 1024;
}

TileCfg make_band_tile(const IgemmArgs& a, int bc, int rows, int tpw = -4) {
  TileCfg t = make_tile(a, bc, 4);
  t.pb = rows;
  t.kchunk = a.ksteps;
  t.tpw = tpw;
  return t;
}

// Band heights worth timing for a channel tile and wave count: those that
// give between 96 and 768 workgroups (about one a CU up to three), at most 5.
int band_heights(const IgemmArgs& a, int bc, int tpw, int* rows, int max) {
  int n = 0;
  for (int r = 1; r <= a.ho && n < max; ++r) {
    if (!band_ok(a, bc, r, tpw)) continue;
    const long wgs = (long)a.n * (a.ho / r) * (a.cout_pad / bc);
    if (wgs >= 96 && wgs <= 768) rows[n++] = r;
  }
  return n;
}

// A detect head's 1x1 fused into the epilogue (a.h_wfrag): one tile holds
// every channel (64 or 80) on the staged kernel (with room for the regroup
// rows in its weight chunk), the row-tile or the band-tile kernel.
bool head_tile_ok(const IgemmArgs& a, const TileCfg& t) {
  if (!(t.bc == 64 || t.bc == 80) || a.cout_pad != t.bc) return false;
  if (t.tpw == -2) return rows_ok(a, t.bc);
  if (t.tpw == -4) return band_ok(a, t.bc, t.pb);
  return t.tpw == 0 && tile_ok(a, t.bc, t.pb) && t.kchunk * t.bc * 64 >= ig::xpose_bytes(t.bc);
}

// Tile shape for a problem: an override from DW_IGEMM_TILE (tests and
// tuning runs), an explicit choice (a.tile_bc / a.tile_pb, set by the graph
// runtime's tuner), else the widest channel tile and the widest pixel tile
// (16 * pb pixels per wave) that still gives about two workgroups per CU.
// The weight slice of the channel tile is staged in chunks of at most
// kWeightLds bytes.
TileCfg pick_any(const IgemmArgs& a);

// A launch that also writes an upsampled copy (a.y_up) takes any tile whose
// epilogue is igemm_store's; the persistent small-K kernel's is its own, so
// its tiles become the staged kernel's of the same shape.
TileCfg pick(const IgemmArgs& a) {
  TileCfg t = pick_any(a);
  if (a.y_up && t.tpw > 0) t = make_tile(a, t.bc, t.pb);
  return t;
}

TileCfg pick_any(const IgemmArgs& a) {
  if (a.h_wfrag) {
    // a DW_IGEMM_TILE row- or band-tile override, else the tuner's choice
    // when it is a head tile, else the staged kernel with the widest pixel
    // tile that fits
    if (const char* env = getenv("DW_IGEMM_TILE")) {
      int v0 = 0, v1 = 0, v2 = 0;
      if (sscanf(env, "%d,%d,%d", &v0, &v1, &v2) == 3 && (v2 == -2 || v2 == -4)) {
        const TileCfg t = v2 == -2 ? make_rows_tile(a, v0) : make_band_tile(a, v0, v1);
        if (head_tile_ok(a, t)) return t;
      }
    }
    if (a.tile_bc) {
      const TileCfg t = a.tile_tpw == -2   ? make_rows_tile(a, a.tile_bc)
                        : a.tile_tpw == -4 ? make_band_tile(a, a.tile_bc, a.tile_pb)
                                           : make_tile(a, a.tile_bc, a.tile_pb);
      if (head_tile_ok(a, t)) return t;
    }
    for (int pb : {4, 2, 1}) {
      const TileCfg t = make_tile(a, a.cout_pad, pb);
      if (head_tile_ok(a, t)) return t;
    }
    return make_tile(a, a.cout_pad, 1);  // launch_igemm refuses it
  }
  if (const char* env = getenv("DW_IGEMM_TILE")) {
    int v0 = 0, v1 = 0, v2 = 0;
    const int nv = sscanf(env, "%d,%d,%d", &v0, &v1, &v2);
    if (nv == 3 && sk_ok(a, v0, v1, v2)) return make_sk_tile(a, v0, v1, v2);
    if (nv == 3 && v2 == -1 && st_ok(a, v0, v1)) return make_st_tile(a, v0, v1);
    if (nv == 3 && v2 == -2 && rows_ok(a, v0)) return make_rows_tile(a, v0);
    if (nv == 3 && v2 == -3 && wide_ok(a, v0)) return make_wide_tile(a, v0);
    if (nv == 3 && (v2 == -4 || v2 == -5) && band_ok(a, v0, v1, v2)) return make_band_tile(a, v0, v1, v2);
    if (nv >= 2 && tile_ok(a, v0, v1)) return make_tile(a, v0, v1);
    if (nv == 1 && tile_ok(a, channel_tile(a.cout), v0)) return make_tile(a, channel_tile(a.cout), v0);
  }
  if (a.tile_bc && sk_ok(a, a.tile_bc, a.tile_pb, a.tile_tpw)) return make_sk_tile(a, a.tile_bc, a.tile_pb, a.tile_tpw);
  if (a.tile_bc && a.tile_tpw == -1 && st_ok(a, a.tile_bc, a.tile_pb)) return make_st_tile(a, a.tile_bc, a.tile_pb);
  if (a.tile_bc && a.tile_tpw == -2 && rows_ok(a, a.tile_bc)) return make_rows_tile(a, a.tile_bc);
  if (a.tile_bc && a.tile_tpw == -3 && wide_ok(a, a.tile_bc)) return make_wide_tile(a, a.tile_bc);
  if (a.tile_bc && (a.tile_tpw == -4 || a.tile_tpw == -5) && band_ok(a, a.tile_bc, a.tile_pb, a.tile_tpw))
    return make_band_tile(a, a.tile_bc, a.tile_pb, a.tile_tpw);
  if (a.tile_bc && tile_ok(a, a.tile_bc, a.tile_pb)) return make_tile(a, a.tile_bc, a.tile_pb);
  const int bc = channel_tile(a.cout);
  const int ctiles = a.cout_pad / bc;
  for (int pb : {4, 2, 1}) {
    const long wgs = (long)((a.m + 64 * pb - 1) / (64 * pb)) * ctiles;
    if (wgs >= 512) return make_tile(a, bc, pb);
  }
  return make_tile(a, bc, 1);
}

// Epilogue specialisation for the arguments.
int epilogue_variant(const IgemmArgs& a, int esize) {
  if (esize != 1 || a.epi != EPI_QU8) return EPV_GENERIC;
  if (a.h_wfrag) return EPV_QU8_LUT_HEAD;
  if (!a.lut) return a.res ? EPV_GENERIC : EPV_QU8;
  return a.res ? EPV_QU8_LUT_RES : EPV_QU8_LUT;
}

}  // namespace

int igemm_channel_tile(int cout) { return channel_tile(cout); }

bool igemm_sibling_tile_ok(const IgemmArgs& a, int bc, int tpw, int esize) {
  const bool common = !a.res && !a.y_up && !a.h_wfrag && bc > 0 && a.split > 0 && a.split % bc == 0 &&
                      a.split < a.cout && a.y2_pix_stride % 4 == 0 && a.y2_c_off % 4 == 0;
  if (esize == 1)  // the u8 table epilogue (its table staged per channel tile)
    return common && a.epi == EPI_QU8 && a.lut && a.lut2 && (tpw == 0 || tpw == -1 || tpw == -4 || tpw == -5);
  // fp16: the generic epilogue chooses the view per four channels; every
  // kernel storing through igemm_store (not the persistent small-K kernel)
  return common && esize == 2 && a.epi == EPI_F16 && tpw <= 0;
}

int igemm_candidates(const IgemmArgs& a, int* bc, int* pb, int* tpw, int max) {
  int n = 0;
  if (a.h_wfrag) {
    for (int p : {4, 2, 1})
      if (n < max && head_tile_ok(a, make_tile(a, a.cout_pad, p))) {
        bc[n] = a.cout_pad;
        pb[n] = p;
        tpw[n] = 0;
        ++n;
      }
    if (n < max && head_tile_ok(a, make_rows_tile(a, a.cout_pad))) {
      bc[n] = a.cout_pad;
      pb[n] = 4;
      tpw[n] = -2;
      ++n;
    }
    int rows[8];
    const int nr = band_heights(a, a.cout_pad, -4, rows, 8);
    for (int i = 0; i < nr && n < max; ++i)
      if (head_tile_ok(a, make_band_tile(a, a.cout_pad, rows[i]))) {
        bc[n] = a.cout_pad;
        pb[n] = rows[i];
        tpw[n] = -4;
        ++n;
      }
    return n;
  }
  // band tiles (8 and 16 waves): the widest channel tile, and 64 or 80
  // channels when that splits a wider layer in two or more (80: a sibling
  // GEMM whose first conv has 80 channels)
  {
    const int bw = std::min(a.cout_pad, 128);
    for (int tw : {-4, -5})
      for (int j = 0; j < 3; ++j) {
        const int b = j == 0 ? bw : (j == 1 ? 64 : 80);
        if (j > 0 && (bw <= b || a.cout_pad % b != 0)) continue;
        int rows[8];
        const int nr = band_heights(a, b, tw, rows, 8);
        for (int i = 0; i < nr && n < max; ++i) {
          bc[n] = b;
          pb[n] = rows[i];
          tpw[n] = tw;
          ++n;
        }
      }
  }
  for (int b : {256, 128, 64})
    if (n < max && wide_ok(a, b)) {
      bc[n] = b;
      pb[n] = 4;
      tpw[n] = -3;
      ++n;
    }
  for (int b : {128, 96, 80, 64, 48, 32, 16})
    for (int p : {4, 2, 1}) {
      if (n < max && tile_ok(a, b, p)) {
        bc[n] = b;
        pb[n] = p;
        tpw[n] = 0;
        ++n;
      }
      if (n < max && st_ok(a, b, p)) {
        bc[n] = b;
        pb[n] = p;
        tpw[n] = -1;
        ++n;
      }
      if (n < max && p == 4 && rows_ok(a, b)) {
        bc[n] = b;
        pb[n] = p;
        tpw[n] = -2;
        ++n;
      }
      // persistent variants that still leave a workgroup for every CU
      const long tiles = (long)((a.m + 64 * p - 1) / (64 * p)) * (a.cout_pad / std::max(b, 1));
      for (int t : {2, 4, 8})
        if (n < max && sk_ok(a, b, p, t) && tiles / t >= 256) {
          bc[n] = b;
          pb[n] = p;
          tpw[n] = t;
          ++n;
        }
    }
  return n;
}

const char* igemm_tile_name(const IgemmArgs& a, int esize) {
  static thread_local char buf[64];
  const TileCfg t = pick(a);
  if (t.tpw > 0)
    snprintf(buf, sizeof buf, "igemm_%s_c%d_p%d_t%d", esize == 1 ? "i8" : "f16", t.bc, 64 * t.pb, t.tpw);
  else if (t.tpw == -1)
    snprintf(buf, sizeof buf, "igemm_%s_c%d_p%d_st", esize == 1 ? "i8" : "f16", t.bc, 64 * t.pb);
  else if (t.tpw == -2)
    snprintf(buf, sizeof buf, "igemm_%s_c%d_rows", esize == 1 ? "i8" : "f16", t.bc);
  else if (t.tpw == -3)
    snprintf(buf, sizeof buf, "igemm_%s_c%d_wide", esize == 1 ? "i8" : "f16", t.bc);
  else if (t.tpw == -4)
    snprintf(buf, sizeof buf, "igemm_%s_c%d_band%d", esize == 1 ? "i8" : "f16", t.bc, t.pb);
  else if (t.tpw == -5)
    snprintf(buf, sizeof buf, "igemm_%s_c%d_band%dw16", esize == 1 ? "i8" : "f16", t.bc, t.pb);
  else
    snprintf(buf, sizeof buf, "igemm_%s_c%d_p%d", esize == 1 ? "i8" : "f16", t.bc, 64 * t.pb);
  if (a.h_wfrag) strncat(buf, "_head", sizeof buf - strlen(buf) - 1);
  if (a.y_up) strncat(buf, "_up", sizeof buf - strlen(buf) - 1);
  if (a.y2) strncat(buf, "_sib", sizeof buf - strlen(buf) - 1);
  return buf;
}

void launch_igemm(hipStream_t st, const IgemmArgs& a_in, int esize) {
  const TileCfg t = pick(a_in);
  if (a_in.cout_pad % t.bc != 0) fail(-4, "igemm: cout_pad not a multiple of the channel tile");
  if (a_in.m >= (1 << 24)) fail(-2, "igemm: more than 2^24 output pixels in one launch");
  if (a_in.kh * a_in.kw > 31) fail(-2, "igemm: more than 31 filter taps");
  IgemmArgs a = a_in;
  a.kchunk = t.kchunk;
  const long long xb = (long long)a.n * a.h * a.w * a.x_pix_stride * esize;
  if (xb >= (1ll << 31)) fail(-2, "igemm: input view larger than 2 GB");
  a.x_bytes = (int)xb;
  const size_t lds = t.tpw > 0     ? ig::sk_lds_bytes(t.bc, a.ksteps)
                     : t.tpw == -1 ? ig::st_lds_bytes(t.bc, a.ksteps, t.pd)
                     : t.tpw == -2 ? ig::rows_lds_bytes(t.bc, a.ksteps, a.w, a.cin, esize)
                     : t.tpw == -3 ? ig::wide_lds_bytes(t.bc, a.ksteps)
                     : t.tpw == -4 || t.tpw == -5
                         ? ig::band_lds_bytes(t.bc, a.ksteps, t.pb, a.wo, a.cin * esize / 16, band_waves(t.tpw), a.sh)
                                   : ig::lds_bytes(t, a.ksteps);
  if (lds > 160 * 1024) fail(-2, "igemm: k-slice table does not fit LDS");
  if ((long long)a.ho * a.wo >= (1ll << 23)) fail(-2, "igemm: more than 2^23 output pixels per image");
  if ((long long)a.ksteps * a.cout_pad * 64 >= (1ll << 32)) fail(-2, "igemm: packed weights larger than 4 GB");
  a.r_cin = 1.0f / (float)a.cin;
  a.r_kw = 1.0f / (float)a.kw;
  a.r_hwo = 1.0f / (float)(a.ho * a.wo);
  a.r_wo = 1.0f / (float)a.wo;
  // u8 output and residual views, addressed by the persistent kernel's
  // buffer stores and loads
  const long long yb = a.epi == EPI_QU8 ? (long long)a.m * a.y_pix_stride : 0;
  const long long rb = a.epi == EPI_QU8 && a.res ? (long long)a.m * a.r_pix_stride : 0;
  if (yb >= (1ll << 31) || rb >= (1ll << 31)) fail(-2, "igemm: output view larger than 2 GB");
  a.y_bytes = (int)yb;
  a.r_bytes = (int)rb;
  a.tile_tpw = t.tpw;
  a.band_rows = t.tpw == -4 || t.tpw == -5 ? t.pb : 0;
  if (a.y_up && (esize == 1 ? (a.epi != EPI_QU8 || a.h_wfrag || (a.res && !a.lut) || a.up_pix_stride % 4 != 0 ||
                                a.up_c_off % 4 != 0)
                             : (a.epi != EPI_F16 || a.up_pix_stride % 4 != 0 || a.up_c_off % 4 != 0)))
    fail(-2, "igemm: an upsampled copy needs a u8 table, requantize or f16 epilogue and aligned views");
  // a sibling GEMM: a kernel whose workgroup keeps one channel tile and
  // stores through igemm_store (staged, streamed-weight, band), the table
  // epilogue, and tiles that do not straddle the split
  if (a.y2 && !igemm_sibling_tile_ok(a, t.bc, t.tpw, esize))
    fail(-2, "igemm: a sibling GEMM needs the table epilogue and a staged, streamed or band tile within one conv");
  bool ok;
  if (esize == 1 && a.h_wfrag) {
    if (a.epi != EPI_QU8 || !a.lut || a.res || !head_tile_ok(a, t))
      fail(-2, "igemm: the fused head 1x1 needs a table epilogue and a tile of every channel");
    ok = igemm_launch_head_i8(st, a, t);
  } else if (esize == 1) {
    const int epv = epilogue_variant(a, esize);
    const bool ab = epv == EPV_GENERIC || epv == EPV_QU8;
    if (t.tpw > 0)
      ok = ab ? igemm_launch_sk_i8_a(st, a, t, epv) : igemm_launch_sk_i8_b(st, a, t, epv);
    else if (t.tpw == -1)
      ok = ab ? igemm_launch_st_i8_a(st, a, t, epv) : igemm_launch_st_i8_b(st, a, t, epv);
    else if (t.tpw == -2)
      ok = ab ? igemm_launch_rows_i8_a(st, a, t, epv) : igemm_launch_rows_i8_b(st, a, t, epv);
    else if (t.tpw == -3)
      ok = ab ? igemm_launch_wide_i8_a(st, a, t, epv) : igemm_launch_wide_i8_b(st, a, t, epv);
    else if (t.tpw == -4 || t.tpw == -5)
      ok = ab ? igemm_launch_band_i8_a(st, a, t, epv) : igemm_launch_band_i8_b(st, a, t, epv);
    else
      ok = ab ? igemm_launch_i8_a(st, a, t, epv) : igemm_launch_i8_b(st, a, t, epv);
  } else {
    ok = t.tpw > 0     ? igemm_launch_sk_f16(st, a, t)
         : t.tpw == -1 ? igemm_launch_st_f16(st, a, t)
         : t.tpw == -2 ? igemm_launch_rows_f16(st, a, t)
         : t.tpw == -3 ? igemm_launch_wide_f16(st, a, t)
         : t.tpw == -4 || t.tpw == -5 ? igemm_launch_band_f16(st, a, t)
                       : igemm_launch_f16(st, a, t);
  }
  if (!ok) fail(-2, "igemm: no kernel for tile");
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
