// Internal declarations shared by the HIP kernels and the C++ host runtime.
// Nothing here crosses the C ABI (include/dw_hip.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

namespace dw {

// ----------------------------------------------------------------------------
// Error plumbing: every C-ABI function converts a thrown dw::Error into a
// status code plus a thread-local message.
// ----------------------------------------------------------------------------
struct Error {
  int code;
  std::string msg;
};
[[noreturn]] void fail(int code, const std::string& msg);
void hip_check(hipError_t e, const char* what);
#define DW_HIP(call) ::dw::hip_check((call), #call)

// Element types (match DW_DTYPE_* in dw_hip.h).
enum Dtype : int { F32 = 0, F16 = 1, I8 = 2, U8 = 3, I32 = 4 };
__host__ __device__ inline int dtype_size(int dt) {
  return dt == F32 || dt == I32 ? 4 : dt == F16 ? 2 : 1;
}

// Activations (match DW_ACT_*).
enum Act : int { ACT_NONE = 0, ACT_RELU = 1, ACT_SILU = 2 };

// Implicit-GEMM epilogues.
enum Epi : int {
  EPI_QU8 = 0,      // u8 out: rint((acc+bias)*M[c]) + zp, clamp [0,255], LUT, residual QLinearAdd
  EPI_QS8_REF = 1,  // s8 out: clamp(acc*scale) then round half away; optional ReLU
  EPI_I32 = 2,      // raw int32 accumulator
  EPI_F16 = 3       // f16 out with the CPU runtime's rounding points
};

// A channel-strided NHWC view: element (pixel p, channel c) lives at
// base + (p * pix_stride + c_off + c) * esize.  Concat/split outputs are
// views into one buffer, so no copy kernels are needed for them.
struct View {
  void* base = nullptr;
  int pix_stride = 0;  // elements between consecutive pixels
  int c_off = 0;       // first channel
};

// Convolution geometry (NHWC, HWIO weights).
struct ConvGeom {
  int n, h, w, cin, cout, kh, kw, sh, sw, pt, pl, ho, wo;
};

// Arguments of the MFMA implicit-GEMM convolution (int8 and fp16).
struct IgemmArgs {
  const uint8_t* x;
  const uint8_t* wpk;  // packed weights [ksteps][cout_pad][64 bytes]
  void* y;
  const void* res;     // residual (EPI_QU8: u8, EPI_F16: f16) or null
  int n, h, w, cin, cout, kh, kw, sh, sw, pt, pl, ho, wo;
  int m;        // n*ho*wo output pixels
  int ksteps;   // ceil(kh*kw*cin*esize / 64)
  int cout_pad; // rows per k-step in wpk
  int x_pix_stride, x_c_off;
  int y_pix_stride, y_c_off;
  int r_pix_stride, r_c_off;
  int epi, act;
  uint32_t xpad;  // padded-input byte pattern (int8 domain after xor)
  uint32_t xxor;  // 0x80808080 when the input is u8, else 0
  const int* bias_i;     // EPI_QU8: bias + (128 - x_zp) * sum_k w[k][c]
  const float* mscale;   // EPI_QU8: per-channel multiplier
  float tscale;          // EPI_QS8_REF: per-tensor requant scale
  int y_zp;
  const uint8_t* lut;    // EPI_QU8 activation table or null
  float ra, rb;          // residual add: rint((a-za)*ra + (b-zb)*rb) + zy
  int za, zb, zy;
  const uint16_t* bias_h;  // EPI_F16 bias (f16 bits) or null
  int kchunk;              // set by the launcher: k-steps per LDS weight chunk
  int tile_bc, tile_pb;    // tile choice (channels, 16-pixel blocks per wave); 0 = heuristic
  int tile_tpw;            // > 0: persistent kernel, pixel tiles per workgroup (small K only);
                           // -1: the streamed-weight kernel (long K); -2: the row-tile kernel;
                           // -3: the wide-tile kernel (c_in % 128 == 0); -4 / -5: the
                           // band-tile kernel with 8 / 16 waves (tile_pb: its band height)
  int band_rows;           // set by the launcher for the band-tile kernel
  // EPI_QU8 (table or plain requantize epilogues) and EPI_F16: a nearest
  // 2x upsample of the output written as well (the resize folded into its
  // producer): every output pixel's values also at its four pixels of this
  // view, (n, 2 ho, 2 wo, cout); null = none
  void* y_up;
  int up_pix_stride, up_c_off;
  int x_bytes;             // set by the launcher: bytes of the input view's buffer (< 2^31)
  float r_cin, r_kw, r_hwo, r_wo;  // set by the launcher: 1/cin, 1/kw, 1/(ho*wo), 1/wo
  int y_bytes, r_bytes;            // set by the launcher: bytes of the output and residual views
  // EPI_QU8 with a detect head's u8 -> f16 1x1 conv fused (h_wfrag set):
  // the u8 results (requantized, table) are not stored but feed that conv,
  // conv1x1_u8_f16's arithmetic, whose f16 outputs are (c_out <= BC)
  const uint16_t* h_wfrag;  // its weights in fragment order [cb][ks][64][8], or null
  const uint16_t* h_bias;   // f16 bias or null
  uint16_t* h_y;            // f16 output view
  int h_cout, h_y_pix_stride, h_y_c_off, h_act;
  float h_scale;            // the u8 results' quantization (the 1x1's input)
  int h_zp;
  // Two sibling convs (same input, same geometry) as one GEMM: the channels
  // from `split` on are the second conv's (its weights, bias' and
  // multipliers follow the first's), stored to their own output view y2
  // (u8: with their own table lut2); every channel tile lies wholly on one
  // side (split % channel tile == 0).  y2 null: one conv.
  void* y2;
  int y2_pix_stride, y2_c_off, split;
  const uint8_t* lut2;
  // EPI_QU8 with a table and a residual: the QLinearAdd's two scaled
  // operands as tables, [q] = f32((lut[q] - za) * ra) for the table input q,
  // [256 + b] = f32((b - zb) * rb), the products qadd_u8 rounds; set by the
  // host when every sum of two entries stays below 2^21 in magnitude (the
  // rounding add then rounds to the nearest even integer, as rintf does).
  // Null: qadd_u8.  Used by the chained-pair and C2f kernels.
  const float* rtab;
};

// Arguments of the direct convolution with the reference accumulation order.
struct DirectArgs {
  const void* x;
  const float* wf;  // HWIO weights as f32 (exact copies of the f16 weights)
  void* y;
  int n, h, w, cin, cout, kh, kw, sh, sw, pt, pl, ho, wo;
  int m;
  int x_pix_stride, x_c_off, y_pix_stride, y_c_off;
  int in_kind;   // 0 f32, 1 f16, 2 u8 dequantized to f16 ((q-zp)*scale),
                 // 3 NCHW f32 planes rounded to f16 (3x3 three-channel stem only)
  int out_kind;  // 0 f32, 1 f16, 2 u8 (QuantizeLinear of the f16 result)
  int act;
  const float* bias_f;     // f32 bias (out f32)
  const uint16_t* bias_h;  // f16 bias (out f16/u8)
  float in_scale; int in_zp;
  float out_scale; int out_zp;
  const uint8_t* lut;      // out u8: optional table applied after quantization
  int vec_out;             // set by the launcher: widest aligned store (16, 4 or 1 bytes)
  const float* bias_hf;    // optional: the f16 bias already widened with the reference decode
  float out_rcp;           // out u8: 1 / out_scale ...
  int out_fast;            // ... and 1 if x / out_scale may be computed as x*rcp plus one
                           // FMA correction (checked exhaustively on the host for every f16 x)
  int fast_epi;            // 1: out_fast holds, and the epilogue may widen its f16 values
                           // as IEEE f16 (the host checked that no subnormal changes a result)
  int x_bytes;             // set by the launcher for buffer-load paths: bytes of the input
  int epi_pk;              // 1 (f16 out): no f16 bias value is subnormal, so the bias pass
                           // may be a packed f16 add (results that round to f16 subnormals
                           // are checked in the kernel);
                           // 1 (u8 out): no f16 bias value is subnormal, out_fast holds and
                           // out_scale >= 2^-13, so the bias pass may be a packed f16 add
                           // and the quantization may widen as IEEE f16 (results that
                           // round to f16 subnormals are checked in the kernel)
  int out_plain;           // 1: rint(x * out_rcp) == rint(x / out_scale) for every finite f16 x
  const float* wq;         // optional (f32 input, c_in % 16 == 0, c_out % 4 == 0): the weights as
                           // [c_out / 4][kh * kw * c_in][4], for the tiled kernel
  const float* wq16;       // optional (1x1, c_out % 16 == 0): the weights as [c_out / 16][c_in][16],
                           // for the 1x1 kernel's 16-channel groups
  int w_finite;            // 1: every weight is finite (the host that holds them checked), so an
                           // out-of-image tap may be accumulated as +0 instead of skipped
};

// 1x1 convolution (stride 1, no padding) with u8 input dequantized to f16,
// on the fp16 matrix cores (k_conv1x1_f16.hip).
struct Conv1x1F16Args {
  const uint8_t* x;        // u8 input view
  const uint16_t* wfrag;   // f16 weights in fragment order [cout/16][ceil(cin/32)][64][8]
  const uint16_t* bias;    // f16 bias [cout] or null
  uint16_t* y;             // f16 output view
  int m, cin, cout;        // pixels, channels
  int x_pix_stride, x_c_off, y_pix_stride, y_c_off;
  float in_scale;
  int in_zp;
  uint32_t zp_bytes;       // in_zp in every byte (the value of K past c_in: dequantizes to 0)
  int act;
};

// A conv whose K (kh * kw * c_in) fits one fp16 MFMA k-step (the fp16
// graphs' three-channel stem; k_stem_f16.hip): f16 NHWC in (or the graph
// input's NCHW f32 planes, each value rounded to f16 as F16::from_f32 does)
// and f16 NHWC out, f16 weights in fragment order [cout / 16][64 lanes][8]
// (K zero-padded to 32).
struct StemF16Args {
  const uint16_t* x;
  const float* x_nchw;  // in_kind 3: dense NCHW f32 [n][cin][h][w], x unused
  int in_kind;          // 1: f16 NHWC view x, 3: x_nchw
  const uint16_t* wfrag;
  const uint16_t* bias;  // f16 bias [cout] or null
  uint16_t* y;
  int n, h, w, cin, ho, wo, kh, kw, sh, sw, pt, pl, cout, m;
  int x_pix_stride, x_c_off, y_pix_stride, y_c_off;
  int act;
};
bool stem_f16_supported(int cin, int kh, int kw, int cout, int wo, int sh, int sw);  // incl. LDS of a band
void launch_stem_f16(hipStream_t st, const StemF16Args& a);

// Rank-4 strided copy (k_shape.hip): y[y_off + sum i_k ys_k] =
// x[x_off + sum i_k xs_k] over 0 <= i_k < dims_k (elements).
struct StridedCopyArgs {
  const void* x;
  void* y;
  int esize;
  int f16_round_trip;  // f16: F16::from_f32(to_f32(v)) (the reference's f16 Transpose / Slice)
  long long dims[4];
  long long xs[4], ys[4];
  long long x_off, y_off;
};

// Broadcasting elementwise op (k_shape.hip): y over dims, every operand
// addressed by its own strides (0 along a broadcast axis).
enum BinOp : int { BIN_ADD = 0, BIN_SUB = 1, BIN_MUL = 2, BIN_DIV = 3 };
struct BinaryArgs {
  const void* a;
  const void* b;
  void* y;
  int op;
  int f16;
  long long dims[4];
  long long as[4], bs[4], ys[4];
  long long a_off, b_off, y_off;
};

// Unpadded NHWC average pool (k_shape.hip).
struct AvgPoolArgs {
  const void* x;
  void* y;
  int n, h, w, c, kh, kw, sh, sw, ho, wo;
  int f16;
};

// Depthwise convolution (channel multiplier 1).
struct DwArgs {
  const void* x;
  const void* wt;   // [kh][kw][c], same element type as x
  const void* bias; // [c] or null
  void* y;
  int n, h, w, c, kh, kw, sh, sw, pt, pl, ho, wo;
  int act;
  int x_pix_stride, x_c_off, y_pix_stride, y_c_off;
  int w_plain;  // 1: no f16 weight is subnormal (checked by whoever fills the struct)
};

// ---------------------------------------------------------------------------
// Kernel launchers (defined in the .hip files).  All enqueue on `st`.
// ---------------------------------------------------------------------------
// Packs HWIO weights (esize 1 or 2) into [ksteps][cout_pad][64B] rows.
void launch_pack_weights(hipStream_t st, const void* w_hwio, void* wpk, int K, int cout,
                         int cout_pad, int ksteps, int esize);
// bias_out[c] = (bias ? bias[c] : 0) + corr * sum_k w[k][c]   (int64 checked on host)
void launch_qconv_bias(hipStream_t st, const int8_t* w_hwio, const int* bias, int* bias_out, int K,
                       int cout, int corr);
// Implicit-GEMM convolution; selects a tile shape for the problem.
void launch_igemm(hipStream_t st, const IgemmArgs& a, int esize);
// Two chained 3x3 QLinearConvs (c -> c -> c, c = 16, 32 or 64, stride 1,
// padding 1; a1 writes what a2 reads, a2's residual is a1's input or none)
// in one launch, the intermediate in LDS, `rows` output rows per workgroup
// of 4 or 16 waves (k_igemm_pair.hip).  igemm_pair_rows lists the valid band
// heights.
bool igemm_pair_ok(const IgemmArgs& a1, const IgemmArgs& a2, int rows);
int igemm_pair_rows(const IgemmArgs& a1, const IgemmArgs& a2, int* rows, int max);
bool igemm_pair_lds_two_per_cu(const IgemmArgs& a1, int rows);  // LDS of the band <= 80 KB
void launch_igemm_pair(hipStream_t st, const IgemmArgs& a1, const IgemmArgs& a2, int rows, int waves = 4);
// A whole int8 C2f block with one bottleneck (k_igemm_c2f.hip): cv1 (1x1,
// c1 -> 2c), the bottleneck's two 3x3 convs (c -> c, the second with the
// shortcut or not) and cv2 (1x1, 3c -> 2c) in one launch, c = 16 or 32,
// the block's intermediates kept in LDS; R output rows per workgroup.
bool igemm_c2f_shapes_ok(const IgemmArgs& a0, const IgemmArgs& a1, const IgemmArgs& a2, const IgemmArgs& a3);
bool igemm_c2f_ok(const IgemmArgs& a0, const IgemmArgs& a1, const IgemmArgs& a2, const IgemmArgs& a3, int rows);
int igemm_c2f_rows(const IgemmArgs& a0, const IgemmArgs& a1, const IgemmArgs& a2, const IgemmArgs& a3, int* rows,
                   int max);
void launch_igemm_c2f(hipStream_t st, const IgemmArgs& a0, const IgemmArgs& a1, const IgemmArgs& a2,
                      const IgemmArgs& a3, int rows);
// Returns the tile name chosen for a problem (for launch descriptions).
const char* igemm_tile_name(const IgemmArgs& a, int esize);
// Channel-tile width used for `cout` output channels; packed weights must
// hold a multiple of it (cout_pad).
int igemm_channel_tile(int cout);
// Tile shapes launch_igemm can run for `a` (channel tile, pixel blocks per
// wave); returns how many were written (at most `max`).
int igemm_candidates(const IgemmArgs& a, int* bc, int* pb, int* tpw, int max);
// whether a sibling GEMM (a.y2 set) may run on channel tile bc of kernel
// family tpw (int8: staged 0, streamed -1, band -4 / -5; fp16: every family
// but the persistent small-K kernel)
bool igemm_sibling_tile_ok(const IgemmArgs& a, int bc, int tpw, int esize);

void launch_direct_conv(hipStream_t st, const DirectArgs& a);
// true if launch_direct_conv runs a on the padded-window stem kernel (3x3,
// stride 2, pad 1, three dense f16 channels in, u8 out, finite weights;
// DW_STEM_PAD=0 turns it off)
bool stem_pad_ok(const DirectArgs& a);
bool conv1x1_u8_f16_supported(int cin, int cout);
void launch_strided_copy(hipStream_t st, const StridedCopyArgs& a);
void launch_broadcast_binary(hipStream_t st, const BinaryArgs& a);
void launch_avgpool(hipStream_t st, const AvgPoolArgs& a);
void launch_conv1x1_u8_f16(hipStream_t st, const Conv1x1F16Args& a);
// HWIO f32 weights [rows][cout] -> [cout / 4][rows][4] (DirectArgs::wq)
void launch_repack_oc4(hipStream_t st, const float* w, float* wq, int rows, int cout);
void launch_dwconv(hipStream_t st, const DwArgs& a, int dtype);
// fp16 3x3 stride-1 depthwise on LDS row bands, packed f16 arithmetic (k_dwtile.hip)
bool dwconv3_tile_ok(const DwArgs& a);
bool dwconv3_tile_cfg_ok(const DwArgs& a, int units, int band_rows);
void launch_dwconv3_tile(hipStream_t st, const DwArgs& a, int units, int band_rows);

// Classifier-head ops (k_head.hip).  gemm: row-major C[m][n] = A[m][k] B[k][n]
// (dtype F32, F16 or I8 with an int32 C); global average pool over NHWC
// [n][hw][c] -> [n][c]; softmax over rows of n f32 values.
void launch_gemm(hipStream_t st, int dtype, const void* a, const void* b, void* c, int m, int n, int k);
// The graph runtime's Gemm (f32 / f16): trans_b takes B as [n][k] and sums
// with separate multiply and add, as the reference's transposed path does;
// bias (blen values, column j takes bias[j % blen]) is added after the sum
// is stored, as the reference's bias pass.
void launch_gemm_ex(hipStream_t st, int dtype, const void* a, const void* b, void* c, int m, int n, int k,
                    bool trans_b, const void* bias, int blen);
void launch_global_avg_pool(hipStream_t st, int dtype, const void* x, void* y, int n, int hw, int c);
void launch_softmax_rows(hipStream_t st, const float* x, float* y, int rows, int n);
void launch_softmax_rows_t(hipStream_t st, int dtype, const void* x, void* y, int rows, int n);

// QLinearGlobalAveragePool (u8 NHWC [n][hw][c] -> [n][c]) with
// m = (x_scale / y_scale) / hw; byte-matrix transpose (dst = src^T).
void launch_qlinear_gap(hipStream_t st, const uint8_t* x, uint8_t* y, int n, int hw, int c, int x_zp, float m,
                        int y_zp);
void launch_transpose_u8(hipStream_t st, const void* src, void* dst, int rows, int cols);

// Layout kernels (k_layout.hip): per batch entry dst[col][row] = src[row][col]
// (esize 1, 2 or 4); NCHW f32 -> NHWC f32 or f16 (rounded as F16::from_f32)
// into a view with pix_stride / c_off; fold_batchnorm on device weights.
void launch_transpose(hipStream_t st, const void* src, void* dst, int batch, int rows, int cols, int esize);
void launch_nchw_f32_to_nhwc(hipStream_t st, const float* src, void* dst, int n, int c, int hw, int out_dtype,
                             int pix_stride, int c_off);
void launch_fold_batchnorm(hipStream_t st, const float* w, const float* bias_in, const float* gamma,
                           const float* beta, const float* mean, const float* var, float eps, int c_out, int per,
                           float* w_out, float* b_out);

// YOLOv8 detect tail and post-processing (k_detect.hip).
// Detection as postprocess.rs:11-19 lays it out (24 bytes).
struct DwDetection {
  float bbox[4];
  uint32_t class_id;
  float confidence;
};
// Per-level NHWC head outputs [n][h][w][pix], 4 * reg_max box channels
// then nc class channels at the start of each pixel.
struct DetectTailArgs {
  const void* x[4];
  int h[4], w[4], pix[4];
  float stride[4];
  int levels, nc, reg_max;
};
void launch_detect_tail(hipStream_t st, int dtype, const DetectTailArgs& t, float* out, int n);
// Most candidates above the threshold one image may hold (LDS capacity of
// the per-image NMS workgroup); at most 16384 anchors per image.
constexpr int kPPMaxCandidates = 8704;
struct PostprocessArgs {
  const float* raw;
  int n, nc, A;
  float sx, sy, img_w, img_h, conf, iou;
  int agnostic, nmax;
  unsigned long long* keys;
  DwDetection* det;
  int* sorted_anchor;
  int* part_pos;
  DwDetection* out_det;
  int* out_pos;
  int* counts;
};
size_t pp_nms_lds_bytes(int nmax);
void launch_yolo_postprocess(hipStream_t st, const PostprocessArgs& a);

// Elementwise glue (count elements, contiguous).
enum EwOp : int {
  EW_RELU = 0, EW_ADD, EW_MUL, EW_SIGMOID, EW_SILU, EW_BIAS_ADD,
  EW_REQUANT_I32_I8, EW_QUANT_F32_I8, EW_DEQUANT_I8_F32, EW_ADD_I8, EW_RELU_I8,
  EW_QUANT_LINEAR_F16_U8, EW_DEQUANT_LINEAR_U8_F16, EW_QADD_U8, EW_LUT_U8,
  EW_F32_TO_F16, EW_F16_TO_F32, EW_CLIP
};
struct EwArgs {
  int op;
  int dtype;  // F32 or F16 for float ops
  const void* a;
  const void* b;
  void* y;
  size_t count;
  int c;  // bias channels
  float s0, s1, s2;
  int z0, z1, z2;
  const uint8_t* lut;
};
void launch_elementwise(hipStream_t st, const EwArgs& a);

// Strided-view versions used by the graph runtime (pixels x channels).
struct Ew2Args {
  int op;
  int dtype;
  View a, b, y;
  int pixels, channels;
  float s0, s1, s2;
  int z0, z1, z2;
  const uint8_t* lut;
};
void launch_elementwise2d(hipStream_t st, const Ew2Args& a);

// Max pool, padded windows, NHWC views.  dtype F32/F16/U8/I8.
struct PoolArgs {
  View x, y;
  int n, h, w, c, kh, kw, sh, sw, pt, pl, ho, wo;
};
void launch_maxpool(hipStream_t st, const PoolArgs& a, int dtype);
// SPPF cascade: y1 = pool(x), y2 = pool(y1), y3 = pool(y2) for a k x k,
// stride 1, pad k/2 pool, in one launch (windows of k, 2k-1, 3k-2).
void launch_maxpool_cascade3(hipStream_t st, const PoolArgs& a, View y2, View y3, int dtype);
// Nearest resize with the reference's index rule.
struct ResizeArgs {
  View x, y;
  int n, h, w, c, ho, wo;
};
void launch_resize_nearest(hipStream_t st, const ResizeArgs& a, int dtype);
// Channel copy between views (concat/split when aliasing is impossible).
void launch_copy_channels(hipStream_t st, View src, View dst, int pixels, int channels, int esize);
// Per-tensor min/max of an f32 view (calibration).  out: [min, max] floats,
// must be initialised to (+inf, -inf) by the caller (done by launch_minmax_init).
void launch_minmax_init(hipStream_t st, float* out);
void launch_minmax(hipStream_t st, View x, int pixels, int channels, float* out);

}  // namespace dw
