/*
 * dw_hip.h — C ABI of the MI355X (gfx950) execution backend for
 * dragonwing-edge-rs.
 *
 * Everything here is plain C: opaque handles, pointers, sizes and int status
 * codes.  No torch or HIP types cross this boundary.  Reference citations are
 * relative to the dragonwing-edge-rs source tree.
 *
 * Conventions
 *   - Every function returning `int` returns DW_OK (0) or a negative
 *     dw_status; the matching message is available from dw_last_error()
 *     (thread-local, valid until the next failing call on the same thread).
 *     This is the C form of dragonwing_core::Error::{Io,Unsupported,Backend}
 *     (crates/dragonwing-core/src/error.rs:13-20).
 *   - Buffers are byte spans; element types travel with the op call
 *     (crates/dragonwing-core/src/backend.rs:21-33).
 *   - All device work is queued on the backend's single HIP stream, in call
 *     order.  dw_hip_download synchronizes first; dw_hip_upload is complete on
 *     return (backend.rs:158-185).
 *   - Tensor layouts: activations NHWC ([N][H][W][C], C fastest); conv
 *     kernels HWIO ([kh][kw][c_in][c_out]) — the layout produced by
 *     convert_nchw_to_nhwc (crates/dragonwing-onnx/src/graph.rs:261-276).
 */
#ifndef DW_HIP_H
#define DW_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------ */
/* Status codes and errors                                                   */
/* ------------------------------------------------------------------------ */

typedef enum dw_status {
  DW_OK = 0,
  DW_ERR_BACKEND = -1,     /* Error::Backend(String): device/runtime failure */
  DW_ERR_UNSUPPORTED = -2, /* Error::Unsupported: op/shape/dtype not handled */
  DW_ERR_IO = -3,          /* Error::Io                                       */
  DW_ERR_INVALID = -4,     /* size mismatch / bad argument (Error::Backend)  */
  DW_ERR_RUNTIME = -5      /* dragonwing_onnx::Error::Runtime               */
} dw_status;

/* Message of the last failing call on this thread ("" if none). */
const char* dw_last_error(void);

/* ------------------------------------------------------------------------ */
/* Backend — replaces dragonwing_core::Backend for VulkanBackend             */
/* (crates/dragonwing-core/src/backend.rs:127-199,                          */
/*  crates/dragonwing-vulkan/src/lib.rs:246-292)                            */
/* ------------------------------------------------------------------------ */

typedef struct dw_hip_backend dw_hip_backend;
typedef struct dw_hip_buffer dw_hip_buffer;

/* BufferKind (backend.rs:89-101).  Only Storage exists. */
#define DW_BUFFER_STORAGE 0

/* Create a backend on HIP device `device` (one stream, default priority).
 * Counterpart of VulkanBackend::new (crates/dragonwing-vulkan/src/lib.rs). */
int dw_hip_backend_create(int device, dw_hip_backend** out);
/* Drop: frees the stream and every internal workspace.  Buffers must be freed
 * before their backend (backend.rs:75-79). */
void dw_hip_backend_destroy(dw_hip_backend* be);
/* Backend::name (backend.rs:142): "hip-gfx950". */
const char* dw_hip_backend_name(const dw_hip_backend* be);

/* Backend::alloc (backend.rs:146-156): contents unspecified; never shrinks. */
int dw_hip_alloc(dw_hip_backend* be, size_t len_bytes, int kind, dw_hip_buffer** out);
/* Drop for a buffer (explicit in C). NULL is ignored. */
void dw_hip_buffer_free(dw_hip_buffer* buf);
/* BackendBuffer::len_bytes (backend.rs:80-87). */
size_t dw_hip_buffer_len_bytes(const dw_hip_buffer* buf);
/* Device address of the buffer (for interop with other HIP code). */
void* dw_hip_buffer_device_ptr(const dw_hip_buffer* buf);

/* Backend::upload (backend.rs:158-173): len must equal len_bytes(dst),
 * otherwise DW_ERR_INVALID; complete on return. */
int dw_hip_upload(dw_hip_backend* be, dw_hip_buffer* dst, const void* src, size_t len);
/* Backend::download (backend.rs:175-185): len must equal len_bytes(src);
 * synchronizes the stream first. */
int dw_hip_download(dw_hip_backend* be, const dw_hip_buffer* src, void* dst, size_t len);
/* Backend::synchronize (backend.rs:187-198). */
int dw_hip_synchronize(dw_hip_backend* be);

/* ------------------------------------------------------------------------ */
/* Op functions.  Free functions taking the backend, as in                   */
/* dragonwing_vulkan::ops (crates/dragonwing-vulkan/src/ops.rs).  Buffer     */
/* sizes are validated exactly (ops.rs:2327-2346) and ops are queued on the  */
/* backend stream (no implicit sync).                                        */
/* ------------------------------------------------------------------------ */

/* Activation fused into an op's epilogue. */
#define DW_ACT_NONE 0
#define DW_ACT_RELU 1 /* ops::relu_f32 / relu_fp16 (ops.rs:189-220, 345-352) */
#define DW_ACT_SILU 2 /* sigmoid_fp16 then mul_fp16 (ops.rs:1881, 1959)     */

/* conv2d_f32_nhwc (crates/dragonwing-vulkan/src/ops.rs:1308; CPU
 * crates/dragonwing-cpu/src/ops.rs:1356-1436).  Direct convolution with the
 * reference's accumulation order (kh -> kw -> ic, one fused multiply-add per
 * term), so results are bit-identical to dragonwing-cpu.  Symmetric padding. */
int dw_hip_conv2d_f32_nhwc(dw_hip_backend* be, const dw_hip_buffer* input,
                           const dw_hip_buffer* kernel, dw_hip_buffer* output, size_t n,
                           size_t h_in, size_t w_in, size_t c_in, size_t c_out, size_t k_h,
                           size_t k_w, size_t stride_h, size_t stride_w, size_t pad_h,
                           size_t pad_w);

/* Conv2d + bias + activation, fp32: CpuGraphRuntime::dispatch_conv2d with
 * bias (crates/dragonwing-onnx/src/runtime.rs:1445-1460) followed by Relu
 * (runtime.rs:944-1002), fused in one launch.  `bias` may be NULL.
 * Bit-identical to the reference's op sequence. */
int dw_hip_conv2d_bias_act_f32_nhwc(dw_hip_backend* be, const dw_hip_buffer* input,
                                    const dw_hip_buffer* kernel, const dw_hip_buffer* bias,
                                    dw_hip_buffer* output, size_t n, size_t h_in, size_t w_in,
                                    size_t c_in, size_t c_out, size_t k_h, size_t k_w,
                                    size_t stride_h, size_t stride_w, size_t pad_h,
                                    size_t pad_w, int act);

/* conv2d_fp16_nhwc (vulkan ops.rs:1385; CPU ops.rs:1442-1500, _mt
 * :2572-2651), f16 storage (IEEE binary16 bits), then optional bias and
 * activation with the reference's f16 rounding points (runtime.rs:1483-1498,
 * ops.rs:1881-1967).  `exact`=1 uses the reference accumulation order
 * (bit-identical); `exact`=0 uses the fp16 MFMA implicit-GEMM kernel
 * (fp32 accumulation in another order: within fp16 tolerance).
 * MFMA path requires c_in % 8 == 0, c_out % 4 == 0 and k_h*k_w <= 31. */
int dw_hip_conv2d_bias_act_f16_nhwc(dw_hip_backend* be, const dw_hip_buffer* input,
                                    const dw_hip_buffer* kernel, const dw_hip_buffer* bias,
                                    dw_hip_buffer* output, size_t n, size_t h_in, size_t w_in,
                                    size_t c_in, size_t c_out, size_t k_h, size_t k_w,
                                    size_t stride_h, size_t stride_w, size_t pad_h,
                                    size_t pad_w, int act, int exact);

/* depthwise_conv2d_fp16_nhwc_mt (crates/dragonwing-cpu/src/ops.rs:2819-2933)
 * with channel_multiplier 1, then bias and activation as in
 * CpuGraphRuntime (runtime.rs:1467-1498).  kernel: [k_h][k_w][c] f16,
 * bias: [c] f16 or NULL.  Requires c % 4 == 0 for a 3x3 kernel with
 * stride_w 1 or 2, else c % 8 == 0. */
int dw_hip_depthwise_conv2d_f16_nhwc(dw_hip_backend* be, const dw_hip_buffer* input,
                                     const dw_hip_buffer* kernel, const dw_hip_buffer* bias,
                                     dw_hip_buffer* output, size_t n, size_t h_in, size_t w_in,
                                     size_t c, size_t k_h, size_t k_w, size_t stride_h,
                                     size_t stride_w, size_t pad_h, size_t pad_w, int act);

/* depthwise_conv2d_f32_nhwc_mt (ops.rs:2734-2815) + bias + activation. */
int dw_hip_depthwise_conv2d_f32_nhwc(dw_hip_backend* be, const dw_hip_buffer* input,
                                     const dw_hip_buffer* kernel, const dw_hip_buffer* bias,
                                     dw_hip_buffer* output, size_t n, size_t h_in, size_t w_in,
                                     size_t c, size_t k_h, size_t k_w, size_t stride_h,
                                     size_t stride_w, size_t pad_h, size_t pad_w, int act);

/* QLinearConv u8 x s8 -> u8 (ONNX QLinearConv; no counterpart in the
 * reference, whose INT8 is symmetric s8 — it generalises
 * conv2d_requant_relu_i8_packed, crates/dragonwing-vulkan/src/ops.rs:2294).
 *   acc[c]  = sum (x - x_zp) * w[c] + bias[c]          (int32, exact)
 *   y       = clamp(rint((float)acc * M[c]) + y_zp, 0, 255)
 *   M[c]    = (x_scale * w_scales[c]) / y_scale         (f32)
 * rint rounds half to even.  Padding uses the zero point (real 0).
 * input u8 NHWC, kernel s8 HWIO, bias int32[c_out] device buffer or NULL,
 * w_scales: host array of c_out floats.  Requires c_in % 16 == 0,
 * c_out % 4 == 0 and k_h*k_w <= 31.  INT8 MFMA implicit GEMM
 * (v_mfma_i32_16x16x64_i8). */
int dw_hip_qlinearconv_u8s8(dw_hip_backend* be, const dw_hip_buffer* input,
                            const dw_hip_buffer* kernel, const dw_hip_buffer* bias,
                            dw_hip_buffer* output, size_t n, size_t h_in, size_t w_in,
                            size_t c_in, size_t c_out, size_t k_h, size_t k_w, size_t stride_h,
                            size_t stride_w, size_t pad_h, size_t pad_w, float x_scale,
                            int x_zp, const float* w_scales, float y_scale, int y_zp);

/* dw_hip_qlinearconv_u8s8 without any device allocation.  No counterpart in
 * the reference: for callers that cannot allocate device memory (tight
 * serving loops, hosts that forbid hipMalloc).  The
 * per-call data the other entry point keeps in grow-only workspaces (packed
 * weights, per-channel multipliers, bias') goes to a fixed 8 MiB scratch
 * array per device instead, set up when the backend is created: c_out at
 * most 4096 and packed weights (ceil(k_h*k_w*c_in / 64) * c_out rounded up
 * to the channel tile * 64 bytes) at most 8 MiB - 32 KiB, else
 * DW_ERR_UNSUPPORTED.  Same arguments, results and errors as
 * dw_hip_qlinearconv_u8s8.  Every call on a device shares that device's
 * scratch; calls through different backends (streams) on one device are
 * ordered on it (each call's stream waits for the previous call's last
 * launch).  Not capturable: the per-channel scales are copied from the
 * caller's host array and the call waits for that copy. */
int dw_hip_qlinearconv_u8s8_noalloc(dw_hip_backend* be, const dw_hip_buffer* input,
                                    const dw_hip_buffer* kernel, const dw_hip_buffer* bias,
                                    dw_hip_buffer* output, size_t n, size_t h_in, size_t w_in,
                                    size_t c_in, size_t c_out, size_t k_h, size_t k_w,
                                    size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w,
                                    float x_scale, int x_zp, const float* w_scales, float y_scale,
                                    int y_zp);

/* conv2d_i8_nhwc (crates/dragonwing-cpu/src/ops.rs:3086-3142): s8 x s8 ->
 * int32 accumulator, zero padding.  Requires c_in % 16 == 0, c_out % 4 == 0,
 * k_h*k_w <= 31. */
int dw_hip_conv2d_i8_nhwc(dw_hip_backend* be, const dw_hip_buffer* input,
                          const dw_hip_buffer* kernel, dw_hip_buffer* output_i32, size_t n,
                          size_t h_in, size_t w_in, size_t c_in, size_t c_out, size_t k_h,
                          size_t k_w, size_t stride_h, size_t stride_w, size_t pad_h,
                          size_t pad_w);

/* conv2d_requant_relu_i8_packed (crates/dragonwing-vulkan/src/ops.rs:2294-2430)
 * with the CPU semantics it stands for: conv2d_i8_nhwc, then
 * requantize_i32_to_i8 (ops.rs:3380-3386: clamp to [-128,127], round half
 * away from zero), then relu_i8 when do_relu.  One per-tensor scale. */
int dw_hip_conv2d_requant_relu_i8(dw_hip_backend* be, const dw_hip_buffer* input,
                                  const dw_hip_buffer* kernel, dw_hip_buffer* output, size_t n,
                                  size_t h_in, size_t w_in, size_t c_in, size_t c_out, size_t k_h,
                                  size_t k_w, size_t stride_h, size_t stride_w, size_t pad_h,
                                  size_t pad_w, float requant_scale, int do_relu);

/* Elementwise ops.  `count` elements; all buffers exactly count*esize. */
int dw_hip_relu_f32(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t count);      /* ops.rs:189-220  */
int dw_hip_relu_fp16(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t count);     /* ops.rs:345-352  */
int dw_hip_add_f32(dw_hip_backend* be, const dw_hip_buffer* a, const dw_hip_buffer* b, dw_hip_buffer* y, size_t count);  /* ops.rs:363-384 */
int dw_hip_add_fp16(dw_hip_backend* be, const dw_hip_buffer* a, const dw_hip_buffer* b, dw_hip_buffer* y, size_t count); /* ops.rs:434-442 */
int dw_hip_mul_f32(dw_hip_backend* be, const dw_hip_buffer* a, const dw_hip_buffer* b, dw_hip_buffer* y, size_t count);  /* ops.rs:1899-1919 */
int dw_hip_mul_fp16(dw_hip_backend* be, const dw_hip_buffer* a, const dw_hip_buffer* b, dw_hip_buffer* y, size_t count); /* ops.rs:1959-1967 */
int dw_hip_sigmoid_f32(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t count);   /* ops.rs:1852-1870 */
int dw_hip_sigmoid_fp16(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t count);  /* ops.rs:1881-1888 */
/* silu_f32 (crates/dragonwing-vulkan/src/ops.rs:2214): x * sigmoid(x). */
int dw_hip_silu_f32(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t count);
/* Sigmoid then Mul in f16 with both f16 roundings (the unfused CPU pair). */
int dw_hip_silu_fp16(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t count);
/* bias_add_f32_nhwc (vulkan ops.rs:2432): y[i] += bias[i % c], in place. */
int dw_hip_bias_add_f32_nhwc(dw_hip_backend* be, dw_hip_buffer* y, const dw_hip_buffer* bias, size_t count, size_t c);

/* INT8 (reference symmetric scheme, zero point 0, round half away). */
int dw_hip_requantize_i32_to_i8(dw_hip_backend* be, const dw_hip_buffer* x_i32, dw_hip_buffer* y_i8, size_t count, float requant_scale); /* ops.rs:3380-3386 */
int dw_hip_quantize_f32_to_i8(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y_i8, size_t count, float scale);           /* ops.rs:3503-3525 */
int dw_hip_dequantize_i8_to_f32(dw_hip_backend* be, const dw_hip_buffer* x_i8, dw_hip_buffer* y, size_t count, float scale);         /* ops.rs:3439-3457 */
int dw_hip_add_i8(dw_hip_backend* be, const dw_hip_buffer* a, const dw_hip_buffer* b, dw_hip_buffer* y, size_t count, float scale_a_over_y, float scale_b_over_y); /* ops.rs:3176-3209 */
int dw_hip_relu_i8(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t count); /* ops.rs:3301-3320 */

/* ONNX-style u8 quantization (zero point, round half to even). */
/* QuantizeLinear: y = clamp(rint(x / scale) + zp, 0, 255), x f16. */
int dw_hip_quantize_linear_f16_u8(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t count, float scale, int zp);
/* DequantizeLinear: y = f16((float)(q - zp) * scale). */
int dw_hip_dequantize_linear_u8_f16(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t count, float scale, int zp);
/* QLinearAdd: y = clamp(rint((a-za)*(sa/sy) + (b-zb)*(sb/sy)) + zy, 0, 255). */
int dw_hip_qlinear_add_u8(dw_hip_backend* be, const dw_hip_buffer* a, const dw_hip_buffer* b, dw_hip_buffer* y, size_t count,
                          float a_scale, int a_zp, float b_scale, int b_zp, float y_scale, int y_zp);
/* y = lut[x] for a 256-entry host table (quantized activations such as SiLU). */
int dw_hip_lut_u8(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t count, const uint8_t* lut256);

/* Data-movement glue, NHWC.  dtype: DW_DTYPE_* element type. */
#define DW_DTYPE_F32 0
#define DW_DTYPE_F16 1
#define DW_DTYPE_I8 2
#define DW_DTYPE_U8 3
#define DW_DTYPE_I32 4

/* maxpool2d_f32_nhwc (ops.rs:1513-1552), extended with padding: padded
 * positions never win (ONNX MaxPool; the reference ignores pads,
 * runtime.rs:902-904).  pads = top, left, bottom, right. */
int dw_hip_maxpool2d_nhwc(dw_hip_backend* be, int dtype, const dw_hip_buffer* x, dw_hip_buffer* y,
                          size_t n, size_t h_in, size_t w_in, size_t c, size_t pool_h,
                          size_t pool_w, size_t stride_h, size_t stride_w, size_t pad_t,
                          size_t pad_l, size_t pad_b, size_t pad_r);
/* resize_f32 Nearest (ops.rs:2320-2351): ih = clamp(round((oh+0.5)*h_in/h_out - 0.5)). */
int dw_hip_resize_nearest_nhwc(dw_hip_backend* be, int dtype, const dw_hip_buffer* x, dw_hip_buffer* y,
                               size_t n, size_t h_in, size_t w_in, size_t h_out, size_t w_out, size_t c);
/* concat_fp16 / concat_f32 along axis 3 (ops.rs:2248-2299). */
int dw_hip_concat_channels_nhwc(dw_hip_backend* be, int dtype, const dw_hip_buffer* const* inputs,
                                const size_t* channels, size_t num_inputs, dw_hip_buffer* y,
                                size_t pixels);
/* split_f32 along axis 3 (ops.rs:2407-2456). */
int dw_hip_split_channels_nhwc(dw_hip_backend* be, int dtype, const dw_hip_buffer* x,
                               dw_hip_buffer* const* outputs, const size_t* channels,
                               size_t num_outputs, size_t pixels);

/* Classifier-head ops.  Row-major, sizes must match exactly. */
/* gemm_f32 (dragonwing-vulkan ops.rs:437; CPU gemm_f32_naive ops.rs:273-290 and
 * gemm_f32_mt :1659-1707): c[m][n] = a[m][k] b[k][n], fma chain over k in order. */
int dw_hip_gemm_f32(dw_hip_backend* be, const dw_hip_buffer* a, const dw_hip_buffer* b, dw_hip_buffer* c,
                    size_t m, size_t n, size_t k);
/* gemm_fp16 (dragonwing-vulkan ops.rs:1184; CPU ops.rs:461-479, :1709-1749): f16 in
 * and out, F16::to_f32 operands, f32 fma chain, F16::from_f32 of the sum. */
int dw_hip_gemm_fp16(dw_hip_backend* be, const dw_hip_buffer* a, const dw_hip_buffer* b, dw_hip_buffer* c,
                     size_t m, size_t n, size_t k);
/* gemm_i8 (CPU ops.rs:2964-2995; the Vulkan gemm_i8_packed ops.rs:1723 takes
 * pre-packed operands): i8 x i8 -> int32 sums. */
int dw_hip_gemm_i8(dw_hip_backend* be, const dw_hip_buffer* a, const dw_hip_buffer* b, dw_hip_buffer* c_i32,
                   size_t m, size_t n, size_t k);
/* GlobalAveragePool, NHWC [n][h][w][c] -> [n][c] (CpuGraphRuntime::
 * dispatch_global_avg_pool, dragonwing-onnx runtime.rs:1109-1175): f32 sum over
 * rows then columns, divided by h*w; dtype F32 or F16. */
int dw_hip_global_avg_pool_nhwc(dw_hip_backend* be, int dtype, const dw_hip_buffer* x, dw_hip_buffer* y,
                                size_t n, size_t h, size_t w, size_t c);
/* softmax_f32 over rows of n (dragonwing-vulkan ops.rs:1519; CPU ops.rs:1609-1638):
 * max subtraction, exp, sum, multiply by 1/sum.  exp is the device's: outputs
 * agree with the CPU to a few ulps. */
int dw_hip_softmax_f32(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t rows, size_t n);

/* Layout transposes on the device (transpose_nchw_to_nhwc /
 * transpose_nhwc_to_nchw, crates/dragonwing-onnx/src/graph.rs:339-379):
 * elements of dtype (any DW_DTYPE_*) moved, never converted. */
int dw_hip_transpose_nchw_to_nhwc(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t n, size_t c,
                                  size_t h, size_t w, int dtype);
int dw_hip_transpose_nhwc_to_nchw(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t n, size_t h,
                                  size_t w, size_t c, int dtype);

/* fold_batchnorm (graph.rs:521-690) on device-resident f32 weights: w is
 * [c_out][per_channel] (OIHW), bias_in optional; in f64 per channel
 * s = gamma / sqrt(var + eps), w_out = (f32)(w * s),
 * bias_out = (f32)((bias_in - mean) * s + beta). */
int dw_hip_fold_batchnorm(dw_hip_backend* be, const dw_hip_buffer* w, const dw_hip_buffer* bias_in,
                          const dw_hip_buffer* gamma, const dw_hip_buffer* beta, const dw_hip_buffer* mean,
                          const dw_hip_buffer* var, float epsilon, size_t c_out, size_t per_channel,
                          dw_hip_buffer* w_out, dw_hip_buffer* bias_out);

/* QGemm u8 x s8 -> u8 (the quantized classifier head; no counterpart in the
 * reference, whose INT8 Gemm is symmetric s8 with a Requantize after it,
 * quantize.rs:225-260): A [m][k] u8 (zero point a_zp, scale a_scale), B s8
 * [k][n] or, with trans_b, [n][k] (per-column scales b_scales[n], zero
 * point 0), optional int32 bias [n] (scale a_scale * b_scales[j]);
 * acc = sum_p (A[i][p] - a_zp) * B[p][j] + bias[j],
 * Y[i][j] = clamp(rint((float)acc * M[j]) + y_zp, 0, 255),
 * M[j] = a_scale * b_scales[j] / y_scale in f32, rint half to even: the
 * QLinearConv definition on a 1x1 kernel (same MFMA kernels).  Needs
 * k % 16 == 0 and n % 4 == 0. */
int dw_hip_qgemm_u8s8(dw_hip_backend* be, const dw_hip_buffer* a, const dw_hip_buffer* b, const dw_hip_buffer* bias,
                      dw_hip_buffer* y, size_t m, size_t n, size_t k, int trans_b, float a_scale, int a_zp,
                      const float* b_scales, float y_scale, int y_zp);

/* QLinearGlobalAveragePool over NHWC u8 (the quantized form of
 * dispatch_global_avg_pool, onnx runtime.rs:1109-1175): per image and
 * channel, acc = sum (x - x_zp) in int32, y = clamp(rint((float)acc * M) +
 * y_zp, 0, 255) with M = (x_scale / y_scale) / (h * w) in f32. */
int dw_hip_qlinear_global_avg_pool_u8(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t n,
                                      size_t h, size_t w, size_t c, float x_scale, int x_zp, float y_scale,
                                      int y_zp);

/* YOLOv8 detect tail: the exported graph's ops after the head convs
 * (ultralytics Detect: DFL softmax over each side's reg_max bins and the 1x1
 * expectation, dist2bbox, times the level stride, sigmoid of the classes),
 * as the reference's f32 ops compute them (softmax_f32 ops.rs:1609-1638,
 * conv2d_f32 ops.rs:1356-1436, sigmoid_f32 ops.rs:1866-1870).  levels[i]:
 * NHWC [n][h[i]][w[i]][4*reg_max + nc] head outputs of element type dtype
 * (DW_DTYPE_F16 or DW_DTYPE_F32); out: [n][4 + nc][A] f32, A = sum h*w,
 * anchors level by level in row-major order.  exp is the device's. */
int dw_hip_yolo_detect_tail(dw_hip_backend* be, int dtype, const dw_hip_buffer* const* levels, const int* h,
                            const int* w, const float* strides, int num_levels, size_t n, int nc, int reg_max,
                            dw_hip_buffer* out);

/* Detection (crates/dragonwing-onnx/src/postprocess.rs:11-19). */
typedef struct dw_detection {
  float bbox[4]; /* x1, y1, x2, y2 in image pixels */
  uint32_t class_id;
  float confidence;
} dw_detection;

/* postprocess_yolo (postprocess.rs:279-305) for each of n images of raw
 * [n][4 + nc][A] f32 on the device: decode_detections_v8 (:78-146), then
 * nms (:214-243), or nms_agnostic (:245-277) when agnostic is nonzero.
 * Results are the reference's, in its order (stable sort by confidence,
 * greedy suppression, swap_remove of the suppressed entries).  out holds
 * cap detections per image (image b at out + b * cap); counts[b] receives
 * image b's number of detections.  DW_ERR_INVALID if one exceeds cap;
 * DW_ERR_UNSUPPORTED above 16384 anchors per image or 8704 candidates
 * over the threshold in one image.  Synchronous (results on the host). */
int dw_hip_yolo_postprocess(dw_hip_backend* be, const dw_hip_buffer* raw, size_t n, int nc, size_t num_det,
                            uint32_t img_w, uint32_t img_h, float conf_threshold, float iou_threshold,
                            int agnostic, dw_detection* out, size_t cap, size_t* counts);

/* ------------------------------------------------------------------------ */
/* Graph IR — the C form of dragonwing_onnx::Graph / CompiledOp / OpParams   */
/* (crates/dragonwing-onnx/src/graph.rs:18-31, builder.rs:204-361), plus the */
/* compiler passes that produce the graphs this backend runs.               */
/* ------------------------------------------------------------------------ */

typedef struct dw_graph dw_graph;

/* OpParams discriminants (builder.rs:219-361), then this backend's
 * quantized-ONNX extensions (no counterpart in the reference). */
typedef enum dw_op_kind {
  DW_OP_NONE = 0,        /* OpParams::None: op_type decides (Relu, SiLU, ...) */
  DW_OP_CONV2D = 1,      /* OpParams::Conv2d                                  */
  DW_OP_ADD = 2,         /* OpParams::Add                                     */
  DW_OP_MUL = 3,         /* OpParams::Mul                                     */
  DW_OP_SIGMOID = 4,     /* OpParams::Sigmoid                                 */
  DW_OP_MAXPOOL = 5,     /* OpParams::MaxPool                                 */
  DW_OP_CONCAT = 6,      /* OpParams::Concat                                  */
  DW_OP_SPLIT = 7,       /* OpParams::Split                                   */
  DW_OP_RESIZE = 8,      /* OpParams::Resize                                  */
  DW_OP_BATCHNORM = 9,   /* ONNX BatchNormalization before fold_batchnorm     */
  DW_OP_REQUANTIZE = 10, /* OpParams::Requantize                              */
  DW_OP_ADD_QUANTIZED = 11, /* OpParams::AddQuantized                         */
  DW_OP_QUANTIZE = 12,   /* OpParams::Quantize                                */
  DW_OP_DEQUANTIZE = 13, /* OpParams::Dequantize                              */
  DW_OP_CONV2D_REQUANT_RELU_I8 = 14, /* OpParams::Conv2dRequantReluI8Nhwc     */
  DW_OP_GEMM = 15,       /* OpParams::Gemm (alpha, beta, trans_a, trans_b)    */
  DW_OP_GLOBAL_AVG_POOL = 16, /* OpParams::GlobalAvgPool                      */
  DW_OP_SOFTMAX = 17,    /* OpParams::Softmax { axis } (axis = last dim only)  */
  DW_OP_CLIP = 18,       /* OpParams::Clip { min, max }                        */
  DW_OP_RESHAPE = 19,    /* OpParams::Reshape (the output tensor's dims)       */
  DW_OP_AVGPOOL = 20,    /* OpParams::AvgPool { kernel_shape, strides, pads }  */
  DW_OP_SUB = 21,        /* OpParams::Sub                                      */
  DW_OP_DIV = 22,        /* OpParams::Div                                      */
  DW_OP_TRANSPOSE = 23,  /* OpParams::Transpose { perm }                       */
  DW_OP_SLICE = 24,      /* OpParams::Slice { starts, ends, axes, steps }      */
  /* extensions */
  DW_OP_QLINEAR_CONV = 32,  /* QLinearConv (+ fused LUT activation, + QLinearAdd residual) */
  DW_OP_QUANTIZE_LINEAR = 33,
  DW_OP_DEQUANTIZE_LINEAR = 34,
  DW_OP_QLINEAR_ADD = 35,
  DW_OP_QLINEAR_LUT = 36,   /* quantized elementwise activation by 256-entry table */
  DW_OP_YOLO_DETECT = 37    /* YOLOv8 detect tail (dw_hip_yolo_detect_tail): inputs the
                             * per-level head outputs, output [n][4 + nc][A] f32 */
} dw_op_kind;

typedef struct dw_op_params {
  int kind;                 /* dw_op_kind                                      */
  int kernel_shape[2];      /* Conv2d / MaxPool: [H, W]                        */
  int strides[2];
  int pads[4];              /* [top, left, bottom, right]                      */
  int dilations[2];
  int group;
  int axis;                 /* Concat / Split                                 */
  int split_sizes[8];       /* Split                                          */
  int num_splits;
  int out_h, out_w;         /* Resize                                          */
  int mode_nearest;         /* Resize: 1 = "nearest", 0 = "linear"            */
  float scale;              /* Requantize/Quantize/Dequantize scale; Conv2dRequantReluI8 requant_scale */
  float scale_a_over_out;   /* AddQuantized                                   */
  float scale_b_over_out;
  int has_relu;             /* Conv2dRequantReluI8Nhwc                        */
  float epsilon;            /* BatchNormalization                             */
  int act;                  /* QLinearLUT: DW_ACT_* the table encodes         */
  float alpha, beta;        /* Gemm (carried; the reference's runtime ignores them) */
  int trans_a, trans_b;     /* Gemm                                           */
  float clip_min, clip_max; /* Clip                                           */
  int reg_max;              /* YoloDetect: DFL bins per box side               */
  float level_strides[4];   /* YoloDetect: stride of each input level          */
  int perm[4];              /* Transpose: output axis k is input axis perm[k]  */
  int num_slice_axes;       /* Slice: entries used in the four arrays below    */
  int slice_axes[4];        /* Slice: axis of each entry                       */
  int slice_starts[4];      /* Slice: first index (resolved: 0 <= start <= dim) */
  int slice_ends[4];        /* Slice: end index (resolved: start <= end <= dim) */
  int slice_steps[4];       /* Slice: step (>= 1)                              */
} dw_op_params;

/* sizeof(dw_op_params) as compiled into the library.  A binding that declares
 * its own copy of the struct (ctypes, Rust #[repr(C)]) checks its size
 * against this before passing one to dw_graph_add_op, which copies the whole
 * struct.  No counterpart in the reference (layout check for FFI callers). */
size_t dw_op_params_size(void);

/* ONNX model loading (crates/dragonwing-onnx/src/proto.rs:129-271,
 * model.rs:324-707; op builders builder.rs:386-420).  dw_graph_from_onnx
 * parses a serialized ModelProto (opset 12 to 20) and builds an F32 graph in
 * ONNX's NCHW layout, ready for dw_graph_fold_batchnorm,
 * dw_graph_convert_nchw_to_nhwc and the rest.  Ops: Conv, Relu, Sigmoid,
 * Clip, Add, Sub, Mul, Div (ONNX broadcasting), MaxPool, AveragePool
 * (unpadded), Concat, Split, Slice, Transpose, Resize / Upsample (nearest,
 * constant scales or sizes), BatchNormalization, GlobalAveragePool,
 * Flatten, Reshape, Squeeze / Unsqueeze (as Reshape), Softmax, Gemm,
 * MatMul, Constant, Identity, Cast of a float activation to float; Shape,
 * Gather, Unsqueeze, Squeeze, Concat, Cast and Add / Sub / Mul / Div of
 * constants are folded into constants (the shape arithmetic of
 * unsimplified exports); a constant zero spatial Pad read by a Conv is
 * folded into the Conv's pads.  A QDQ model (QuantizeLinear / DequantizeLinear, u8 activations,
 * symmetric s8 weights, int32 biases) loads as the float graph with its
 * quantization fixed, which dw_graph_quantize_qdq then uses as given (no
 * calibration).  dw_onnx_inspect writes a JSON summary of the parsed model
 * (nodes, attributes, initializers, inputs, outputs) into buf (cap bytes);
 * *need receives the size it takes. */
int dw_graph_from_onnx(const void* bytes, size_t len, dw_graph** out);
int dw_onnx_inspect(const void* bytes, size_t len, char* buf, size_t cap, size_t* need);

/* Graph dtypes (dragonwing_core::Dtype subset, crates/dragonwing-core/src/dtype.rs). */
#define DW_GRAPH_F32 0
#define DW_GRAPH_F16 1
#define DW_GRAPH_I8 2  /* Dtype::I8: the reference's symmetric INT8 form      */
                       /* (QuantizedGraphCompiler, quantize.rs:73-368)        */
#define DW_GRAPH_QU8 3 /* quantized: u8 activations with zero points (QDQ-folded) */

int dw_graph_create(int dtype, dw_graph** out);
void dw_graph_destroy(dw_graph* g);
/* Declare a tensor: name, shape (rank <= 4), element dtype (DW_DTYPE_*). */
int dw_graph_add_tensor(dw_graph* g, const char* name, const int64_t* dims, int rank, int dtype);
/* Attach initializer bytes to a declared tensor (weights, biases, BN params). */
int dw_graph_set_initializer(dw_graph* g, const char* name, const void* data, size_t len);
/* Quantization parameters of a u8 tensor: real = (q - zero_point) * scale
 * (the x_scale/x_zero_point inputs of an ONNX QLinearConv). */
int dw_graph_set_quant(dw_graph* g, const char* name, float scale, int zero_point);
/* Per-output-channel scales of an s8 weight tensor (zero point 0). */
int dw_graph_set_channel_scales(dw_graph* g, const char* name, const float* scales, size_t count);
/* Append a CompiledOp.  Empty-string inputs are optional-absent. */
int dw_graph_add_op(dw_graph* g, const char* name, const char* op_type, const char* const* inputs,
                    int num_inputs, const char* const* outputs, int num_outputs,
                    const dw_op_params* params);
int dw_graph_set_io(dw_graph* g, const char* const* inputs, int num_inputs,
                    const char* const* outputs, int num_outputs);

/* Passes (crates/dragonwing-onnx/src/graph.rs, fusion.rs, quantize.rs). */
int dw_graph_fold_batchnorm(dw_graph* g);         /* graph.rs:521-690 (f64 math)   */
int dw_graph_convert_nchw_to_nhwc(dw_graph* g);   /* graph.rs:248-290              */
/* apply_fusion_passes (fusion.rs:42-348), all three passes on one snapshot
 * of the op list: 1. Conv + Relu -> Conv "<conv>_fused_relu" writing the
 * Relu's output, with has_relu = 1 (the reference drops the ReLU there; here
 * the flag keeps it); 2. Sigmoid + Mul -> SiLU "<mul>_silu" (either Mul
 * operand order); 3. INT8 Conv + Requantize (+ Relu) -> Conv2dRequantReluI8.
 * *num_fused receives the number of fused ops written. */
int dw_graph_apply_fusion_passes(dw_graph* g, int* num_fused);
int dw_graph_convert_to_f16(dw_graph* g);          /* runtime.rs:800-811: f32 initializers -> F16 RNE */

/* Calibration statistics (calibration.rs:56-69) and the QDQ quantizer that
 * turns an F32 graph into a DW_GRAPH_QU8 graph of QLinearConv ops. */
int dw_graph_set_activation_range(dw_graph* g, const char* name, float min_v, float max_v);
int dw_graph_quantize_qdq(dw_graph* g, const char* const* keep_f16_ops, int num_keep);
/* Calibrator::new + feed + compute_params (calibration.rs:90-260) on the GPU:
 * runs the F32 NHWC graph over `num_images` images (host f32, NHWC, each
 * floats_per_image values; a multiple of the graph batch), records per-tensor
 * min/max and stores the ranges in the graph. */
int dw_hip_calibrate(dw_hip_backend* be, dw_graph* g, const char* input_name, const float* images,
                     size_t floats_per_image, int num_images);

/* Introspection (for oracles and tools): JSON text describing dtype, tensors,
 * ops, params and quantization parameters.  The string stays valid until the
 * graph is modified or destroyed. */
const char* dw_graph_to_json(dw_graph* g);
/* Initializer bytes of a tensor (NULL/0 if none). */
int dw_graph_get_initializer(dw_graph* g, const char* name, const void** data, size_t* len);

/* ------------------------------------------------------------------------ */
/* Graph runtime — VulkanGraphRuntime's API                                  */
/* (crates/dragonwing-onnx/src/vulkan_runtime.rs:115-469, :2113-2141).      */
/* ------------------------------------------------------------------------ */

typedef struct dw_hip_graph_runtime dw_hip_graph_runtime;

/* VulkanGraphRuntime::new: plans device memory, packs weights, builds the
 * launch list.  The graph is copied; it can be destroyed afterwards. */
int dw_hip_graph_runtime_create(dw_hip_backend* be, const dw_graph* g, dw_hip_graph_runtime** out);
/* dw_hip_graph_runtime_create with plan options (flags 0: the same plan).
 * DW_RT_EXACT_U8_F16_CONV: convs that read u8 activations (dequantized to
 * f16) and write f16 -- the fp16 layers of a QDQ graph after its int8 part,
 * e.g. a detect head's last 1x1 convs -- run in dragonwing-cpu's
 * accumulation order, bit-identical to CpuGraphRuntime, instead of on the
 * fp16 matrix cores (results within the fp16 tolerance).  The INT8 layers
 * are bit-exact either way.  Unknown flags: DW_ERR_INVALID. */
#define DW_RT_EXACT_U8_F16_CONV 1u
/* DW_RT_EXACT_F16_DEPTHWISE: fp16 depthwise convs in dragonwing-cpu's
 * accumulation order (an f32 fma chain, bit-identical before the
 * activation) instead of the packed-f16 band kernel (fp16 tolerance). */
#define DW_RT_EXACT_F16_DEPTHWISE 2u
int dw_hip_graph_runtime_create_ex(dw_hip_backend* be, const dw_graph* g, unsigned flags,
                                   dw_hip_graph_runtime** out);
void dw_hip_graph_runtime_destroy(dw_hip_graph_runtime* rt);
/* set_input_f32 (vulkan_runtime.rs:238): converts to the graph dtype (F16 RNE). */
int dw_hip_graph_set_input_f32(dw_hip_graph_runtime* rt, const char* name, const float* data, size_t count);
/* set_input_bytes (vulkan_runtime.rs:2113): raw bytes in the tensor's dtype. */
int dw_hip_graph_set_input_bytes(dw_hip_graph_runtime* rt, const char* name, const void* data, size_t len);
/* An input given in NCHW f32, the layout a graph has before
 * convert_nchw_to_nhwc (what transpose_nchw_to_nhwc, graph.rs:339-356,
 * prepares on the host in the reference's recipe): the values are the same
 * as set_input_f32 of the transposed data.  When the input feeds only a 3x3
 * three-channel stem conv (f16 graphs), that conv reads the NCHW planes and
 * rounds them to f16 in its loader; otherwise each run starts with a
 * transpose launch into the NHWC input.  set_input_nchw_f32 copies host
 * data (count = n*c*h*w); bind_input_nchw_f32 reads the device buffer at
 * every run until the next set_input or bind call for that input (the
 * buffer must outlive those runs).  No counterpart in the reference. */
int dw_hip_graph_set_input_nchw_f32(dw_hip_graph_runtime* rt, const char* name, const float* data, size_t count);
int dw_hip_graph_bind_input_nchw_f32(dw_hip_graph_runtime* rt, const char* name, const dw_hip_buffer* buf);
/* run (vulkan_runtime.rs:359-419): enqueue every op; returns without waiting. */
int dw_hip_graph_run(dw_hip_graph_runtime* rt);
/* run_unbatched (vulkan_runtime.rs:423-470): enqueue the launches one by one
 * (never as a HIP graph); a failing launch is reported with its index and
 * op names.  With the environment variable DW_TRACE set, every launch is
 * printed to stderr and followed by a synchronize (as DRAGONWING_TRACE does). */
int dw_hip_graph_run_unbatched(dw_hip_graph_runtime* rt);
/* inputs() / outputs() (vulkan_runtime.rs:213-221): count and names of the
 * graph inputs (which = 0) or outputs (which = 1); names stay valid for the
 * runtime's lifetime.  Tensor shapes via dw_hip_graph_tensor_shape. */
int dw_hip_graph_num_io(dw_hip_graph_runtime* rt, int which);
const char* dw_hip_graph_io_name(dw_hip_graph_runtime* rt, int which, int index);
/* Shape of a graph tensor (NHWC for activations): up to 4 dims. */
int dw_hip_graph_tensor_shape(dw_hip_graph_runtime* rt, const char* name, int64_t* dims4, int* rank);
/* get_output_f32 (vulkan_runtime.rs:296): synchronizes, converts to f32. */
int dw_hip_graph_get_output_f32(dw_hip_graph_runtime* rt, const char* name, float* data, size_t count);
/* get_output_bytes (vulkan_runtime.rs:2131): synchronizes, raw bytes. */
int dw_hip_graph_get_output_bytes(dw_hip_graph_runtime* rt, const char* name, void* data, size_t len);
/* Activation memory (SlabStats, crates/dragonwing-vulkan/src/slab.rs:349-367):
 * the bytes of the runtime's activation arena, where storage roots whose
 * lifetimes do not overlap share bytes, and what the same roots would take
 * each in its own allocation.  Either pointer may be null. */
int dw_hip_graph_activation_bytes(dw_hip_graph_runtime* rt, size_t* arena, size_t* unshared);
/* Byte size of a graph tensor as the runtime stores it. */
int dw_hip_graph_tensor_bytes(dw_hip_graph_runtime* rt, const char* name, size_t* len);
/* Capture the launch list into a HIP graph and replay it on later runs
 * (the analogue of OpsRecorder's single command buffer, record.rs:49-679). */
int dw_hip_graph_enable_capture(dw_hip_graph_runtime* rt, int enable);
/* Number of kernel launches per run, and a per-launch description
 * ("<kernel> <op name> <algorithmic ops> <bytes>"). */
int dw_hip_graph_num_launches(dw_hip_graph_runtime* rt);
const char* dw_hip_graph_launch_info(dw_hip_graph_runtime* rt, int index);
/* One run with a HIP event pair around every launch; writes per-launch
 * milliseconds (array of dw_hip_graph_num_launches floats). */
int dw_hip_graph_run_profiled(dw_hip_graph_runtime* rt, float* launch_ms);
/* Per-launch device time: every launch of one run is enqueued `repeat`
 * times back to back between one HIP event pair, and launch_ms[i] is the
 * elapsed time divided by `repeat`: the kernel's duration plus the gap
 * between consecutive dispatches on the stream (the event overhead is spread
 * over the repeats).  Every launch only reads its inputs and writes its
 * outputs, so repeating it leaves the run's results as one run would. */
int dw_hip_graph_time_launches(dw_hip_graph_runtime* rt, int repeat, float* launch_ms);
/* As dw_hip_graph_time_launches, but the repeats of launch i cycle through
 * n_rt runtimes built from the same graph on the same backend (repeat r
 * runs runtime r % n_rt), so a working set larger than the Infinity Cache
 * is timed from HBM.  No counterpart in the reference (measurement only). */
int dw_hip_graph_time_launches_rotated(dw_hip_graph_runtime* const* rts, int n_rt, int repeat,
                                       float* launch_ms);

#ifdef __cplusplus
}
#endif
#endif /* DW_HIP_H */
