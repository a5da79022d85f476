// HIP backend: the dragonwing_core::Backend contract
// (crates/dragonwing-core/src/backend.rs:127-199) on one gfx950 device,
// plus the op functions of dragonwing_vulkan::ops re-targeted to the HIP
// kernels.  Every op validates buffer sizes exactly and enqueues on the
// backend's single stream; nothing here computes on the CPU.
#include "backend.h"

#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <exception>
#include <vector>

#include "../../include/dw_hip.h"

namespace dw {

static thread_local std::string g_last_error;

void set_last_error(const std::string& m) { g_last_error = m; }
void fail(int code, const std::string& msg) { throw Error{code, msg}; }
void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) fail(DW_ERR_BACKEND, std::string(what) + ": " + hipGetErrorString(e));
}

void* Backend::workspace(int slot, size_t bytes) {
  if (slot < 0 || slot >= kWsSlots) fail(DW_ERR_INVALID, "bad workspace slot");
  Ws& w = ws[slot];
  if (w.bytes < bytes) {
    if (w.ptr) {
      DW_HIP(hipStreamSynchronize(stream));
      DW_HIP(hipFree(w.ptr));
      w.ptr = nullptr;
      w.bytes = 0;
    }
    size_t want = std::max<size_t>(bytes, 4096);
    DW_HIP(hipMalloc(&w.ptr, want));
    w.bytes = want;
  }
  return w.ptr;
}

// Host -> device copy of small per-call parameter tables.  The source is a
// caller-owned (pageable) array, so the copy is completed before returning.
void Backend::upload_async(void* dst, const void* src, size_t bytes) {
  if (!bytes) return;
  DW_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream));
  DW_HIP(hipStreamSynchronize(stream));
}

Backend::~Backend() {
  if (stream) {
    (void)hipStreamSynchronize(stream);
    for (auto& w : ws)
      if (w.ptr) (void)hipFree(w.ptr);
    (void)hipStreamDestroy(stream);
  }
}

}  // namespace dw

using dw::Backend;

struct dw_hip_buffer {
  Backend* be;
  void* ptr;
  size_t len;
};

#define API_BEGIN try {
#define API_END                                     \
  }                                                 \
  catch (const dw::Error& e) {                      \
    dw::set_last_error(e.msg);                      \
    return e.code;                                  \
  }                                                 \
  catch (const std::exception& e) {                 \
    dw::set_last_error(e.what());                   \
    return DW_ERR_BACKEND;                          \
  }                                                 \
  return DW_OK;

namespace {

Backend* B(dw_hip_backend* be) {
  if (!be) dw::fail(DW_ERR_INVALID, "null backend");
  Backend* b = reinterpret_cast<Backend*>(be);
  DW_HIP(hipSetDevice(b->device));
  return b;
}

void need(const dw_hip_buffer* b, size_t bytes, const char* what) {
  if (!b) dw::fail(DW_ERR_INVALID, std::string(what) + ": null buffer");
  if (b->len != bytes)
    dw::fail(DW_ERR_INVALID, std::string(what) + " mismatch: expected " + std::to_string(bytes) +
                                 ", got " + std::to_string(b->len));
}

void check_i32(size_t v, const char* what) {
  if (v >= (size_t)INT32_MAX) dw::fail(DW_ERR_UNSUPPORTED, std::string(what) + " exceeds 2^31");
}

struct Geo {
  size_t n, h, w, ci, co, kh, kw, sh, sw, ph, pw, ho, wo;
};

Geo geo(size_t n, size_t h, size_t w, size_t ci, size_t co, size_t kh, size_t kw, size_t sh,
        size_t sw, size_t ph, size_t pw) {
  if (!n || !h || !w || !ci || !co || !kh || !kw || !sh || !sw)
    dw::fail(DW_ERR_INVALID, "conv: zero-sized dimension");
  if (h + 2 * ph < kh || w + 2 * pw < kw) dw::fail(DW_ERR_INVALID, "conv: kernel larger than padded input");
  Geo g{n, h, w, ci, co, kh, kw, sh, sw, ph, pw, (h + 2 * ph - kh) / sh + 1, (w + 2 * pw - kw) / sw + 1};
  check_i32(n * h * w * ci * 4, "input bytes");
  check_i32(n * g.ho * g.wo * co * 4, "output bytes");
  return g;
}

dw::DirectArgs direct_args(const Geo& g, const void* x, const float* wf, void* y) {
  dw::DirectArgs a{};
  a.x = x;
  a.wf = wf;
  a.y = y;
  a.n = (int)g.n; a.h = (int)g.h; a.w = (int)g.w; a.cin = (int)g.ci; a.cout = (int)g.co;
  a.kh = (int)g.kh; a.kw = (int)g.kw; a.sh = (int)g.sh; a.sw = (int)g.sw;
  a.pt = (int)g.ph; a.pl = (int)g.pw; a.ho = (int)g.ho; a.wo = (int)g.wo;
  a.m = (int)(g.n * g.ho * g.wo);
  a.x_pix_stride = (int)g.ci; a.x_c_off = 0;
  a.y_pix_stride = (int)g.co; a.y_c_off = 0;
  return a;
}

dw::IgemmArgs igemm_args(const Geo& g, const void* x, const void* wpk, void* y, int esize) {
  dw::IgemmArgs a{};
  a.x = (const uint8_t*)x;
  a.wpk = (const uint8_t*)wpk;
  a.y = y;
  a.n = (int)g.n; a.h = (int)g.h; a.w = (int)g.w; a.cin = (int)g.ci; a.cout = (int)g.co;
  a.kh = (int)g.kh; a.kw = (int)g.kw; a.sh = (int)g.sh; a.sw = (int)g.sw;
  a.pt = (int)g.ph; a.pl = (int)g.pw; a.ho = (int)g.ho; a.wo = (int)g.wo;
  a.m = (int)(g.n * g.ho * g.wo);
  const size_t kbytes = g.kh * g.kw * g.ci * esize;
  a.ksteps = (int)((kbytes + 63) / 64);
  const int bc = dw::igemm_channel_tile((int)g.co);
  a.cout_pad = (int)((g.co + bc - 1) / bc * bc);
  a.x_pix_stride = (int)g.ci; a.x_c_off = 0;
  a.y_pix_stride = (int)g.co; a.y_c_off = 0;
  a.r_pix_stride = (int)g.co; a.r_c_off = 0;
  return a;
}

void require_igemm(const Geo& g, int esize) {
  if ((g.ci * esize) % 16 != 0)
    dw::fail(DW_ERR_UNSUPPORTED, "MFMA conv needs c_in*esize % 16 == 0 (got c_in=" +
                                     std::to_string(g.ci) + ")");
  if (g.co % 4 != 0) dw::fail(DW_ERR_UNSUPPORTED, "MFMA conv needs c_out % 4 == 0");
  if (g.kh * g.kw > 31) dw::fail(DW_ERR_UNSUPPORTED, "MFMA conv supports at most 31 filter taps");
}

// Packs HWIO weights into workspace slot 0 and returns the pointer.
void* pack_into_ws(Backend* b, const dw_hip_buffer* kernel, const dw::IgemmArgs& a, const Geo& g,
                   int esize) {
  const size_t bytes = (size_t)a.ksteps * a.cout_pad * 64;
  void* wpk = b->workspace(Backend::WS_WPACK, bytes);
  dw::launch_pack_weights(b->stream, kernel->ptr, wpk, (int)(g.kh * g.kw * g.ci), (int)g.co,
                          a.cout_pad, a.ksteps, esize);
  return wpk;
}

void ew(Backend* b, int op, int dtype, const dw_hip_buffer* x, const dw_hip_buffer* y2,
        dw_hip_buffer* y, size_t count, size_t in_es, size_t out_es, float s0 = 0, float s1 = 0,
        int z0 = 0, int z1 = 0, int z2 = 0, float s2 = 0, const uint8_t* lut = nullptr) {
  need(x, count * in_es, "input");
  if (y2) need(y2, count * in_es, "input b");
  need(y, count * out_es, "output");
  dw::EwArgs a{};
  a.op = op; a.dtype = dtype; a.a = x->ptr; a.b = y2 ? y2->ptr : nullptr; a.y = y->ptr;
  a.count = count; a.c = 1; a.s0 = s0; a.s1 = s1; a.s2 = s2; a.z0 = z0; a.z1 = z1; a.z2 = z2;
  a.lut = lut;
  dw::launch_elementwise(b->stream, a);
}

}  // namespace

extern "C" {

const char* dw_last_error(void) { return dw::g_last_error.c_str(); }

int dw_hip_backend_create(int device, dw_hip_backend** out) {
  API_BEGIN
  if (!out) dw::fail(DW_ERR_INVALID, "null out");
  int count = 0;
  DW_HIP(hipGetDeviceCount(&count));
  if (device < 0 || device >= count)
    dw::fail(DW_ERR_BACKEND, "no HIP device " + std::to_string(device) + " (found " +
                                 std::to_string(count) + ")");
  DW_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  DW_HIP(hipGetDeviceProperties(&prop, device));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    dw::fail(DW_ERR_UNSUPPORTED, std::string("device is ") + prop.gcnArchName + ", need gfx950");
  void* scratch = dw::noalloc_scratch_setup(device);
  Backend* b = new Backend();
  b->device = device;
  b->num_cus = prop.multiProcessorCount;
  b->scratch = scratch;
  DW_HIP(hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking));
  *out = reinterpret_cast<dw_hip_backend*>(b);
  API_END
}

void dw_hip_backend_destroy(dw_hip_backend* be) {
  if (be) dw::release(reinterpret_cast<Backend*>(be));
}

const char* dw_hip_backend_name(const dw_hip_backend* be) {
  (void)be;
  return "hip-gfx950";
}

int dw_hip_alloc(dw_hip_backend* be, size_t len_bytes, int kind, dw_hip_buffer** out) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  if (kind != DW_BUFFER_STORAGE) dw::fail(DW_ERR_UNSUPPORTED, "unknown buffer kind");
  if (!out) dw::fail(DW_ERR_INVALID, "null out");
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, std::max<size_t>(len_bytes, 1));
  if (e != hipSuccess)
    dw::fail(DW_ERR_BACKEND, "alloc of " + std::to_string(len_bytes) + " bytes failed: " +
                                 hipGetErrorString(e));
  *out = new dw_hip_buffer{b, p, len_bytes};
  dw::hold(b);
  API_END
}

void dw_hip_buffer_free(dw_hip_buffer* buf) {
  if (!buf) return;
  Backend* b = buf->be;
  (void)hipSetDevice(b->device);
  (void)hipStreamSynchronize(b->stream);
  (void)hipFree(buf->ptr);
  delete buf;
  dw::release(b);
}

size_t dw_hip_buffer_len_bytes(const dw_hip_buffer* buf) { return buf ? buf->len : 0; }
void* dw_hip_buffer_device_ptr(const dw_hip_buffer* buf) { return buf ? buf->ptr : nullptr; }

int dw_hip_upload(dw_hip_backend* be, dw_hip_buffer* dst, const void* src, size_t len) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  if (!dst) dw::fail(DW_ERR_INVALID, "null buffer");
  if (len != dst->len)
    dw::fail(DW_ERR_INVALID, "upload size mismatch: buffer " + std::to_string(dst->len) +
                                 " bytes, source " + std::to_string(len) + " bytes");
  if (len) {
    DW_HIP(hipMemcpyAsync(dst->ptr, src, len, hipMemcpyHostToDevice, b->stream));
    DW_HIP(hipStreamSynchronize(b->stream));
  }
  API_END
}

int dw_hip_download(dw_hip_backend* be, const dw_hip_buffer* src, void* dst, size_t len) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  if (!src) dw::fail(DW_ERR_INVALID, "null buffer");
  if (len != src->len)
    dw::fail(DW_ERR_INVALID, "download size mismatch: buffer " + std::to_string(src->len) +
                                 " bytes, destination " + std::to_string(len) + " bytes");
  DW_HIP(hipStreamSynchronize(b->stream));
  if (len) {
    DW_HIP(hipMemcpyAsync(dst, src->ptr, len, hipMemcpyDeviceToHost, b->stream));
    DW_HIP(hipStreamSynchronize(b->stream));
  }
  API_END
}

int dw_hip_synchronize(dw_hip_backend* be) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  DW_HIP(hipStreamSynchronize(b->stream));
  API_END
}

// ---------------------------------------------------------------------------
// Convolutions
// ---------------------------------------------------------------------------

static int conv_f32_common(dw_hip_backend* be, const dw_hip_buffer* input, const dw_hip_buffer* kernel,
                           const dw_hip_buffer* bias, dw_hip_buffer* output, size_t n, size_t h_in,
                           size_t w_in, size_t c_in, size_t c_out, size_t k_h, size_t k_w,
                           size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w, int act) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  Geo g = geo(n, h_in, w_in, c_in, c_out, k_h, k_w, stride_h, stride_w, pad_h, pad_w);
  need(input, n * h_in * w_in * c_in * 4, "conv2d_f32: input");
  need(kernel, k_h * k_w * c_in * c_out * 4, "conv2d_f32: kernel");
  need(output, n * g.ho * g.wo * c_out * 4, "conv2d_f32: output");
  if (bias) need(bias, c_out * 4, "conv2d_f32: bias");
  dw::DirectArgs a = direct_args(g, input->ptr, (const float*)kernel->ptr, output->ptr);
  a.in_kind = 0;
  a.out_kind = 0;
  a.act = act;
  a.bias_f = bias ? (const float*)bias->ptr : nullptr;
  if (c_in % 16 == 0 && c_out % 4 == 0) {
    float* wq = (float*)b->workspace(Backend::WS_WPACK, k_h * k_w * c_in * c_out * 4);
    dw::launch_repack_oc4(b->stream, (const float*)kernel->ptr, wq, (int)(k_h * k_w * c_in), (int)c_out);
    a.wq = wq;
  }
  dw::launch_direct_conv(b->stream, a);
  API_END
}

int dw_hip_conv2d_f32_nhwc(dw_hip_backend* be, const dw_hip_buffer* input, const dw_hip_buffer* kernel,
                           dw_hip_buffer* output, size_t n, size_t h_in, size_t w_in, size_t c_in,
                           size_t c_out, size_t k_h, size_t k_w, size_t stride_h, size_t stride_w,
                           size_t pad_h, size_t pad_w) {
  return conv_f32_common(be, input, kernel, nullptr, output, n, h_in, w_in, c_in, c_out, k_h, k_w,
                         stride_h, stride_w, pad_h, pad_w, DW_ACT_NONE);
}

int dw_hip_conv2d_bias_act_f32_nhwc(dw_hip_backend* be, const dw_hip_buffer* input,
                                    const dw_hip_buffer* kernel, const dw_hip_buffer* bias,
                                    dw_hip_buffer* output, size_t n, size_t h_in, size_t w_in,
                                    size_t c_in, size_t c_out, size_t k_h, size_t k_w,
                                    size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w,
                                    int act) {
  return conv_f32_common(be, input, kernel, bias, output, n, h_in, w_in, c_in, c_out, k_h, k_w,
                         stride_h, stride_w, pad_h, pad_w, act);
}

int dw_hip_conv2d_bias_act_f16_nhwc(dw_hip_backend* be, const dw_hip_buffer* input,
                                    const dw_hip_buffer* kernel, const dw_hip_buffer* bias,
                                    dw_hip_buffer* output, size_t n, size_t h_in, size_t w_in,
                                    size_t c_in, size_t c_out, size_t k_h, size_t k_w,
                                    size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w,
                                    int act, int exact) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  Geo g = geo(n, h_in, w_in, c_in, c_out, k_h, k_w, stride_h, stride_w, pad_h, pad_w);
  need(input, n * h_in * w_in * c_in * 2, "conv2d_fp16: input");
  need(kernel, k_h * k_w * c_in * c_out * 2, "conv2d_fp16: kernel");
  need(output, n * g.ho * g.wo * c_out * 2, "conv2d_fp16: output");
  if (bias) need(bias, c_out * 2, "conv2d_fp16: bias");
  if (exact) {
    const size_t kcount = k_h * k_w * c_in * c_out;
    float* wf = (float*)b->workspace(Backend::WS_WPACK, kcount * 4);
    dw::EwArgs e{};
    e.op = dw::EW_F16_TO_F32; e.a = kernel->ptr; e.y = wf; e.count = kcount;
    dw::launch_elementwise(b->stream, e);
    dw::DirectArgs a = direct_args(g, input->ptr, wf, output->ptr);
    a.in_kind = 1;
    a.out_kind = 1;
    a.act = act;
    a.bias_h = bias ? (const uint16_t*)bias->ptr : nullptr;
    dw::launch_direct_conv(b->stream, a);
  } else {
    require_igemm(g, 2);
    dw::IgemmArgs a = igemm_args(g, input->ptr, nullptr, output->ptr, 2);
    a.wpk = (const uint8_t*)pack_into_ws(b, kernel, a, g, 2);
    a.epi = dw::EPI_F16;
    a.act = act;
    a.bias_h = bias ? (const uint16_t*)bias->ptr : nullptr;
    dw::launch_igemm(b->stream, a, 2);
  }
  API_END
}

static int dwconv_common(dw_hip_backend* be, int dtype, const dw_hip_buffer* input,
                         const dw_hip_buffer* kernel, const dw_hip_buffer* bias, dw_hip_buffer* output,
                         size_t n, size_t h_in, size_t w_in, size_t c, size_t k_h, size_t k_w,
                         size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w, int act) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  const size_t es = dtype == DW_DTYPE_F16 ? 2 : 4;
  Geo g = geo(n, h_in, w_in, c, c, k_h, k_w, stride_h, stride_w, pad_h, pad_w);
  // f16 3x3 with stride 1 or 2 runs on the sliding-window kernel (channel
  // groups of 4); every other shape on the generic one (groups of 8)
  const bool sliding = dtype == DW_DTYPE_F16 && k_h == 3 && k_w == 3 && (stride_w == 1 || stride_w == 2);
  if (c % (sliding ? 4 : 8) != 0)
    dw::fail(DW_ERR_UNSUPPORTED, sliding ? "depthwise: c must be a multiple of 4" : "depthwise: c must be a multiple of 8");
  need(input, n * h_in * w_in * c * es, "depthwise: input");
  need(kernel, k_h * k_w * c * es, "depthwise: kernel");
  need(output, n * g.ho * g.wo * c * es, "depthwise: output");
  if (bias) need(bias, c * es, "depthwise: bias");
  dw::DwArgs a{};
  a.x = input->ptr; a.wt = kernel->ptr; a.bias = bias ? bias->ptr : nullptr; a.y = output->ptr;
  a.n = (int)n; a.h = (int)h_in; a.w = (int)w_in; a.c = (int)c; a.kh = (int)k_h; a.kw = (int)k_w;
  a.sh = (int)stride_h; a.sw = (int)stride_w; a.pt = (int)pad_h; a.pl = (int)pad_w;
  a.ho = (int)g.ho; a.wo = (int)g.wo; a.act = act;
  a.x_pix_stride = (int)c; a.y_pix_stride = (int)c;
  dw::launch_dwconv(b->stream, a, dtype == DW_DTYPE_F16 ? dw::F16 : dw::F32);
  API_END
}

int dw_hip_depthwise_conv2d_f16_nhwc(dw_hip_backend* be, const dw_hip_buffer* input,
                                     const dw_hip_buffer* kernel, const dw_hip_buffer* bias,
                                     dw_hip_buffer* output, size_t n, size_t h_in, size_t w_in,
                                     size_t c, size_t k_h, size_t k_w, size_t stride_h,
                                     size_t stride_w, size_t pad_h, size_t pad_w, int act) {
  return dwconv_common(be, DW_DTYPE_F16, input, kernel, bias, output, n, h_in, w_in, c, k_h, k_w,
                       stride_h, stride_w, pad_h, pad_w, act);
}

int dw_hip_depthwise_conv2d_f32_nhwc(dw_hip_backend* be, const dw_hip_buffer* input,
                                     const dw_hip_buffer* kernel, const dw_hip_buffer* bias,
                                     dw_hip_buffer* output, size_t n, size_t h_in, size_t w_in,
                                     size_t c, size_t k_h, size_t k_w, size_t stride_h,
                                     size_t stride_w, size_t pad_h, size_t pad_w, int act) {
  return dwconv_common(be, DW_DTYPE_F32, input, kernel, bias, output, n, h_in, w_in, c, k_h, k_w,
                       stride_h, stride_w, pad_h, pad_w, act);
}

namespace {

// Where a QLinearConv's per-call device data goes: the backend's grow-only
// workspaces (wpk == nullptr), or caller-provided space of fixed capacity.
struct QconvSpace {
  void* wpk = nullptr;
  size_t wpk_cap = 0;
  float* ms = nullptr;
  int* bi = nullptr;
};

void qlinearconv_impl(Backend* b, const dw_hip_buffer* input, const dw_hip_buffer* kernel,
                      const dw_hip_buffer* bias, dw_hip_buffer* output, size_t n, size_t h_in, size_t w_in,
                      size_t c_in, size_t c_out, size_t k_h, size_t k_w, size_t stride_h, size_t stride_w,
                      size_t pad_h, size_t pad_w, float x_scale, int x_zp, const float* w_scales,
                      float y_scale, int y_zp, QconvSpace sp, float* m_host) {
  Geo g = geo(n, h_in, w_in, c_in, c_out, k_h, k_w, stride_h, stride_w, pad_h, pad_w);
  require_igemm(g, 1);
  need(input, n * h_in * w_in * c_in, "qlinearconv: input");
  need(kernel, k_h * k_w * c_in * c_out, "qlinearconv: kernel");
  need(output, n * g.ho * g.wo * c_out, "qlinearconv: output");
  if (bias) need(bias, c_out * 4, "qlinearconv: bias");
  if (!w_scales) dw::fail(DW_ERR_INVALID, "qlinearconv: null w_scales");
  if (x_zp < 0 || x_zp > 255 || y_zp < 0 || y_zp > 255)
    dw::fail(DW_ERR_INVALID, "qlinearconv: zero points must be in [0, 255]");
  if (!(x_scale > 0) || !(y_scale > 0)) dw::fail(DW_ERR_INVALID, "qlinearconv: scales must be > 0");
  for (size_t c = 0; c < c_out; ++c) {
    if (!(w_scales[c] > 0)) dw::fail(DW_ERR_INVALID, "qlinearconv: weight scales must be > 0");
    m_host[c] = (x_scale * w_scales[c]) / y_scale;
  }
  dw::IgemmArgs a = igemm_args(g, input->ptr, nullptr, output->ptr, 1);
  const size_t wpk_bytes = (size_t)a.ksteps * a.cout_pad * 64;
  if (sp.wpk) {
    if (wpk_bytes > sp.wpk_cap)
      dw::fail(DW_ERR_UNSUPPORTED, "qlinearconv: packed weights of " + std::to_string(wpk_bytes) +
                                       " bytes exceed the no-alloc scratch's " + std::to_string(sp.wpk_cap));
    dw::launch_pack_weights(b->stream, kernel->ptr, sp.wpk, (int)(g.kh * g.kw * g.ci), (int)g.co, a.cout_pad,
                            a.ksteps, 1);
    a.wpk = (const uint8_t*)sp.wpk;
  } else {
    a.wpk = (const uint8_t*)pack_into_ws(b, kernel, a, g, 1);
    sp.ms = (float*)b->workspace(Backend::WS_SCALE, c_out * 4);
    sp.bi = (int*)b->workspace(Backend::WS_BIAS, c_out * 4);
  }
  b->upload_async(sp.ms, m_host, c_out * 4);
  dw::launch_qconv_bias(b->stream, (const int8_t*)kernel->ptr, bias ? (const int*)bias->ptr : nullptr,
                        sp.bi, (int)(k_h * k_w * c_in), (int)c_out, 128 - x_zp);
  a.epi = dw::EPI_QU8;
  a.xxor = 0x80808080u;
  const uint32_t pb = (uint32_t)((x_zp ^ 0x80) & 0xff);
  a.xpad = pb * 0x01010101u;
  a.bias_i = sp.bi;
  a.mscale = sp.ms;
  a.y_zp = y_zp;
  dw::launch_igemm(b->stream, a, 1);
}

}  // namespace

int dw_hip_qlinearconv_u8s8(dw_hip_backend* be, const dw_hip_buffer* input, const dw_hip_buffer* kernel,
                            const dw_hip_buffer* bias, dw_hip_buffer* output, size_t n, size_t h_in,
                            size_t w_in, size_t c_in, size_t c_out, size_t k_h, size_t k_w,
                            size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w,
                            float x_scale, int x_zp, const float* w_scales, float y_scale, int y_zp) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  std::vector<float> m(c_out);
  qlinearconv_impl(b, input, kernel, bias, output, n, h_in, w_in, c_in, c_out, k_h, k_w, stride_h, stride_w,
                   pad_h, pad_w, x_scale, x_zp, w_scales, y_scale, y_zp, QconvSpace{}, m.data());
  API_END
}

int dw_hip_qlinearconv_u8s8_noalloc(dw_hip_backend* be, const dw_hip_buffer* input, const dw_hip_buffer* kernel,
                                    const dw_hip_buffer* bias, dw_hip_buffer* output, size_t n, size_t h_in,
                                    size_t w_in, size_t c_in, size_t c_out, size_t k_h, size_t k_w,
                                    size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w,
                                    float x_scale, int x_zp, const float* w_scales, float y_scale, int y_zp) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  if (!b->scratch) dw::fail(DW_ERR_BACKEND, "qlinearconv_noalloc: no scratch on this device");
  if (c_out > dw::kNoAllocMaxChannels)
    dw::fail(DW_ERR_UNSUPPORTED, "qlinearconv_noalloc: c_out above " + std::to_string(dw::kNoAllocMaxChannels));
  float m[dw::kNoAllocMaxChannels];
  dw::ScratchUse use(b->device, b->stream);
  QconvSpace sp;
  uint8_t* base = (uint8_t*)b->scratch;
  sp.ms = (float*)base;
  sp.bi = (int*)(base + dw::kNoAllocMaxChannels * 4);
  sp.wpk = base + dw::kNoAllocTableBytes;
  sp.wpk_cap = dw::kNoAllocScratchBytes - dw::kNoAllocTableBytes;
  qlinearconv_impl(b, input, kernel, bias, output, n, h_in, w_in, c_in, c_out, k_h, k_w, stride_h, stride_w,
                   pad_h, pad_w, x_scale, x_zp, w_scales, y_scale, y_zp, sp, m);
  API_END
}

int dw_hip_qgemm_u8s8(dw_hip_backend* be, const dw_hip_buffer* a, const dw_hip_buffer* b, const dw_hip_buffer* bias,
                      dw_hip_buffer* y, size_t m, size_t n, size_t k, int trans_b, float a_scale, int a_zp,
                      const float* b_scales, float y_scale, int y_zp) {
  API_BEGIN
  Backend* bk = B(be);
  std::lock_guard<std::mutex> lock(bk->mu);
  if (!m || !n || !k) dw::fail(DW_ERR_INVALID, "qgemm: zero size");
  check_i32(m * k, "qgemm: A");
  check_i32(k * n, "qgemm: B");
  need(b, k * n, "qgemm: B");
  // B as [k][n] (the 1x1 HWIO layout); a transposed B goes through a
  // workspace copy first
  dw_hip_buffer bt{bk, b->ptr, b->len};
  if (trans_b) {
    bt.ptr = bk->workspace(Backend::WS_POST, k * n);
    dw::launch_transpose_u8(bk->stream, b->ptr, bt.ptr, (int)n, (int)k);
  }
  std::vector<float> ms(n);
  // rows of A are the pixels of a 1x1 convolution over n = m images of 1 x 1
  qlinearconv_impl(bk, a, &bt, bias, y, m, 1, 1, k, n, 1, 1, 1, 1, 0, 0, a_scale, a_zp, b_scales, y_scale, y_zp,
                   QconvSpace{}, ms.data());
  API_END
}

int dw_hip_qlinear_global_avg_pool_u8(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t n,
                                      size_t h, size_t w, size_t c, float x_scale, int x_zp, float y_scale,
                                      int y_zp) {
  API_BEGIN
  Backend* bk = B(be);
  std::lock_guard<std::mutex> lock(bk->mu);
  if (!n || !h || !w || !c) dw::fail(DW_ERR_INVALID, "qlinear_gap: zero size");
  check_i32(n * h * w * c, "qlinear_gap: input");
  if (h * w > (size_t)(1 << 23)) dw::fail(DW_ERR_UNSUPPORTED, "qlinear_gap: more than 2^23 pixels per image");
  if (!(x_scale > 0) || !(y_scale > 0)) dw::fail(DW_ERR_INVALID, "qlinear_gap: scales must be > 0");
  if (x_zp < 0 || x_zp > 255 || y_zp < 0 || y_zp > 255) dw::fail(DW_ERR_INVALID, "qlinear_gap: zero points");
  need(x, n * h * w * c, "qlinear_gap: input");
  need(y, n * c, "qlinear_gap: output");
  const float m = (x_scale / y_scale) / (float)(h * w);
  dw::launch_qlinear_gap(bk->stream, (const uint8_t*)x->ptr, (uint8_t*)y->ptr, (int)n, (int)(h * w), (int)c, x_zp, m,
                         y_zp);
  API_END
}

int dw_hip_conv2d_i8_nhwc(dw_hip_backend* be, const dw_hip_buffer* input, const dw_hip_buffer* kernel,
                          dw_hip_buffer* output_i32, size_t n, size_t h_in, size_t w_in, size_t c_in,
                          size_t c_out, size_t k_h, size_t k_w, size_t stride_h, size_t stride_w,
                          size_t pad_h, size_t pad_w) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  Geo g = geo(n, h_in, w_in, c_in, c_out, k_h, k_w, stride_h, stride_w, pad_h, pad_w);
  require_igemm(g, 1);
  need(input, n * h_in * w_in * c_in, "conv2d_i8: input");
  need(kernel, k_h * k_w * c_in * c_out, "conv2d_i8: kernel");
  need(output_i32, n * g.ho * g.wo * c_out * 4, "conv2d_i8: output");
  dw::IgemmArgs a = igemm_args(g, input->ptr, nullptr, output_i32->ptr, 1);
  a.wpk = (const uint8_t*)pack_into_ws(b, kernel, a, g, 1);
  a.epi = dw::EPI_I32;
  dw::launch_igemm(b->stream, a, 1);
  API_END
}

int dw_hip_conv2d_requant_relu_i8(dw_hip_backend* be, const dw_hip_buffer* input,
                                  const dw_hip_buffer* kernel, dw_hip_buffer* output, size_t n,
                                  size_t h_in, size_t w_in, size_t c_in, size_t c_out, size_t k_h,
                                  size_t k_w, size_t stride_h, size_t stride_w, size_t pad_h,
                                  size_t pad_w, float requant_scale, int do_relu) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  Geo g = geo(n, h_in, w_in, c_in, c_out, k_h, k_w, stride_h, stride_w, pad_h, pad_w);
  require_igemm(g, 1);
  need(input, n * h_in * w_in * c_in, "conv_fused: input");
  need(kernel, k_h * k_w * c_in * c_out, "conv_fused: kernel");
  need(output, n * g.ho * g.wo * c_out, "conv_fused: output");
  dw::IgemmArgs a = igemm_args(g, input->ptr, nullptr, output->ptr, 1);
  a.wpk = (const uint8_t*)pack_into_ws(b, kernel, a, g, 1);
  a.epi = dw::EPI_QS8_REF;
  a.tscale = requant_scale;
  a.act = do_relu ? dw::ACT_RELU : dw::ACT_NONE;
  dw::launch_igemm(b->stream, a, 1);
  API_END
}

// ---------------------------------------------------------------------------
// Elementwise
// ---------------------------------------------------------------------------
#define EW1(NAME, OP, DT, IES, OES)                                                              \
  int NAME(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t count) {         \
    API_BEGIN Backend* b = B(be); std::lock_guard<std::mutex> lock(b->mu);                       \
    ew(b, OP, DT, x, nullptr, y, count, IES, OES);                                              \
    API_END                                                                                      \
  }
#define EW2(NAME, OP, DT, ES)                                                                    \
  int NAME(dw_hip_backend* be, const dw_hip_buffer* a, const dw_hip_buffer* bb, dw_hip_buffer* y, \
           size_t count) {                                                                       \
    API_BEGIN Backend* b = B(be); std::lock_guard<std::mutex> lock(b->mu);                       \
    ew(b, OP, DT, a, bb, y, count, ES, ES);                                                     \
    API_END                                                                                      \
  }

EW1(dw_hip_relu_f32, dw::EW_RELU, dw::F32, 4, 4)
EW1(dw_hip_relu_fp16, dw::EW_RELU, dw::F16, 2, 2)
EW1(dw_hip_sigmoid_f32, dw::EW_SIGMOID, dw::F32, 4, 4)
EW1(dw_hip_sigmoid_fp16, dw::EW_SIGMOID, dw::F16, 2, 2)
EW1(dw_hip_silu_f32, dw::EW_SILU, dw::F32, 4, 4)
EW1(dw_hip_silu_fp16, dw::EW_SILU, dw::F16, 2, 2)
EW1(dw_hip_relu_i8, dw::EW_RELU_I8, dw::I8, 1, 1)
EW2(dw_hip_add_f32, dw::EW_ADD, dw::F32, 4)
EW2(dw_hip_add_fp16, dw::EW_ADD, dw::F16, 2)
EW2(dw_hip_mul_f32, dw::EW_MUL, dw::F32, 4)
EW2(dw_hip_mul_fp16, dw::EW_MUL, dw::F16, 2)

int dw_hip_bias_add_f32_nhwc(dw_hip_backend* be, dw_hip_buffer* y, const dw_hip_buffer* bias,
                             size_t count, size_t c) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  need(y, count * 4, "bias_add: y");
  need(bias, c * 4, "bias_add: bias");
  if (c == 0 || count % c != 0) dw::fail(DW_ERR_INVALID, "bias_add: count must be a multiple of c");
  dw::EwArgs a{};
  a.op = dw::EW_BIAS_ADD; a.dtype = dw::F32; a.a = y->ptr; a.b = bias->ptr; a.y = y->ptr;
  a.count = count; a.c = (int)c;
  dw::launch_elementwise(b->stream, a);
  API_END
}

int dw_hip_requantize_i32_to_i8(dw_hip_backend* be, const dw_hip_buffer* x_i32, dw_hip_buffer* y_i8,
                                size_t count, float requant_scale) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  ew(b, dw::EW_REQUANT_I32_I8, dw::I32, x_i32, nullptr, y_i8, count, 4, 1, requant_scale);
  API_END
}

int dw_hip_quantize_f32_to_i8(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y_i8,
                              size_t count, float scale) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  const float inv = 1.0f / scale;  // quantize_f32_to_i8 (ops.rs:3503-3516) multiplies by 1/scale
  ew(b, dw::EW_QUANT_F32_I8, dw::F32, x, nullptr, y_i8, count, 4, 1, inv);
  API_END
}

int dw_hip_dequantize_i8_to_f32(dw_hip_backend* be, const dw_hip_buffer* x_i8, dw_hip_buffer* y,
                                size_t count, float scale) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  ew(b, dw::EW_DEQUANT_I8_F32, dw::I8, x_i8, nullptr, y, count, 1, 4, scale);
  API_END
}

int dw_hip_add_i8(dw_hip_backend* be, const dw_hip_buffer* a, const dw_hip_buffer* bb, dw_hip_buffer* y,
                  size_t count, float scale_a_over_y, float scale_b_over_y) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  ew(b, dw::EW_ADD_I8, dw::I8, a, bb, y, count, 1, 1, scale_a_over_y, scale_b_over_y);
  API_END
}

int dw_hip_quantize_linear_f16_u8(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y,
                                  size_t count, float scale, int zp) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  ew(b, dw::EW_QUANT_LINEAR_F16_U8, dw::F16, x, nullptr, y, count, 2, 1, scale, 0, zp);
  API_END
}

int dw_hip_dequantize_linear_u8_f16(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y,
                                    size_t count, float scale, int zp) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  ew(b, dw::EW_DEQUANT_LINEAR_U8_F16, dw::U8, x, nullptr, y, count, 1, 2, scale, 0, zp);
  API_END
}

int dw_hip_qlinear_add_u8(dw_hip_backend* be, const dw_hip_buffer* a, const dw_hip_buffer* bb,
                          dw_hip_buffer* y, size_t count, float a_scale, int a_zp, float b_scale,
                          int b_zp, float y_scale, int y_zp) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  const float ra = a_scale / y_scale, rb = b_scale / y_scale;
  ew(b, dw::EW_QADD_U8, dw::U8, a, bb, y, count, 1, 1, ra, rb, a_zp, b_zp, y_zp);
  API_END
}

int dw_hip_lut_u8(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t count,
                  const uint8_t* lut256) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  if (!lut256) dw::fail(DW_ERR_INVALID, "lut: null table");
  uint8_t* lut = (uint8_t*)b->workspace(Backend::WS_LUT, 256);
  b->upload_async(lut, lut256, 256);
  ew(b, dw::EW_LUT_U8, dw::U8, x, nullptr, y, count, 1, 1, 0, 0, 0, 0, 0, 0, lut);
  API_END
}

// ---------------------------------------------------------------------------
// Data movement
// ---------------------------------------------------------------------------

int dw_hip_maxpool2d_nhwc(dw_hip_backend* be, int dtype, const dw_hip_buffer* x, dw_hip_buffer* y,
                          size_t n, size_t h_in, size_t w_in, size_t c, size_t pool_h, size_t pool_w,
                          size_t stride_h, size_t stride_w, size_t pad_t, size_t pad_l, size_t pad_b,
                          size_t pad_r) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  if (dtype != DW_DTYPE_F32 && dtype != DW_DTYPE_F16 && dtype != DW_DTYPE_U8 && dtype != DW_DTYPE_I8)
    dw::fail(DW_ERR_UNSUPPORTED, "maxpool: dtype");
  if (!pool_h || !pool_w || !stride_h || !stride_w) dw::fail(DW_ERR_INVALID, "maxpool: zero size");
  if (pad_t >= pool_h || pad_b >= pool_h || pad_l >= pool_w || pad_r >= pool_w)
    dw::fail(DW_ERR_INVALID, "maxpool: pad must be smaller than the window");
  if (h_in + pad_t + pad_b < pool_h || w_in + pad_l + pad_r < pool_w)
    dw::fail(DW_ERR_INVALID, "maxpool: window larger than padded input");
  const size_t ho = (h_in + pad_t + pad_b - pool_h) / stride_h + 1;
  const size_t wo = (w_in + pad_l + pad_r - pool_w) / stride_w + 1;
  const size_t es = dw::dtype_size(dtype);
  need(x, n * h_in * w_in * c * es, "maxpool: input");
  need(y, n * ho * wo * c * es, "maxpool: output");
  dw::PoolArgs a{};
  a.x = {x->ptr, (int)c, 0};
  a.y = {y->ptr, (int)c, 0};
  a.n = (int)n; a.h = (int)h_in; a.w = (int)w_in; a.c = (int)c; a.kh = (int)pool_h; a.kw = (int)pool_w;
  a.sh = (int)stride_h; a.sw = (int)stride_w; a.pt = (int)pad_t; a.pl = (int)pad_l;
  a.ho = (int)ho; a.wo = (int)wo;
  dw::launch_maxpool(b->stream, a, dtype);
  API_END
}

int dw_hip_resize_nearest_nhwc(dw_hip_backend* be, int dtype, const dw_hip_buffer* x, dw_hip_buffer* y,
                               size_t n, size_t h_in, size_t w_in, size_t h_out, size_t w_out, size_t c) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  const size_t es = dw::dtype_size(dtype);
  if (!h_in || !w_in || !h_out || !w_out) dw::fail(DW_ERR_INVALID, "resize: zero size");
  need(x, n * h_in * w_in * c * es, "resize: input");
  need(y, n * h_out * w_out * c * es, "resize: output");
  dw::ResizeArgs a{};
  a.x = {x->ptr, (int)c, 0};
  a.y = {y->ptr, (int)c, 0};
  a.n = (int)n; a.h = (int)h_in; a.w = (int)w_in; a.c = (int)c; a.ho = (int)h_out; a.wo = (int)w_out;
  dw::launch_resize_nearest(b->stream, a, dtype);
  API_END
}

int dw_hip_concat_channels_nhwc(dw_hip_backend* be, int dtype, const dw_hip_buffer* const* inputs,
                                const size_t* channels, size_t num_inputs, dw_hip_buffer* y,
                                size_t pixels) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  const size_t es = dw::dtype_size(dtype);
  size_t total = 0;
  for (size_t i = 0; i < num_inputs; ++i) total += channels[i];
  need(y, pixels * total * es, "concat: output");
  size_t off = 0;
  for (size_t i = 0; i < num_inputs; ++i) {
    need(inputs[i], pixels * channels[i] * es, "concat: input");
    dw::launch_copy_channels(b->stream, {inputs[i]->ptr, (int)channels[i], 0},
                             {y->ptr, (int)total, (int)off}, (int)pixels, (int)channels[i], (int)es);
    off += channels[i];
  }
  API_END
}

int dw_hip_split_channels_nhwc(dw_hip_backend* be, int dtype, const dw_hip_buffer* x,
                               dw_hip_buffer* const* outputs, const size_t* channels,
                               size_t num_outputs, size_t pixels) {
  API_BEGIN
  Backend* b = B(be);
  std::lock_guard<std::mutex> lock(b->mu);
  const size_t es = dw::dtype_size(dtype);
  size_t total = 0;
  for (size_t i = 0; i < num_outputs; ++i) total += channels[i];
  need(x, pixels * total * es, "split: input");
  size_t off = 0;
  for (size_t i = 0; i < num_outputs; ++i) {
    need(outputs[i], pixels * channels[i] * es, "split: output");
    dw::launch_copy_channels(b->stream, {x->ptr, (int)total, (int)off},
                             {outputs[i]->ptr, (int)channels[i], 0}, (int)pixels, (int)channels[i],
                             (int)es);
    off += channels[i];
  }
  API_END
}

// Classifier-head ops (see dw_hip.h for the reference functions each mirrors).
int dw_hip_gemm_f32(dw_hip_backend* be, const dw_hip_buffer* a, const dw_hip_buffer* b, dw_hip_buffer* c,
                    size_t m, size_t n, size_t k) {
  API_BEGIN
  Backend* bk = B(be);
  std::lock_guard<std::mutex> lock(bk->mu);
  if (!m || !n || !k) dw::fail(DW_ERR_INVALID, "gemm_f32: zero size");
  if (m > 65535 || n > INT32_MAX || k > INT32_MAX) dw::fail(DW_ERR_UNSUPPORTED, "gemm_f32: m > 65535 or n, k > 2^31 - 1");
  need(a, m * k * 4, "gemm_f32: A size");
  need(b, k * n * 4, "gemm_f32: B size");
  need(c, m * n * 4, "gemm_f32: C size");
  dw::launch_gemm(bk->stream, dw::F32, a->ptr, b->ptr, c->ptr, (int)m, (int)n, (int)k);
  API_END
}

int dw_hip_gemm_fp16(dw_hip_backend* be, const dw_hip_buffer* a, const dw_hip_buffer* b, dw_hip_buffer* c,
                     size_t m, size_t n, size_t k) {
  API_BEGIN
  Backend* bk = B(be);
  std::lock_guard<std::mutex> lock(bk->mu);
  if (!m || !n || !k) dw::fail(DW_ERR_INVALID, "gemm_fp16: zero size");
  if (m > 65535 || n > INT32_MAX || k > INT32_MAX) dw::fail(DW_ERR_UNSUPPORTED, "gemm_fp16: m > 65535 or n, k > 2^31 - 1");
  need(a, m * k * 2, "gemm_fp16: A size");
  need(b, k * n * 2, "gemm_fp16: B size");
  need(c, m * n * 2, "gemm_fp16: C size");
  dw::launch_gemm(bk->stream, dw::F16, a->ptr, b->ptr, c->ptr, (int)m, (int)n, (int)k);
  API_END
}

int dw_hip_gemm_i8(dw_hip_backend* be, const dw_hip_buffer* a, const dw_hip_buffer* b, dw_hip_buffer* c_i32,
                   size_t m, size_t n, size_t k) {
  API_BEGIN
  Backend* bk = B(be);
  std::lock_guard<std::mutex> lock(bk->mu);
  if (!m || !n || !k) dw::fail(DW_ERR_INVALID, "gemm_i8: zero size");
  if (m > 65535 || n > INT32_MAX || k > INT32_MAX) dw::fail(DW_ERR_UNSUPPORTED, "gemm_i8: m > 65535 or n, k > 2^31 - 1");
  need(a, m * k, "gemm_i8: A size");
  need(b, k * n, "gemm_i8: B size");
  need(c_i32, m * n * 4, "gemm_i8: C size");
  dw::launch_gemm(bk->stream, dw::I8, a->ptr, b->ptr, c_i32->ptr, (int)m, (int)n, (int)k);
  API_END
}

int dw_hip_global_avg_pool_nhwc(dw_hip_backend* be, int dtype, const dw_hip_buffer* x, dw_hip_buffer* y,
                                size_t n, size_t h, size_t w, size_t c) {
  API_BEGIN
  Backend* bk = B(be);
  std::lock_guard<std::mutex> lock(bk->mu);
  if (dtype != DW_DTYPE_F32 && dtype != DW_DTYPE_F16)
    dw::fail(DW_ERR_UNSUPPORTED, "global_avg_pool: unsupported dtype");
  if (!n || !h || !w || !c) dw::fail(DW_ERR_INVALID, "global_avg_pool: zero size");
  if (h * w > INT32_MAX || n > 65535 || c > INT32_MAX) dw::fail(DW_ERR_UNSUPPORTED, "global_avg_pool: size");
  const size_t es = dw::dtype_size(dtype);
  need(x, n * h * w * c * es, "global_avg_pool: input size");
  need(y, n * c * es, "global_avg_pool: output size");
  dw::launch_global_avg_pool(bk->stream, dtype, x->ptr, y->ptr, (int)n, (int)(h * w), (int)c);
  API_END
}

int dw_hip_softmax_f32(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t rows, size_t n) {
  API_BEGIN
  Backend* bk = B(be);
  std::lock_guard<std::mutex> lock(bk->mu);
  if (!rows || !n) dw::fail(DW_ERR_INVALID, "softmax_f32: zero size");
  if (rows > INT32_MAX || n > INT32_MAX) dw::fail(DW_ERR_UNSUPPORTED, "softmax_f32: size");
  need(x, rows * n * 4, "softmax_f32: input size");
  need(y, rows * n * 4, "softmax_f32: output size");
  dw::launch_softmax_rows(bk->stream, (const float*)x->ptr, (float*)y->ptr, (int)rows, (int)n);
  API_END
}

static size_t dtype_bytes(int dtype) {
  if (dtype == DW_DTYPE_F32 || dtype == DW_DTYPE_I32) return 4;
  if (dtype == DW_DTYPE_F16) return 2;
  if (dtype == DW_DTYPE_I8 || dtype == DW_DTYPE_U8) return 1;
  dw::fail(DW_ERR_INVALID, "unknown dtype");
}

int dw_hip_transpose_nchw_to_nhwc(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t n, size_t c,
                                  size_t h, size_t w, int dtype) {
  API_BEGIN
  Backend* bk = B(be);
  std::lock_guard<std::mutex> lock(bk->mu);
  const size_t es = dtype_bytes(dtype);
  if (!n || !c || !h || !w) dw::fail(DW_ERR_INVALID, "transpose: zero size");
  check_i32(c * h * w, "transpose: image");
  if (n > 65535) dw::fail(DW_ERR_UNSUPPORTED, "transpose: batch above 65535");
  need(x, n * c * h * w * es, "transpose: input");
  need(y, n * c * h * w * es, "transpose: output");
  dw::launch_transpose(bk->stream, x->ptr, y->ptr, (int)n, (int)c, (int)(h * w), (int)es);
  API_END
}

int dw_hip_transpose_nhwc_to_nchw(dw_hip_backend* be, const dw_hip_buffer* x, dw_hip_buffer* y, size_t n, size_t h,
                                  size_t w, size_t c, int dtype) {
  API_BEGIN
  Backend* bk = B(be);
  std::lock_guard<std::mutex> lock(bk->mu);
  const size_t es = dtype_bytes(dtype);
  if (!n || !c || !h || !w) dw::fail(DW_ERR_INVALID, "transpose: zero size");
  check_i32(c * h * w, "transpose: image");
  if (n > 65535) dw::fail(DW_ERR_UNSUPPORTED, "transpose: batch above 65535");
  need(x, n * c * h * w * es, "transpose: input");
  need(y, n * c * h * w * es, "transpose: output");
  dw::launch_transpose(bk->stream, x->ptr, y->ptr, (int)n, (int)(h * w), (int)c, (int)es);
  API_END
}

int dw_hip_fold_batchnorm(dw_hip_backend* be, const dw_hip_buffer* w, const dw_hip_buffer* bias_in,
                          const dw_hip_buffer* gamma, const dw_hip_buffer* beta, const dw_hip_buffer* mean,
                          const dw_hip_buffer* var, float epsilon, size_t c_out, size_t per_channel,
                          dw_hip_buffer* w_out, dw_hip_buffer* bias_out) {
  API_BEGIN
  Backend* bk = B(be);
  std::lock_guard<std::mutex> lock(bk->mu);
  if (!c_out || !per_channel) dw::fail(DW_ERR_INVALID, "fold_batchnorm: zero size");
  if (c_out > 65535) dw::fail(DW_ERR_UNSUPPORTED, "fold_batchnorm: more than 65535 channels");
  check_i32(c_out * per_channel, "fold_batchnorm: weights");
  need(w, c_out * per_channel * 4, "fold_batchnorm: weights");
  need(w_out, c_out * per_channel * 4, "fold_batchnorm: output weights");
  if (bias_in) need(bias_in, c_out * 4, "fold_batchnorm: bias");
  need(gamma, c_out * 4, "fold_batchnorm: gamma");
  need(beta, c_out * 4, "fold_batchnorm: beta");
  need(mean, c_out * 4, "fold_batchnorm: mean");
  need(var, c_out * 4, "fold_batchnorm: var");
  need(bias_out, c_out * 4, "fold_batchnorm: output bias");
  dw::launch_fold_batchnorm(bk->stream, (const float*)w->ptr, bias_in ? (const float*)bias_in->ptr : nullptr,
                            (const float*)gamma->ptr, (const float*)beta->ptr, (const float*)mean->ptr,
                            (const float*)var->ptr, epsilon, (int)c_out, (int)per_channel, (float*)w_out->ptr,
                            (float*)bias_out->ptr);
  API_END
}

int dw_hip_yolo_detect_tail(dw_hip_backend* be, int dtype, const dw_hip_buffer* const* levels, const int* h,
                            const int* w, const float* strides, int num_levels, size_t n, int nc, int reg_max,
                            dw_hip_buffer* out) {
  API_BEGIN
  Backend* bk = B(be);
  std::lock_guard<std::mutex> lock(bk->mu);
  if (!levels || !h || !w || !strides) dw::fail(DW_ERR_INVALID, "detect tail: null argument");
  if (num_levels < 1 || num_levels > 4) dw::fail(DW_ERR_UNSUPPORTED, "detect tail: 1 to 4 levels");
  if (dtype != DW_DTYPE_F16 && dtype != DW_DTYPE_F32) dw::fail(DW_ERR_UNSUPPORTED, "detect tail: f16 or f32");
  if (!n || nc < 1 || reg_max < 1) dw::fail(DW_ERR_INVALID, "detect tail: zero size");
  check_i32(n, "detect tail: batch");
  const size_t es = dtype == DW_DTYPE_F16 ? 2 : 4;
  const size_t pix = (size_t)4 * reg_max + (size_t)nc;
  dw::DetectTailArgs t{};
  size_t A = 0;
  for (int s = 0; s < num_levels; ++s) {
    if (h[s] < 1 || w[s] < 1) dw::fail(DW_ERR_INVALID, "detect tail: empty level");
    need(levels[s], n * (size_t)h[s] * w[s] * pix * es, "detect tail: level size");
    t.x[s] = levels[s]->ptr;
    t.h[s] = h[s];
    t.w[s] = w[s];
    t.pix[s] = (int)pix;
    t.stride[s] = strides[s];
    A += (size_t)h[s] * w[s];
  }
  check_i32(A * (4 + nc), "detect tail: output row");
  need(out, n * (4 + (size_t)nc) * A * 4, "detect tail: output size");
  t.levels = num_levels;
  t.nc = nc;
  t.reg_max = reg_max;
  dw::launch_detect_tail(bk->stream, dtype == DW_DTYPE_F16 ? dw::F16 : dw::F32, t, (float*)out->ptr, (int)n);
  API_END
}

int dw_hip_yolo_postprocess(dw_hip_backend* be, const dw_hip_buffer* raw, size_t n, int nc, size_t num_det,
                            uint32_t img_w, uint32_t img_h, float conf_threshold, float iou_threshold,
                            int agnostic, dw_detection* out, size_t cap, size_t* counts) {
  API_BEGIN
  Backend* bk = B(be);
  std::lock_guard<std::mutex> lock(bk->mu);
  static_assert(sizeof(dw_detection) == sizeof(dw::DwDetection), "detection layout");
  if (!counts || (cap && !out)) dw::fail(DW_ERR_INVALID, "postprocess: null output");
  if (!n || nc < 1 || !num_det) dw::fail(DW_ERR_INVALID, "postprocess: zero size");
  if (nc > 1024) dw::fail(DW_ERR_UNSUPPORTED, "postprocess: more than 1024 classes");
  if (num_det > 16384) dw::fail(DW_ERR_UNSUPPORTED, "postprocess: more than 16384 anchors per image");
  check_i32(n, "postprocess: batch");
  need(raw, n * (4 + (size_t)nc) * num_det * 4, "postprocess: raw output size");
  int dev_lds = 0;
  DW_HIP(hipDeviceGetAttribute(&dev_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, bk->device));
  const int nmax = dw::kPPMaxCandidates;
  if ((size_t)dev_lds < dw::pp_nms_lds_bytes(nmax)) dw::fail(DW_ERR_UNSUPPORTED, "postprocess: LDS per workgroup");
  // workspace: keys, per-anchor detections, then per image nmax-sized arrays
  const size_t A = num_det;
  auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
  const size_t o_keys = 0, o_det = o_keys + al(n * A * 8), o_sa = o_det + al(n * A * 24);
  const size_t o_pp = o_sa + al(n * nmax * 4), o_od = o_pp + al(n * nmax * 4);
  const size_t o_op = o_od + al(n * nmax * 24), o_cnt = o_op + al(n * nmax * 4), total = o_cnt + al(n * 16);
  uint8_t* ws = (uint8_t*)bk->workspace(Backend::WS_POST, total);
  dw::PostprocessArgs a{};
  a.raw = (const float*)raw->ptr;
  a.n = (int)n;
  a.nc = nc;
  a.A = (int)A;
  const float model = 640.0f;  // the reference's fixed model size (postprocess.rs:98)
  a.sx = (float)img_w / model;
  a.sy = (float)img_h / model;
  a.img_w = (float)img_w;
  a.img_h = (float)img_h;
  a.conf = conf_threshold;
  a.iou = iou_threshold;
  a.agnostic = agnostic ? 1 : 0;
  a.nmax = nmax;
  a.keys = (unsigned long long*)(ws + o_keys);
  a.det = (dw::DwDetection*)(ws + o_det);
  a.sorted_anchor = (int*)(ws + o_sa);
  a.part_pos = (int*)(ws + o_pp);
  a.out_det = (dw::DwDetection*)(ws + o_od);
  a.out_pos = (int*)(ws + o_op);
  a.counts = (int*)(ws + o_cnt);
  dw::launch_yolo_postprocess(bk->stream, a);
  std::vector<int> cnt(n * 4);
  DW_HIP(hipMemcpyAsync(cnt.data(), a.counts, n * 16, hipMemcpyDeviceToHost, bk->stream));
  DW_HIP(hipStreamSynchronize(bk->stream));
  size_t maxk = 0;
  for (size_t b = 0; b < n; ++b) {
    if (cnt[4 * b + 2])
      dw::fail(DW_ERR_UNSUPPORTED, "postprocess: image " + std::to_string(b) + " has " +
                                       std::to_string(cnt[4 * b]) + " candidates over the threshold (at most " +
                                       std::to_string(nmax) + ")");
    maxk = std::max(maxk, (size_t)cnt[4 * b + 1]);
  }
  std::vector<dw::DwDetection> kd(n * (size_t)nmax);
  std::vector<int> kp(n * (size_t)nmax);
  if (maxk) {
    DW_HIP(hipMemcpy2DAsync(kd.data(), (size_t)nmax * 24, a.out_det, (size_t)nmax * 24, maxk * 24, n,
                            hipMemcpyDeviceToHost, bk->stream));
    DW_HIP(hipMemcpy2DAsync(kp.data(), (size_t)nmax * 4, a.out_pos, (size_t)nmax * 4, maxk * 4, n,
                            hipMemcpyDeviceToHost, bk->stream));
    DW_HIP(hipStreamSynchronize(bk->stream));
  }
  // The reference removes suppressed entries from the back with swap_remove
  // (postprocess.rs:235-242): walking the sorted positions downwards, a
  // suppressed slot takes the current last element and the list shrinks.
  // Replayed on slots that name kept detections (-1: suppressed).
  bool over = false;
  std::vector<int> slot;
  for (size_t b = 0; b < n; ++b) {
    const int nc_b = cnt[4 * b], k = cnt[4 * b + 1];
    counts[b] = (size_t)k;
    if ((size_t)k > cap) {
      over = true;
      continue;
    }
    slot.assign((size_t)nc_b, -1);
    for (int i = 0; i < k; ++i) slot[(size_t)kp[b * nmax + i]] = i;
    int len = nc_b;
    for (int i = nc_b - 1; i >= 0; --i)
      if (slot[(size_t)i] < 0) {
        slot[(size_t)i] = slot[(size_t)len - 1];
        --len;
      }
    dw_detection* o = out + b * cap;
    for (int i = 0; i < len; ++i) memcpy(&o[i], &kd[b * nmax + (size_t)slot[(size_t)i]], sizeof(dw_detection));
  }
  if (over) dw::fail(DW_ERR_INVALID, "postprocess: more detections than cap in an image (see counts)");
  API_END
}

}  // extern "C"
