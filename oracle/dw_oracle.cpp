// ============================================================================
// dragonwing-cpu oracle — TEST INFRASTRUCTURE ONLY.
//
// A CPU restatement of the dragonwing-edge-rs algorithms on the MI355X
// backend's hot path, used as the checker for parity tests, by smoke() and
// as bench.py's cpu_baseline.  Nothing in the product links or calls this
// library.  Every function cites the reference file:line it follows
// (paths relative to the dragonwing-edge-rs tree).  The x86-64 reference
// takes the scalar paths (e.g. crates/dragonwing-cpu/src/ops.rs:57-60), so
// those are the ones restated.
//
// Part A: functions the reference implements (pinned by its known-answer
//         tests, see tests/test_oracle_*.py).
// Part B: ONNX quantized extensions the reference does NOT implement
//         (QLinearConv u8 x s8 with zero points and round-half-even,
//         QuantizeLinear/DequantizeLinear, QLinearAdd, padded MaxPool,
//         quantized activation tables).  Pinned by closed forms, hand-made
//         fixtures and brute force, as stated in the tests.
//
// Build: -O3, default x86-64 ISA, no fast-math, no FP contraction
// (the reference's cargo --release profile never contracts either).
// ============================================================================
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

extern "C" {

// ---------------------------------------------------------------------------
// Part A.1 — F16 (crates/dragonwing-core/src/dtype.rs:164-263)
// ---------------------------------------------------------------------------

// F16::from_f32_soft (dtype.rs:164-222): IEEE binary16, round to nearest
// even, subnormals kept, overflow -> inf, NaN -> 0x7E00 | payload.
uint16_t dwo_f16_from_f32(float v) {
  uint32_t bits;
  memcpy(&bits, &v, 4);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const int32_t exp = (int32_t)((bits >> 23) & 0xFF);
  const uint32_t mant = bits & 0x007FFFFFu;
  if (exp == 255) {
    if (mant == 0) return (uint16_t)(sign | 0x7C00u);
    uint32_t pay = mant >> 13;
    if (pay > 0x1FF) pay = 0x1FF;
    return (uint16_t)(sign | 0x7E00u | pay);
  }
  const int32_t new_exp = exp - 127 + 15;
  if (new_exp >= 31) return (uint16_t)(sign | 0x7C00u);
  if (new_exp <= 0) {
    if (new_exp < -10) return (uint16_t)sign;
    const int32_t shift = 1 - new_exp;
    const uint32_t mh = mant | 0x00800000u;
    const uint32_t shifted = mh >> (13 + shift);
    const uint32_t round_bit = (mh >> (12 + shift)) & 1u;
    const uint32_t sticky = (mh & ((1u << (12 + shift)) - 1u)) != 0 ? 1u : 0u;
    const uint32_t rounded = shifted + (round_bit & (sticky | (shifted & 1u)));
    return (uint16_t)(sign | rounded);
  }
  const uint32_t m16 = mant >> 13;
  const uint32_t round_bit = (mant >> 12) & 1u;
  const uint32_t sticky = (mant & 0x0FFFu) != 0 ? 1u : 0u;
  const uint32_t rounded = m16 + (round_bit & (sticky | (m16 & 1u)));
  if (rounded >= 0x400u) {
    const int32_t e2 = new_exp + 1;
    if (e2 >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((uint32_t)e2 << 10));
  }
  return (uint16_t)(sign | ((uint32_t)new_exp << 10) | rounded);
}

// F16::to_f32_soft (dtype.rs:226-263): exact widening.
float dwo_f16_to_f32(uint16_t h) {
  const uint32_t bits = h;
  const uint32_t sign = (bits & 0x8000u) << 16;
  const uint32_t exp = (bits >> 10) & 0x1Fu;
  const uint32_t mant = bits & 0x03FFu;
  uint32_t out;
  if (exp == 0) {
    if (mant == 0) {
      out = sign;
    } else {
      uint32_t m = mant;
      int32_t e = 0;
      while ((m & 0x0400u) == 0) {
        m <<= 1;
        ++e;
      }
      out = sign | ((uint32_t)(127 - 15 - e) << 23) | ((m & 0x03FFu) << 13);
    }
  } else if (exp == 31) {
    out = mant == 0 ? (sign | 0x7F800000u) : (sign | 0x7FC00000u | (mant << 13));
  } else {
    out = sign | ((exp + 127 - 15) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &out, 4);
  return f;
}

void dwo_f32_to_f16_array(const float* x, uint16_t* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = dwo_f16_from_f32(x[i]);
}
void dwo_f16_to_f32_array(const uint16_t* x, float* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = dwo_f16_to_f32(x[i]);
}

// ---------------------------------------------------------------------------
// Part A.2 — thread pool semantics (crates/dragonwing-cpu/src/pool.rs)
// ---------------------------------------------------------------------------

// num_cpus (pool.rs:222-264): count of /sys/devices/system/cpu/online.
int dwo_num_cpus(void) {
  FILE* f = fopen("/sys/devices/system/cpu/online", "r");
  if (f) {
    char buf[256] = {0};
    size_t r = fread(buf, 1, sizeof buf - 1, f);
    fclose(f);
    buf[r] = 0;
    int count = 0;
    char* p = buf;
    bool ok = r > 0;
    while (ok && *p && *p != '\n') {
      char* end;
      long a = strtol(p, &end, 10);
      if (end == p) { ok = false; break; }
      long b = a;
      p = end;
      if (*p == '-') {
        ++p;
        b = strtol(p, &end, 10);
        if (end == p) { ok = false; break; }
        p = end;
      }
      count += (int)(b - a + 1);
      if (*p == ',') ++p;
    }
    if (ok && count > 0) return count;
  }
  unsigned hc = std::thread::hardware_concurrency();
  return hc ? (int)hc : 1;
}

}  // extern "C"

// parallel_for_scoped (pool.rs:317-350): chunk = ceil(total / threads),
// thread i runs [i*chunk, min((i+1)*chunk, total)).
template <typename F>
static void parallel_for_scoped(int num_threads, size_t total, F f) {
  if (total == 0) return;
  size_t nt = std::max<size_t>(1, std::min<size_t>((size_t)num_threads, total));
  if (nt <= 1) {
    f((size_t)0, total);
    return;
  }
  const size_t chunk = (total + nt - 1) / nt;
  std::vector<std::thread> ts;
  for (size_t i = 0; i < nt; ++i) {
    const size_t s = i * chunk, e = std::min(total, (i + 1) * chunk);
    if (s >= total) break;
    ts.emplace_back([=] { f(s, e); });
  }
  for (auto& t : ts) t.join();
}

static inline size_t out_dim(size_t in, size_t pad, size_t k, size_t s) { return (in + 2 * pad - k) / s + 1; }

extern "C" {

// ---------------------------------------------------------------------------
// Part A.3 — convolutions (crates/dragonwing-cpu/src/ops.rs)
// ---------------------------------------------------------------------------

// Rows [r0, r1) of n*h_out of conv2d_f32_nhwc (ops.rs:1356-1436): for each
// output, acc = 0; kh -> kw (out-of-image taps skipped) -> ic:
// acc = x.mul_add(w, acc).  HWIO kernel, NHWC in/out.
static void conv_f32_rows(float* out, const float* in, const float* ker, size_t h_in, size_t w_in,
                          size_t c_in, size_t c_out, size_t k_h, size_t k_w, size_t sh, size_t sw,
                          size_t ph, size_t pw, size_t h_out, size_t w_out, size_t r0, size_t r1) {
  for (size_t row = r0; row < r1; ++row) {
    const size_t b = row / h_out, oh = row % h_out;
    for (size_t ow = 0; ow < w_out; ++ow) {
      for (size_t oc = 0; oc < c_out; ++oc) {
        float acc = 0.0f;
        for (size_t kh = 0; kh < k_h; ++kh) {
          for (size_t kw = 0; kw < k_w; ++kw) {
            const long ih = (long)(oh * sh + kh) - (long)ph;
            const long iw = (long)(ow * sw + kw) - (long)pw;
            if (ih < 0 || ih >= (long)h_in || iw < 0 || iw >= (long)w_in) continue;
            const float* xp = in + ((b * h_in + (size_t)ih) * w_in + (size_t)iw) * c_in;
            const float* wp = ker + ((kh * k_w + kw) * c_in) * c_out + oc;
            for (size_t ic = 0; ic < c_in; ++ic) acc = fmaf(xp[ic], wp[ic * c_out], acc);
          }
        }
        out[((b * h_out + oh) * w_out + ow) * c_out + oc] = acc;
      }
    }
  }
}

// conv2d_f32_nhwc (ops.rs:1356-1436), single thread.
void dwo_conv2d_f32_nhwc(float* out, const float* in, const float* ker, size_t n, size_t h_in,
                         size_t w_in, size_t c_in, size_t c_out, size_t k_h, size_t k_w, size_t sh,
                         size_t sw, size_t ph, size_t pw) {
  const size_t ho = out_dim(h_in, ph, k_h, sh), wo = out_dim(w_in, pw, k_w, sw);
  conv_f32_rows(out, in, ker, h_in, w_in, c_in, c_out, k_h, k_w, sh, sw, ph, pw, ho, wo, 0, n * ho);
}

// conv2d_f32_nhwc_mt (ops.rs:1756-1837): serial below 8192 MAC-elements or
// one thread, else rows of n*h_out split with parallel_for_scoped over
// min(threads, n*h_out, num_cpus()) threads.  Same arithmetic per output.
void dwo_conv2d_f32_nhwc_mt(float* out, const float* in, const float* ker, size_t n, size_t h_in,
                            size_t w_in, size_t c_in, size_t c_out, size_t k_h, size_t k_w, size_t sh,
                            size_t sw, size_t ph, size_t pw, int num_threads) {
  const size_t ho = out_dim(h_in, ph, k_h, sh), wo = out_dim(w_in, pw, k_w, sw);
  const size_t work = n * ho * wo * c_out * k_h * k_w * c_in;
  if (work < 8192 || num_threads <= 1) {
    dwo_conv2d_f32_nhwc(out, in, ker, n, h_in, w_in, c_in, c_out, k_h, k_w, sh, sw, ph, pw);
    return;
  }
  const int nt = (int)std::min<size_t>(std::min<size_t>((size_t)num_threads, n * ho), (size_t)dwo_num_cpus());
  parallel_for_scoped(nt, n * ho, [&](size_t r0, size_t r1) {
    conv_f32_rows(out, in, ker, h_in, w_in, c_in, c_out, k_h, k_w, sh, sw, ph, pw, ho, wo, r0, r1);
  });
}

// conv2d_fp16_nhwc_mt (ops.rs:2572-2651; single-thread form :1442-1500):
// identical loop on F16 storage with to_f32() of every operand and
// F16::from_f32(acc) at the end.  to_f32 is exact, so operands are widened
// once up front; the per-output FMA sequence is unchanged.
void dwo_conv2d_fp16_nhwc_mt(uint16_t* out, const uint16_t* in, const uint16_t* ker, size_t n,
                             size_t h_in, size_t w_in, size_t c_in, size_t c_out, size_t k_h,
                             size_t k_w, size_t sh, size_t sw, size_t ph, size_t pw, int num_threads) {
  const size_t ho = out_dim(h_in, ph, k_h, sh), wo = out_dim(w_in, pw, k_w, sw);
  std::vector<float> fi(n * h_in * w_in * c_in), fk(k_h * k_w * c_in * c_out), fo(n * ho * wo * c_out);
  dwo_f16_to_f32_array(in, fi.data(), fi.size());
  dwo_f16_to_f32_array(ker, fk.data(), fk.size());
  dwo_conv2d_f32_nhwc_mt(fo.data(), fi.data(), fk.data(), n, h_in, w_in, c_in, c_out, k_h, k_w, sh, sw,
                         ph, pw, num_threads);
  dwo_f32_to_f16_array(fo.data(), out, fo.size());
}

static void dw_rows_f32(float* out, const float* in, const float* ker, size_t h_in, size_t w_in,
                        size_t c_in, size_t mult, size_t k_h, size_t k_w, size_t sh, size_t sw, size_t ph,
                        size_t pw, size_t ho, size_t wo, size_t r0, size_t r1) {
  const size_t c_out = c_in * mult;
  for (size_t row = r0; row < r1; ++row) {
    const size_t b = row / ho, oh = row % ho;
    for (size_t ow = 0; ow < wo; ++ow)
      for (size_t ic = 0; ic < c_in; ++ic)
        for (size_t m = 0; m < mult; ++m) {
          float acc = 0.0f;
          for (size_t kh = 0; kh < k_h; ++kh)
            for (size_t kw = 0; kw < k_w; ++kw) {
              const long ih = (long)(oh * sh + kh) - (long)ph;
              const long iw = (long)(ow * sw + kw) - (long)pw;
              if (ih < 0 || ih >= (long)h_in || iw < 0 || iw >= (long)w_in) continue;
              acc = fmaf(in[((b * h_in + (size_t)ih) * w_in + (size_t)iw) * c_in + ic],
                         ker[((kh * k_w + kw) * c_in + ic) * mult + m], acc);
            }
          out[((b * ho + oh) * wo + ow) * c_out + ic * mult + m] = acc;
        }
  }
}

// depthwise_conv2d_f32_nhwc_mt (ops.rs:2734-2815): kernel [kh][kw][c][mult];
// serial below 4096 work or one thread.
void dwo_depthwise_conv2d_f32_nhwc_mt(float* out, const float* in, const float* ker, size_t n,
                                      size_t h_in, size_t w_in, size_t c_in, size_t mult, size_t k_h,
                                      size_t k_w, size_t sh, size_t sw, size_t ph, size_t pw,
                                      int num_threads) {
  const size_t ho = out_dim(h_in, ph, k_h, sh), wo = out_dim(w_in, pw, k_w, sw);
  const size_t work = n * ho * wo * c_in * mult * k_h * k_w;
  if (work < 4096 || num_threads <= 1) {
    dw_rows_f32(out, in, ker, h_in, w_in, c_in, mult, k_h, k_w, sh, sw, ph, pw, ho, wo, 0, n * ho);
    return;
  }
  const int nt = (int)std::min<size_t>(std::min<size_t>((size_t)num_threads, n * ho), (size_t)dwo_num_cpus());
  parallel_for_scoped(nt, n * ho, [&](size_t r0, size_t r1) {
    dw_rows_f32(out, in, ker, h_in, w_in, c_in, mult, k_h, k_w, sh, sw, ph, pw, ho, wo, r0, r1);
  });
}

// depthwise_conv2d_fp16_nhwc_mt (ops.rs:2819-2933): as above on F16
// storage (exact widening up front), F16::from_f32(acc) per output.
void dwo_depthwise_conv2d_fp16_nhwc_mt(uint16_t* out, const uint16_t* in, const uint16_t* ker,
                                       size_t n, size_t h_in, size_t w_in, size_t c_in, size_t mult,
                                       size_t k_h, size_t k_w, size_t sh, size_t sw, size_t ph,
                                       size_t pw, int num_threads) {
  const size_t ho = out_dim(h_in, ph, k_h, sh), wo = out_dim(w_in, pw, k_w, sw);
  std::vector<float> fi(n * h_in * w_in * c_in), fk(k_h * k_w * c_in * mult), fo(n * ho * wo * c_in * mult);
  dwo_f16_to_f32_array(in, fi.data(), fi.size());
  dwo_f16_to_f32_array(ker, fk.data(), fk.size());
  dwo_depthwise_conv2d_f32_nhwc_mt(fo.data(), fi.data(), fk.data(), n, h_in, w_in, c_in, mult, k_h,
                                   k_w, sh, sw, ph, pw, num_threads);
  dwo_f32_to_f16_array(fo.data(), out, fo.size());
}

static void conv_i8_rows(int32_t* out, const int8_t* in, const int8_t* ker, size_t h_in, size_t w_in,
                         size_t c_in, size_t c_out, size_t k_h, size_t k_w, size_t sh, size_t sw,
                         size_t ph, size_t pw, size_t ho, size_t wo, size_t r0, size_t r1) {
  for (size_t row = r0; row < r1; ++row) {
    const size_t b = row / ho, oh = row % ho;
    for (size_t ow = 0; ow < wo; ++ow)
      for (size_t oc = 0; oc < c_out; ++oc) {
        int32_t acc = 0;
        for (size_t kh = 0; kh < k_h; ++kh)
          for (size_t kw = 0; kw < k_w; ++kw) {
            const long ih = (long)(oh * sh + kh) - (long)ph;
            const long iw = (long)(ow * sw + kw) - (long)pw;
            if (ih < 0 || ih >= (long)h_in || iw < 0 || iw >= (long)w_in) continue;
            const int8_t* xp = in + ((b * h_in + (size_t)ih) * w_in + (size_t)iw) * c_in;
            const int8_t* wp = ker + ((kh * k_w + kw) * c_in) * c_out + oc;
            for (size_t ic = 0; ic < c_in; ++ic) acc += (int32_t)xp[ic] * (int32_t)wp[ic * c_out];
          }
        out[((b * ho + oh) * wo + ow) * c_out + oc] = acc;
      }
  }
}

// conv2d_i8_nhwc (ops.rs:3086-3142): s8 x s8 -> i32, zero padding, single
// threaded (the reference has no multi-threaded variant).
void dwo_conv2d_i8_nhwc(int32_t* out, const int8_t* in, const int8_t* ker, size_t n, size_t h_in,
                        size_t w_in, size_t c_in, size_t c_out, size_t k_h, size_t k_w, size_t sh,
                        size_t sw, size_t ph, size_t pw) {
  const size_t ho = out_dim(h_in, ph, k_h, sh), wo = out_dim(w_in, pw, k_w, sw);
  conv_i8_rows(out, in, ker, h_in, w_in, c_in, c_out, k_h, k_w, sh, sw, ph, pw, ho, wo, 0, n * ho);
}

// Row-parallel variant of dwo_conv2d_i8_nhwc (not in the reference; integer
// sums are order-independent, so the result is bit-identical).  Used only
// to time a multi-core CPU baseline.
void dwo_conv2d_i8_nhwc_rowpar(int32_t* out, const int8_t* in, const int8_t* ker, size_t n,
                               size_t h_in, size_t w_in, size_t c_in, size_t c_out, size_t k_h,
                               size_t k_w, size_t sh, size_t sw, size_t ph, size_t pw, int num_threads) {
  const size_t ho = out_dim(h_in, ph, k_h, sh), wo = out_dim(w_in, pw, k_w, sw);
  parallel_for_scoped(num_threads, n * ho, [&](size_t r0, size_t r1) {
    conv_i8_rows(out, in, ker, h_in, w_in, c_in, c_out, k_h, k_w, sh, sw, ph, pw, ho, wo, r0, r1);
  });
}

// ---------------------------------------------------------------------------
// Part A.4 — CpuGraphRuntime conv bias passes
// (crates/dragonwing-onnx/src/runtime.rs:1445-1460 f32, :1483-1498 f16)
// ---------------------------------------------------------------------------
void dwo_bias_add_f32_nhwc(float* y, const float* bias, size_t pixels, size_t c) {
  for (size_t p = 0; p < pixels; ++p)
    for (size_t ch = 0; ch < c; ++ch) y[p * c + ch] += bias[ch];
}
void dwo_bias_add_f16_nhwc(uint16_t* y, const uint16_t* bias, size_t pixels, size_t c) {
  for (size_t p = 0; p < pixels; ++p)
    for (size_t ch = 0; ch < c; ++ch)
      y[p * c + ch] = dwo_f16_from_f32(dwo_f16_to_f32(y[p * c + ch]) + dwo_f16_to_f32(bias[ch]));
}

// ---------------------------------------------------------------------------
// Part A.5 — elementwise (ops.rs)
// ---------------------------------------------------------------------------
// relu_f32_scalar (ops.rs:208-220): >0 keeps x, NaN propagates, else +0.
void dwo_relu_f32(float* y, const float* x, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const float v = x[i];
    y[i] = v > 0.0f ? v : (v != v ? v : 0.0f);
  }
}
// relu_fp16 (ops.rs:345-352)
void dwo_relu_fp16(uint16_t* y, const uint16_t* x, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const float v = dwo_f16_to_f32(x[i]);
    y[i] = dwo_f16_from_f32(v > 0.0f ? v : 0.0f);
  }
}
// add_f32_scalar (ops.rs:378-384), add_fp16 (ops.rs:434-442)
void dwo_add_f32(float* y, const float* a, const float* b, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = a[i] + b[i];
}
void dwo_add_fp16(uint16_t* y, const uint16_t* a, const uint16_t* b, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = dwo_f16_from_f32(dwo_f16_to_f32(a[i]) + dwo_f16_to_f32(b[i]));
}
// mul_f32_scalar (ops.rs:1913-1919), mul_fp16 (ops.rs:1959-1967)
void dwo_mul_f32(float* y, const float* a, const float* b, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = a[i] * b[i];
}
void dwo_mul_fp16(uint16_t* y, const uint16_t* a, const uint16_t* b, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = dwo_f16_from_f32(dwo_f16_to_f32(a[i]) * dwo_f16_to_f32(b[i]));
}
// sigmoid_f32_scalar (ops.rs:1865-1870): 1 / (1 + exp(-x)), exp = libm expf.
void dwo_sigmoid_f32(float* y, const float* x, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = 1.0f / (1.0f + expf(-x[i]));
}
// sigmoid_fp16 (ops.rs:1881-1888)
void dwo_sigmoid_fp16(uint16_t* y, const uint16_t* x, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const float v = dwo_f16_to_f32(x[i]);
    y[i] = dwo_f16_from_f32(1.0f / (1.0f + expf(-v)));
  }
}

// ---------------------------------------------------------------------------
// Part A.6 — reference INT8 (symmetric, zero point 0)
// ---------------------------------------------------------------------------
// requantize_i32_to_i8_scalar (ops.rs:3380-3386): (x as f32) * s, clamp
// [-128,127], f32::round (half away from zero).
void dwo_requantize_i32_to_i8(int8_t* y, const int32_t* x, size_t n, float s) {
  for (size_t i = 0; i < n; ++i) {
    float f = (float)x[i] * s;
    f = f < -128.0f ? -128.0f : (f > 127.0f ? 127.0f : f);
    y[i] = (int8_t)roundf(f);
  }
}
// quantize_f32_to_i8 (ops.rs:3503-3525): inv = 1/scale; round(clamp(x*inv)).
void dwo_quantize_f32_to_i8(int8_t* y, const float* x, size_t n, float scale) {
  const float inv = 1.0f / scale;
  for (size_t i = 0; i < n; ++i) {
    float f = x[i] * inv;
    f = f < -128.0f ? -128.0f : (f > 127.0f ? 127.0f : f);
    y[i] = (int8_t)roundf(f);
  }
}
// dequantize_i8_to_f32_scalar (ops.rs:3453-3457)
void dwo_dequantize_i8_to_f32(float* y, const int8_t* x, size_t n, float scale) {
  for (size_t i = 0; i < n; ++i) y[i] = (float)x[i] * scale;
}
// add_i8_scalar (ops.rs:3197-3209)
void dwo_add_i8(int8_t* y, const int8_t* a, const int8_t* b, size_t n, float sa, float sb) {
  for (size_t i = 0; i < n; ++i) {
    float r = (float)a[i] * sa + (float)b[i] * sb;
    r = r < -128.0f ? -128.0f : (r > 127.0f ? 127.0f : r);
    y[i] = (int8_t)roundf(r);
  }
}
// relu_i8_scalar (ops.rs:3315-3320)
void dwo_relu_i8(int8_t* y, const int8_t* x, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = x[i] > 0 ? x[i] : 0;
}
// QuantScale::from_range (crates/dragonwing-core/src/quantization.rs:85-89)
float dwo_scale_from_range(float mn, float mx) {
  const float a = fmaxf(fabsf(mn), fabsf(mx));
  return a > 0.0f ? a / 127.0f : 1.0f;
}
// PerChannelScale::from_weights (quantization.rs:150-170) over `channels`
// contiguous rows, then quantize_weights_per_channel
// (crates/dragonwing-onnx/src/quantize.rs:344-368): q = clamp(round(w * (1/s))).
void dwo_quantize_weights_per_channel(int8_t* q, float* scales, const float* w, size_t channels,
                                      size_t per_channel) {
  for (size_t c = 0; c < channels; ++c) {
    float am = 0.0f;
    for (size_t k = 0; k < per_channel; ++k) am = fmaxf(am, fabsf(w[c * per_channel + k]));
    const float s = am > 0.0f ? am / 127.0f : 1.0f;
    scales[c] = s;
    const float inv = 1.0f / s;
    for (size_t k = 0; k < per_channel; ++k) {
      float r = roundf(w[c * per_channel + k] * inv);
      r = r < -128.0f ? -128.0f : (r > 127.0f ? 127.0f : r);
      q[c * per_channel + k] = (int8_t)r;
    }
  }
}

// ---------------------------------------------------------------------------
// Part A.7 — data movement (ops.rs)
// ---------------------------------------------------------------------------
// maxpool2d_f32_nhwc (ops.rs:1513-1552): unpadded window max, start -inf,
// f32::max.
void dwo_maxpool2d_f32_nhwc(float* out, const float* in, size_t n, size_t h_in, size_t w_in, size_t c,
                            size_t ph_, size_t pw_, size_t sh, size_t sw) {
  const size_t ho = (h_in - ph_) / sh + 1, wo = (w_in - pw_) / sw + 1;
  for (size_t b = 0; b < n; ++b)
    for (size_t oh = 0; oh < ho; ++oh)
      for (size_t ow = 0; ow < wo; ++ow)
        for (size_t ch = 0; ch < c; ++ch) {
          float m = -INFINITY;
          for (size_t y = 0; y < ph_; ++y)
            for (size_t x = 0; x < pw_; ++x)
              m = fmaxf(m, in[((b * h_in + oh * sh + y) * w_in + ow * sw + x) * c + ch]);
          out[((b * ho + oh) * wo + ow) * c + ch] = m;
        }
}
// resize_f32 Nearest (ops.rs:2320-2351), any element size (a pure copy):
// ih = clamp(round((oh + 0.5) * (h_in / h_out) - 0.5), 0, h_in-1) in f32.
void dwo_resize_nearest_nhwc(void* out, const void* in, size_t n, size_t h_in, size_t w_in,
                             size_t h_out, size_t w_out, size_t c, size_t esize) {
  const float sh = (float)h_in / (float)h_out, sw = (float)w_in / (float)w_out;
  for (size_t b = 0; b < n; ++b)
    for (size_t oh = 0; oh < h_out; ++oh)
      for (size_t ow = 0; ow < w_out; ++ow) {
        float fh = roundf(((float)oh + 0.5f) * sh - 0.5f);
        fh = fminf(fmaxf(fh, 0.0f), (float)(h_in - 1));
        float fw = roundf(((float)ow + 0.5f) * sw - 0.5f);
        fw = fminf(fmaxf(fw, 0.0f), (float)(w_in - 1));
        const size_t ih = (size_t)fh, iw = (size_t)fw;
        memcpy((uint8_t*)out + ((b * h_out + oh) * w_out + ow) * c * esize,
               (const uint8_t*)in + ((b * h_in + ih) * w_in + iw) * c * esize, c * esize);
      }
}
// concat_fp16 / concat_f32 axis 3 (ops.rs:2248-2299): per pixel, inputs'
// channel rows back to back.
void dwo_concat_channels(void* out, const void* const* ins, const size_t* chans, size_t num,
                         size_t pixels, size_t esize) {
  size_t total = 0;
  for (size_t i = 0; i < num; ++i) total += chans[i];
  for (size_t p = 0; p < pixels; ++p) {
    size_t off = 0;
    for (size_t i = 0; i < num; ++i) {
      memcpy((uint8_t*)out + (p * total + off) * esize, (const uint8_t*)ins[i] + p * chans[i] * esize,
             chans[i] * esize);
      off += chans[i];
    }
  }
}
// split_f32 axis 3 (ops.rs:2407-2456).
void dwo_split_channels(void* const* outs, const void* in, const size_t* chans, size_t num,
                        size_t pixels, size_t esize) {
  size_t total = 0;
  for (size_t i = 0; i < num; ++i) total += chans[i];
  for (size_t p = 0; p < pixels; ++p) {
    size_t off = 0;
    for (size_t i = 0; i < num; ++i) {
      memcpy((uint8_t*)outs[i] + p * chans[i] * esize, (const uint8_t*)in + (p * total + off) * esize,
             chans[i] * esize);
      off += chans[i];
    }
  }
}

// ---------------------------------------------------------------------------
// Part A.8 — BatchNorm fold (crates/dragonwing-onnx/src/graph.rs:597-613),
// OIHW weights: w' = (f32)(w * g/sqrt(var+eps)) and
// b' = (f32)((b - mean) * g/sqrt(var+eps) + beta), all in f64.
// ---------------------------------------------------------------------------
void dwo_fold_batchnorm(float* w, float* bias_out, const float* bias_in, const float* gamma,
                        const float* beta, const float* mean, const float* var, float eps,
                        size_t c_out, size_t per_channel) {
  for (size_t c = 0; c < c_out; ++c) {
    const double std_inv = 1.0 / sqrt((double)var[c] + (double)eps);
    const double sf = (double)gamma[c] * std_inv;
    for (size_t k = 0; k < per_channel; ++k) w[c * per_channel + k] = (float)((double)w[c * per_channel + k] * sf);
    const double ob = bias_in ? (double)bias_in[c] : 0.0;
    bias_out[c] = (float)((ob - (double)mean[c]) * sf + (double)beta[c]);
  }
}

// ---------------------------------------------------------------------------
// Part A.7 — classifier-head ops
// ---------------------------------------------------------------------------

// gemm_f32_naive (ops.rs:273-290; gemm_f32_mt :1659-1707 runs the same
// per-output chain by rows): C[m][n] = A[m][k] B[k][n], acc = fma(a, b, acc)
// over p in order from +0.
void dwo_gemm_f32(float* c, const float* a, const float* b, size_t m, size_t n, size_t k) {
  for (size_t i = 0; i < m; ++i)
    for (size_t j = 0; j < n; ++j) {
      float acc = 0.0f;
      for (size_t p = 0; p < k; ++p) acc = fmaf(a[i * k + p], b[p * n + j], acc);
      c[i * n + j] = acc;
    }
}

// gemm_fp16 (ops.rs:461-479; gemm_fp16_mt :1709-1749): operands widened
// with F16::to_f32, the same f32 chain, F16::from_f32 of the sum.
void dwo_gemm_fp16(uint16_t* c, const uint16_t* a, const uint16_t* b, size_t m, size_t n, size_t k) {
  for (size_t i = 0; i < m; ++i)
    for (size_t j = 0; j < n; ++j) {
      float acc = 0.0f;
      for (size_t p = 0; p < k; ++p) acc = fmaf(dwo_f16_to_f32(a[i * k + p]), dwo_f16_to_f32(b[p * n + j]), acc);
      c[i * n + j] = dwo_f16_from_f32(acc);
    }
}

// gemm_i8_scalar (ops.rs:2981-2995): int32 sum of i8 products (wrapping, as
// the release build's i32 addition).
void dwo_gemm_i8(int32_t* c, const int8_t* a, const int8_t* b, size_t m, size_t n, size_t k) {
  for (size_t i = 0; i < m; ++i)
    for (size_t j = 0; j < n; ++j) {
      uint32_t acc = 0;
      for (size_t p = 0; p < k; ++p) acc += (uint32_t)((int32_t)a[i * k + p] * (int32_t)b[p * n + j]);
      c[i * n + j] = (int32_t)acc;
    }
}

// CpuGraphRuntime::dispatch_gemm's transposed path (onnx runtime.rs:
// 1220-1233, f16 :1256-1266) with trans_b: B is [n][k]; sum += a * b with
// the product rounded before the add (no fma); f16 widens with F16::to_f32
// and stores F16::from_f32 of the sum.
void dwo_gemm_f32_tb(float* c, const float* a, const float* b, size_t m, size_t n, size_t k) {
  for (size_t i = 0; i < m; ++i)
    for (size_t j = 0; j < n; ++j) {
      float sum = 0.0f;
      for (size_t p = 0; p < k; ++p) {
        volatile float prod = a[i * k + p] * b[j * k + p];
        sum += prod;
      }
      c[i * n + j] = sum;
    }
}

void dwo_gemm_fp16_tb(uint16_t* c, const uint16_t* a, const uint16_t* b, size_t m, size_t n, size_t k) {
  for (size_t i = 0; i < m; ++i)
    for (size_t j = 0; j < n; ++j) {
      float sum = 0.0f;
      for (size_t p = 0; p < k; ++p) {
        volatile float prod = dwo_f16_to_f32(a[i * k + p]) * dwo_f16_to_f32(b[j * k + p]);
        sum += prod;
      }
      c[i * n + j] = dwo_f16_from_f32(sum);
    }
}

// CpuGraphRuntime::dispatch_global_avg_pool (onnx runtime.rs:1109-1175),
// NHWC: per (batch, channel) an f32 sum over rows then columns, divided by
// h * w as f32; f16 widens with F16::to_f32 and stores F16::from_f32.
void dwo_global_avg_pool_f32(float* y, const float* x, size_t n, size_t h, size_t w, size_t c) {
  for (size_t b = 0; b < n; ++b)
    for (size_t ch = 0; ch < c; ++ch) {
      float sum = 0.0f;
      for (size_t r = 0; r < h; ++r)
        for (size_t col = 0; col < w; ++col) sum += x[((b * h + r) * w + col) * c + ch];
      y[b * c + ch] = sum / (float)(h * w);
    }
}

void dwo_global_avg_pool_fp16(uint16_t* y, const uint16_t* x, size_t n, size_t h, size_t w, size_t c) {
  for (size_t b = 0; b < n; ++b)
    for (size_t ch = 0; ch < c; ++ch) {
      float sum = 0.0f;
      for (size_t r = 0; r < h; ++r)
        for (size_t col = 0; col < w; ++col) sum += dwo_f16_to_f32(x[((b * h + r) * w + col) * c + ch]);
      y[b * c + ch] = dwo_f16_from_f32(sum / (float)(h * w));
    }
}

// softmax_f32 (ops.rs:1609-1638) over rows of n: max by f32::max from -inf
// (a NaN operand loses), e = exp(x - max), sum in order, out = e * (1 / sum).
void dwo_softmax_f32(float* y, const float* x, size_t rows, size_t n) {
  for (size_t r = 0; r < rows; ++r) {
    const float* xi = x + r * n;
    float* yo = y + r * n;
    float mx = -INFINITY;
    for (size_t i = 0; i < n; ++i) mx = fmaxf(mx, xi[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
      const float e = expf(xi[i] - mx);
      yo[i] = e;
      sum += e;
    }
    const float inv = 1.0f / sum;
    for (size_t i = 0; i < n; ++i) yo[i] *= inv;
  }
}

// ===========================================================================
// Part B — ONNX quantized extensions (no counterpart in the reference)
// ===========================================================================

// QLinearConv (ONNX), u8 activations with zero points, s8 per-channel
// weights (zero point 0), int32 bias:
//   acc = bias[c] + sum over ALL taps of (x - x_zp) * w, where taps outside
//         the image read x_zp (so contribute 0);
//   y   = clamp(rint((float)acc * M[c]) + y_zp, 0, 255), rint = half even,
//   M[c] = (x_scale * w_scale[c]) / y_scale computed in f32.
// Rows r0..r1 of n*h_out.
static void qconv_rows(uint8_t* out, const uint8_t* in, const int8_t* ker, const int32_t* bias,
                       const float* M, int x_zp, int y_zp, size_t h_in, size_t w_in, size_t c_in,
                       size_t c_out, size_t k_h, size_t k_w, size_t sh, size_t sw, size_t ph, size_t pw,
                       size_t ho, size_t wo, size_t r0, size_t r1) {
  for (size_t row = r0; row < r1; ++row) {
    const size_t b = row / ho, oh = row % ho;
    for (size_t ow = 0; ow < wo; ++ow)
      for (size_t oc = 0; oc < c_out; ++oc) {
        int64_t acc = bias ? bias[oc] : 0;
        for (size_t kh = 0; kh < k_h; ++kh)
          for (size_t kw = 0; kw < k_w; ++kw) {
            const long ih = (long)(oh * sh + kh) - (long)ph;
            const long iw = (long)(ow * sw + kw) - (long)pw;
            const bool in_img = !(ih < 0 || ih >= (long)h_in || iw < 0 || iw >= (long)w_in);
            const int8_t* wp = ker + ((kh * k_w + kw) * c_in) * c_out + oc;
            for (size_t ic = 0; ic < c_in; ++ic) {
              const int xv = in_img ? in[((b * h_in + (size_t)ih) * w_in + (size_t)iw) * c_in + ic] : x_zp;
              acc += (int64_t)(xv - x_zp) * (int64_t)wp[ic * c_out];
            }
          }
        const int32_t a32 = (int32_t)acc;
        float q = nearbyintf((float)a32 * M[oc]) + (float)y_zp;
        q = q < 0.0f ? 0.0f : (q > 255.0f ? 255.0f : q);
        out[((b * ho + oh) * wo + ow) * c_out + oc] = (uint8_t)q;
      }
  }
}

void dwo_qlinearconv_u8s8(uint8_t* out, const uint8_t* in, const int8_t* ker, const int32_t* bias,
                          size_t n, size_t h_in, size_t w_in, size_t c_in, size_t c_out, size_t k_h,
                          size_t k_w, size_t sh, size_t sw, size_t ph, size_t pw, float x_scale,
                          int x_zp, const float* w_scales, float y_scale, int y_zp, int num_threads) {
  const size_t ho = out_dim(h_in, ph, k_h, sh), wo = out_dim(w_in, pw, k_w, sw);
  std::vector<float> M(c_out);
  for (size_t c = 0; c < c_out; ++c) M[c] = (x_scale * w_scales[c]) / y_scale;
  parallel_for_scoped(num_threads, n * ho, [&](size_t r0, size_t r1) {
    qconv_rows(out, in, ker, bias, M.data(), x_zp, y_zp, h_in, w_in, c_in, c_out, k_h, k_w, sh, sw,
               ph, pw, ho, wo, r0, r1);
  });
}

// QuantizeLinear (ONNX) from f16: y = clamp(rint(x / scale) + zp, 0, 255).
void dwo_quantize_linear_f16_u8(uint8_t* y, const uint16_t* x, size_t n, float scale, int zp) {
  for (size_t i = 0; i < n; ++i) {
    float q = nearbyintf(dwo_f16_to_f32(x[i]) / scale) + (float)zp;
    q = q < 0.0f ? 0.0f : (q > 255.0f ? 255.0f : q);
    y[i] = (uint8_t)q;
  }
}
// DequantizeLinear (ONNX) into f16: y = F16((float)(q - zp) * scale).
void dwo_dequantize_linear_u8_f16(uint16_t* y, const uint8_t* x, size_t n, float scale, int zp) {
  for (size_t i = 0; i < n; ++i) y[i] = dwo_f16_from_f32((float)((int)x[i] - zp) * scale);
}
// QLinearAdd: the reference add_i8 form (ops.rs:3197-3209) with zero points
// and round-half-even: y = clamp(rint((a-za)*(sa/sy) + (b-zb)*(sb/sy)) + zy).
void dwo_qlinear_add_u8(uint8_t* y, const uint8_t* a, const uint8_t* b, size_t n, float sa, int za,
                        float sb, int zb, float sy, int zy) {
  const float ra = sa / sy, rb = sb / sy;
  for (size_t i = 0; i < n; ++i) {
    const float f = (float)((int)a[i] - za) * ra + (float)((int)b[i] - zb) * rb;
    float q = nearbyintf(f) + (float)zy;
    q = q < 0.0f ? 0.0f : (q > 255.0f ? 255.0f : q);
    y[i] = (uint8_t)q;
  }
}
// Quantized SiLU table: lut[q] = clamp(rint(silu((q - zx) * sx) / sy) + zy),
// silu(v) = v * (1 / (1 + expf(-v))) as Sigmoid then Mul in f32.
void dwo_silu_lut_u8(uint8_t* lut, float sx, int zx, float sy, int zy) {
  for (int q = 0; q < 256; ++q) {
    const float v = (float)(q - zx) * sx;
    const float s = 1.0f / (1.0f + expf(-v));
    const float a = v * s;
    float r = nearbyintf(a / sy) + (float)zy;
    r = r < 0.0f ? 0.0f : (r > 255.0f ? 255.0f : r);
    lut[q] = (uint8_t)r;
  }
}
void dwo_lut_u8(uint8_t* y, const uint8_t* x, size_t n, const uint8_t* lut) {
  for (size_t i = 0; i < n; ++i) y[i] = lut[x[i]];
}
// QLinearGlobalAveragePool (the quantized dispatch_global_avg_pool, onnx
// runtime.rs:1109-1175): acc = sum over h*w of (x - x_zp) in int32,
// y = clamp(rint((float)acc * ((x_scale / y_scale) / (h*w))) + y_zp, 0, 255).
void dwo_qlinear_gap_u8(uint8_t* y, const uint8_t* x, size_t n, size_t h, size_t w, size_t c, float x_scale,
                        int x_zp, float y_scale, int y_zp) {
  const float m = (x_scale / y_scale) / (float)(h * w);
  for (size_t b = 0; b < n; ++b)
    for (size_t ch = 0; ch < c; ++ch) {
      int32_t acc = 0;
      for (size_t p = 0; p < h * w; ++p) acc += (int32_t)x[(b * h * w + p) * c + ch] - x_zp;
      float q = nearbyintf((float)acc * m) + (float)y_zp;
      q = q < 0.0f ? 0.0f : (q > 255.0f ? 255.0f : q);
      y[b * c + ch] = (uint8_t)q;
    }
}
// MaxPool with padding (ONNX): padded taps never win.  Element type by
// esize: 4 = f32, 2 = f16 (compared as f32), 1 = u8.
void dwo_maxpool2d_padded_nhwc(void* out, const void* in, size_t n, size_t h_in, size_t w_in, size_t c,
                               size_t kh, size_t kw, size_t sh, size_t sw, size_t pt, size_t pl,
                               size_t pb, size_t pr, size_t esize) {
  const size_t ho = (h_in + pt + pb - kh) / sh + 1, wo = (w_in + pl + pr - kw) / sw + 1;
  for (size_t b = 0; b < n; ++b)
    for (size_t oh = 0; oh < ho; ++oh)
      for (size_t ow = 0; ow < wo; ++ow)
        for (size_t ch = 0; ch < c; ++ch) {
          float best = -INFINITY;
          size_t best_i = (size_t)-1;
          for (size_t y = 0; y < kh; ++y)
            for (size_t x = 0; x < kw; ++x) {
              const long ih = (long)(oh * sh + y) - (long)pt;
              const long iw = (long)(ow * sw + x) - (long)pl;
              if (ih < 0 || ih >= (long)h_in || iw < 0 || iw >= (long)w_in) continue;
              const size_t idx = ((b * h_in + (size_t)ih) * w_in + (size_t)iw) * c + ch;
              float v;
              if (esize == 4) v = ((const float*)in)[idx];
              else if (esize == 2) v = dwo_f16_to_f32(((const uint16_t*)in)[idx]);
              else v = (float)((const uint8_t*)in)[idx];
              if (best_i == (size_t)-1 || v > best) { best = v; best_i = idx; }
            }
          const size_t o = ((b * ho + oh) * wo + ow) * c + ch;
          memcpy((uint8_t*)out + o * esize, (const uint8_t*)in + best_i * esize, esize);
        }
}

// ===========================================================================
// Part C — YOLOv8 detect tail and post-processing
// ===========================================================================

// The detect tail of an exported YOLOv8 graph (ultralytics Detect in
// inference: DFL, dist2bbox, sigmoid, concat), written with the reference's
// f32 ops in the order the exported graph applies them:
//   per anchor (level s, grid cell gy, gx; stride st), x = the level's 4*R + nc
//   channels widened by F16::to_f32 (dtype.rs:226-263);
//   side j in 0..4: p = softmax_f32 over x[j*R .. j*R+R) (ops.rs:1609-1638),
//     d_j = the 1x1 DFL conv with weights 0..R-1: acc = fma(p_k, k, acc) from
//     +0 in k order (conv2d_f32_nhwc, ops.rs:1356-1436);
//   anchor (gx + 0.5, gy + 0.5); x1 = ax - d0, y1 = ay - d1, x2 = ax + d2,
//     y2 = ay + d3 (sub_f32 / add_f32); cx = (x1 + x2) / 2, cy = (y1 + y2) / 2,
//     w = x2 - x1, h = y2 - y1 (div_f32 by 2), each times st (mul_f32);
//   class c: sigmoid_f32 (ops.rs:1866-1870, 1 / (1 + exp(-x))).
// Output [n][4 + nc][A], A = sum of the levels' h * w, level-major then
// row-major anchors (the ONNX export's [1, 84, 8400] layout).
// x[s]: [n][h_s][w_s][4*R + nc] f16 bits.
void dwo_yolo_detect_tail_f16(float* out, const uint16_t* const* x, const int* hs, const int* ws,
                              const float* strides, int levels, int n, int nc, int reg_max) {
  int A = 0;
  for (int s = 0; s < levels; ++s) A += hs[s] * ws[s];
  const int ch = 4 * reg_max + nc;
  std::vector<float> v(reg_max), e(reg_max);
  for (int b = 0; b < n; ++b) {
    int a = 0;
    for (int s = 0; s < levels; ++s)
      for (int gy = 0; gy < hs[s]; ++gy)
        for (int gx = 0; gx < ws[s]; ++gx, ++a) {
          const uint16_t* px = x[s] + (((size_t)b * hs[s] + gy) * ws[s] + gx) * ch;
          float* o = out + (size_t)b * (4 + nc) * A + a;
          float d[4];
          for (int j = 0; j < 4; ++j) {
            for (int k = 0; k < reg_max; ++k) v[k] = dwo_f16_to_f32(px[j * reg_max + k]);
            dwo_softmax_f32(e.data(), v.data(), 1, reg_max);
            float acc = 0.0f;
            for (int k = 0; k < reg_max; ++k) acc = fmaf(e[k], (float)k, acc);
            d[j] = acc;
          }
          const float ax = (float)gx + 0.5f, ay = (float)gy + 0.5f;
          const float x1 = ax - d[0], y1 = ay - d[1], x2 = ax + d[2], y2 = ay + d[3];
          const float cx = (x1 + x2) / 2.0f, cy = (y1 + y2) / 2.0f;
          const float w = x2 - x1, h = y2 - y1;
          o[0] = cx * strides[s];
          o[(size_t)A] = cy * strides[s];
          o[(size_t)2 * A] = w * strides[s];
          o[(size_t)3 * A] = h * strides[s];
          for (int c = 0; c < nc; ++c) {
            const float xv = dwo_f16_to_f32(px[4 * reg_max + c]);
            o[(size_t)(4 + c) * A] = 1.0f / (1.0f + expf(-xv));
          }
        }
  }
}

// Detection (postprocess.rs:11-19): bbox [x1, y1, x2, y2], class id, confidence.
struct DwoDetection {
  float bbox[4];
  uint32_t class_id;
  float confidence;
};

static float det_area(const DwoDetection& d) {  // Detection::area, postprocess.rs:28-32
  const float w = fmaxf(d.bbox[2] - d.bbox[0], 0.0f);
  const float h = fmaxf(d.bbox[3] - d.bbox[1], 0.0f);
  return w * h;
}

// iou (postprocess.rs:36-55).
float dwo_iou(const float* a, const float* b) {
  DwoDetection da{}, db{};
  memcpy(da.bbox, a, 16);
  memcpy(db.bbox, b, 16);
  const float x1 = fmaxf(a[0], b[0]), y1 = fmaxf(a[1], b[1]);
  const float x2 = fminf(a[2], b[2]), y2 = fminf(a[3], b[3]);
  const float iw = fmaxf(x2 - x1, 0.0f), ih = fmaxf(y2 - y1, 0.0f);
  const float inter = iw * ih;
  const float uni = det_area(da) + det_area(db) - inter;
  return uni > 0.0f ? inter / uni : 0.0f;
}

// decode_detections_v8 (postprocess.rs:78-146) on one image's [4 + nc][A]
// output: best class by strict '>' from (0, 0.0); skipped below the
// threshold; corners from the centre and size through the fixed 640 model
// size, clamped to the image.
static void decode_v8(std::vector<DwoDetection>& dets, const float* raw, size_t nc, size_t A,
                      uint32_t img_w, uint32_t img_h, float conf) {
  const float model = 640.0f;
  const float sx = (float)img_w / model, sy = (float)img_h / model;
  for (size_t a = 0; a < A; ++a) {
    const float cx = raw[a], cy = raw[A + a], w = raw[2 * A + a], h = raw[3 * A + a];
    size_t best = 0;
    float best_conf = 0.0f;
    for (size_t c = 0; c < nc; ++c) {
      const float v = raw[(4 + c) * A + a];
      if (v > best_conf) {
        best_conf = v;
        best = c;
      }
    }
    if (best_conf < conf) continue;
    float x1 = (cx - w / 2.0f) * sx, y1 = (cy - h / 2.0f) * sy;
    float x2 = (cx + w / 2.0f) * sx, y2 = (cy + h / 2.0f) * sy;
    x1 = fminf(fmaxf(x1, 0.0f), (float)img_w);
    y1 = fminf(fmaxf(y1, 0.0f), (float)img_h);
    x2 = fminf(fmaxf(x2, 0.0f), (float)img_w);
    y2 = fminf(fmaxf(y2, 0.0f), (float)img_h);
    dets.push_back({{x1, y1, x2, y2}, (uint32_t)best, best_conf});
  }
}

// nms / nms_agnostic (postprocess.rs:214-277): stable sort by confidence,
// descending; greedy suppression (same class unless agnostic) where
// IoU > threshold; suppressed entries removed by swap_remove from the back.
static void nms_v8(std::vector<DwoDetection>& d, float iou_thr, bool agnostic) {
  std::stable_sort(d.begin(), d.end(), [](const DwoDetection& a, const DwoDetection& b) {
    return b.confidence < a.confidence;  // partial_cmp(b, a) == Less
  });
  std::vector<char> keep(d.size(), 1);
  for (size_t i = 0; i < d.size(); ++i) {
    if (!keep[i]) continue;
    for (size_t j = i + 1; j < d.size(); ++j) {
      if (!keep[j]) continue;
      if (!agnostic && d[i].class_id != d[j].class_id) continue;
      if (dwo_iou(d[i].bbox, d[j].bbox) > iou_thr) keep[j] = 0;
    }
  }
  size_t i = d.size();
  while (i > 0) {
    --i;
    if (!keep[i]) {
      d[i] = d.back();
      d.pop_back();
    }
  }
}

// postprocess_yolo (postprocess.rs:279-305) for each of n images of
// raw [n][4 + nc][A]; agnostic selects nms_agnostic.  Writes at most `cap`
// detections per image to out[b * cap ...] and the full count to counts[b].
void dwo_yolo_postprocess(DwoDetection* out, size_t* counts, const float* raw, size_t n, size_t nc,
                          size_t A, uint32_t img_w, uint32_t img_h, float conf, float iou_thr,
                          int agnostic, size_t cap) {
  for (size_t b = 0; b < n; ++b) {
    std::vector<DwoDetection> d;
    decode_v8(d, raw + b * (4 + nc) * A, nc, A, img_w, img_h, conf);
    nms_v8(d, iou_thr, agnostic != 0);
    counts[b] = d.size();
    for (size_t i = 0; i < d.size() && i < cap; ++i) out[b * cap + i] = d[i];
  }
}

}  // extern "C"
