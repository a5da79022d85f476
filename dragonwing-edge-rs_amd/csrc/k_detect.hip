// YOLOv8 detect tail and post-processing on the GPU.
//
// detect_tail_kernel: the exported graph's tail after the three head convs
// (ultralytics Detect in inference): per anchor, DFL (softmax over each
// side's reg_max bins, then the 1x1 expectation with weights 0..reg_max-1),
// dist2bbox (anchor -/+ distances, centre and size) times the level's
// stride, and the sigmoid of every class logit, written as [n][4 + nc][A]
// f32 (the [1, 84, 8400] layout of an export).  Each step is the reference
// f32 op the exported graph applies: softmax_f32 (ops.rs:1609-1638), the
// conv's fma chain (ops.rs:1356-1436), sub/add/div/mul, sigmoid_f32
// (ops.rs:1866-1870).  exp is the device's expf (a few ulps from the host
// libm's), everything else is IEEE single-rounded.
//
// Post-processing (postprocess_yolo, onnx postprocess.rs:279-305), per image:
//   pp_candidates_kernel  decode_detections_v8 (:78-146) for every anchor:
//                         best class, threshold, corners, clamp; a 64-bit
//                         sort key (confidence descending, anchor ascending);
//   pp_nms_kernel         one workgroup per image: bitonic sort of the keys
//                         in LDS (the reference's stable sort by confidence),
//                         a stable partition by class, greedy NMS per class
//                         on LDS-resident boxes, one wave per class
//                         (nms, :214-243; nms_agnostic as one class), and the
//                         kept detections written in sorted order with their
//                         sorted positions.
// The reference then removes the suppressed entries with swap_remove from
// the back, which reorders the survivors; the host applies that order to
// the kept list (a permutation of the survivors, no arithmetic).
#include "dw_common.h"
#include "dw_device.h"

namespace dw {
namespace {

struct TailLevels {
  const void* x[4];
  int h[4], w[4];
  int start[4];
  int pix[4];  // elements per pixel
  float stride[4];
  int levels;
  int A;
};

template <bool H>
__device__ __forceinline__ float tail_ld(const void* p, size_t i) {
  if constexpr (H)
    return h2f(((const uint16_t*)p)[i]);
  else
    return ((const float*)p)[i];
}

template <bool H>
__global__ __launch_bounds__(256) void detect_tail_kernel(TailLevels L, float* out, int nc, int reg_max) {
  const int a = blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (a >= L.A) return;
  int s = 0;
  while (s + 1 < L.levels && a >= L.start[s + 1]) ++s;
  const int local = a - L.start[s];
  const int gy = local / L.w[s];
  const int gx = local - gy * L.w[s];
  const size_t px = (((size_t)b * L.h[s] + gy) * L.w[s] + gx) * (size_t)L.pix[s];
  const void* x = L.x[s];
  float* o = out + (size_t)b * (4 + nc) * L.A + a;
  float d[4];
  for (int j = 0; j < 4; ++j) {
    const size_t base = px + (size_t)j * reg_max;
    float mx = -INFINITY;
    for (int k = 0; k < reg_max; ++k) mx = fmaxf(mx, tail_ld<H>(x, base + k));
    float sum = 0.0f;
    for (int k = 0; k < reg_max; ++k) sum += expf(tail_ld<H>(x, base + k) - mx);
    const float inv = __fdiv_rn(1.0f, sum);
    float acc = 0.0f;
    for (int k = 0; k < reg_max; ++k) {
      const float p = expf(tail_ld<H>(x, base + k) - mx) * inv;
      acc = fmaf(p, (float)k, acc);
    }
    d[j] = acc;
  }
  const float ax = (float)gx + 0.5f, ay = (float)gy + 0.5f;
  const float x1 = ax - d[0], y1 = ay - d[1], x2 = ax + d[2], y2 = ay + d[3];
  const float st = L.stride[s];
  const size_t A = (size_t)L.A;
  o[0] = __fdiv_rn(x1 + x2, 2.0f) * st;
  o[A] = __fdiv_rn(y1 + y2, 2.0f) * st;
  o[2 * A] = (x2 - x1) * st;
  o[3 * A] = (y2 - y1) * st;
  const size_t cbase = px + (size_t)4 * reg_max;
  for (int c = 0; c < nc; ++c) {
    const float v = tail_ld<H>(x, cbase + c);
    o[(size_t)(4 + c) * A] = __fdiv_rn(1.0f, 1.0f + expf(-v));
  }
}

// ---------------------------------------------------------------------------
// post-processing

struct PPArgs {
  const float* raw;  // [n][4 + nc][A]
  int nc, A;
  float sx, sy, img_w, img_h, conf, iou;
  int agnostic;
  int nmax;          // capacity of the per-image arrays below
  int sort_n;        // power of two >= A
  unsigned long long* keys;  // [n][A]
  DwDetection* det;          // [n][A], per anchor
  int* sorted_anchor;        // [n][nmax]
  int* part_pos;             // [n][nmax]
  DwDetection* out_det;      // [n][nmax]
  int* out_pos;              // [n][nmax]
  int* counts;               // [n][4]: candidates, kept, overflow
};

__global__ __launch_bounds__(256) void pp_candidates_kernel(PPArgs p) {
  const int a = blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (a >= p.A) return;
  const size_t A = (size_t)p.A;
  const float* r = p.raw + (size_t)b * (4 + p.nc) * A + a;
  const float cx = r[0], cy = r[A], w = r[2 * A], h = r[3 * A];
  int best = 0;
  float best_conf = 0.0f;
  for (int c = 0; c < p.nc; ++c) {
    const float v = r[(size_t)(4 + c) * A];
    if (v > best_conf) {
      best_conf = v;
      best = c;
    }
  }
  unsigned long long key = ~0ull;
  if (!(best_conf < p.conf)) {
    const float hw = __fdiv_rn(w, 2.0f), hh = __fdiv_rn(h, 2.0f);
    float x1 = (cx - hw) * p.sx, y1 = (cy - hh) * p.sy;
    float x2 = (cx + hw) * p.sx, y2 = (cy + hh) * p.sy;
    x1 = fminf(fmaxf(x1, 0.0f), p.img_w);
    y1 = fminf(fmaxf(y1, 0.0f), p.img_h);
    x2 = fminf(fmaxf(x2, 0.0f), p.img_w);
    y2 = fminf(fmaxf(y2, 0.0f), p.img_h);
    DwDetection d;
    d.bbox[0] = x1;
    d.bbox[1] = y1;
    d.bbox[2] = x2;
    d.bbox[3] = y2;
    d.class_id = (uint32_t)best;
    d.confidence = best_conf;
    p.det[(size_t)b * A + a] = d;
    // confidence >= +0, so its bits order like its value
    key = ((unsigned long long)(0xFFFFFFFFu - __float_as_uint(best_conf)) << 32) | (unsigned)a;
  }
  p.keys[(size_t)b * A + a] = key;
}

// Detection::area and iou (postprocess.rs:28-32, :36-55), each operation
// rounded as written (no contraction).
__device__ __forceinline__ float box_area(float4 d) {
  return fmaxf(d.z - d.x, 0.0f) * fmaxf(d.w - d.y, 0.0f);
}
__device__ __forceinline__ float box_iou(float4 a, float aa, float4 b) {
  const float x1 = fmaxf(a.x, b.x), y1 = fmaxf(a.y, b.y);
  const float x2 = fminf(a.z, b.z), y2 = fminf(a.w, b.w);
  const float inter = fmaxf(x2 - x1, 0.0f) * fmaxf(y2 - y1, 0.0f);
  const float uni = aa + box_area(b) - inter;
  return uni > 0.0f ? __fdiv_rn(inter, uni) : 0.0f;
}

constexpr int kNmsThreads = 1024;
constexpr int kNmsPer = (kPPMaxCandidates + kNmsThreads - 1) / kNmsThreads;

// LDS layout (bytes), phase by phase:
//   [0, 16 nmax)            sort keys (sort_n * 8 <= 16 nmax), then class ids
//                           of the sorted candidates (u16), then the boxes in
//                           class-partitioned order (float4)
//   [16 nmax, 17 nmax)      keep flags (partitioned order)
//   then 1024 ints          per-class counts / scan scratch
//   then 1024 ints          per-class offsets
//   then nmax / 32 words    kept bitmap over sorted positions
//   then 4 ints             candidate count, next class
__host__ __device__ constexpr size_t nms_lds_bytes(int nmax) {
  return (size_t)17 * nmax + 2 * 1024 * 4 + (size_t)((nmax + 31) / 32) * 4 + 16;
}

__global__ __launch_bounds__(kNmsThreads) void pp_nms_kernel(PPArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int nmax = p.nmax;
  unsigned long long* sk = (unsigned long long*)smem;
  uint16_t* scls = (uint16_t*)smem;
  float4* sbox = (float4*)smem;
  volatile uint8_t* keep = smem + (size_t)16 * nmax;
  int* scnt = (int*)(smem + (size_t)17 * nmax);
  int* soff = scnt + 1024;
  uint32_t* kbits = (uint32_t*)(soff + 1024);
  int* sn = (int*)(kbits + (nmax + 31) / 32);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = blockIdx.x;
  const int A = p.A, S = p.sort_n;
  const int ncls = p.agnostic ? 1 : p.nc;

  if (tid == 0) {
    sn[0] = 0;
    sn[1] = 0;
  }
  for (int i = tid; i < S; i += kNmsThreads) sk[i] = i < A ? p.keys[(size_t)b * A + i] : ~0ull;
  __syncthreads();
  // bitonic sort, ascending: confidence descending, then anchor ascending
  for (int k = 2; k <= S; k <<= 1)
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < S; i += kNmsThreads) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const unsigned long long u = sk[i], v = sk[ixj];
          if ((u > v) == ((i & k) == 0)) {
            sk[i] = v;
            sk[ixj] = u;
          }
        }
      }
      __syncthreads();
    }
  for (int i = tid; i < S; i += kNmsThreads)
    if (sk[i] != ~0ull && (i + 1 == S || sk[i + 1] == ~0ull)) sn[0] = i + 1;
  __syncthreads();
  const int n = sn[0];
  int* cnt = p.counts + 4 * b;
  if (n > nmax) {
    if (tid == 0) {
      cnt[0] = n;
      cnt[1] = 0;
      cnt[2] = 1;
    }
    return;
  }
  // sorted candidates: anchors to global, classes kept in registers
  int my_cls[kNmsPer];
#pragma unroll
  for (int t = 0; t < kNmsPer; ++t) {
    const int q = tid + t * kNmsThreads;
    my_cls[t] = -1;
    if (q < n) {
      const int a = (int)(unsigned)(sk[q] & 0xFFFFFFFFull);
      p.sorted_anchor[(size_t)b * nmax + q] = a;
      my_cls[t] = p.agnostic ? 0 : (int)p.det[(size_t)b * A + a].class_id;
    }
  }
  for (int c = tid; c < 1024; c += kNmsThreads) scnt[c] = 0;
  for (int w = tid; w < (nmax + 31) / 32; w += kNmsThreads) kbits[w] = 0;
  __syncthreads();  // keys no longer read
#pragma unroll
  for (int t = 0; t < kNmsPer; ++t) {
    const int q = tid + t * kNmsThreads;
    if (q < n) {
      scls[q] = (uint16_t)my_cls[t];
      atomicAdd(&scnt[my_cls[t]], 1);
    }
  }
  __syncthreads();
  // exclusive scan of the class counts (ncls <= 1024), Hillis-Steele in soff
  int v = tid < ncls ? scnt[tid] : 0;
  soff[tid] = v;
  __syncthreads();
  for (int d = 1; d < 1024; d <<= 1) {
    const int add = tid >= d ? soff[tid - d] : 0;
    __syncthreads();
    soff[tid] += add;
    __syncthreads();
  }
  soff[tid] -= v;  // inclusive -> exclusive
  __syncthreads();
  // stable partition by class: one wave per class, ballots over the sorted order
  for (int c = wave; c < ncls; c += kNmsThreads / 64) {
    int cursor = soff[c];
    for (int q0 = 0; q0 < n; q0 += 64) {
      const int q = q0 + lane;
      const bool m = q < n && (int)scls[q] == c;
      const unsigned long long bal = __ballot(m);
      if (m) {
        const int rank = __popcll(bal & ((1ull << lane) - 1));
        p.part_pos[(size_t)b * nmax + cursor + rank] = q;
      }
      cursor += __popcll(bal);
    }
  }
  __syncthreads();
  // boxes in partitioned order
  for (int q = tid; q < n; q += kNmsThreads) {
    const int sp = p.part_pos[(size_t)b * nmax + q];
    const int a = p.sorted_anchor[(size_t)b * nmax + sp];
    const DwDetection d = p.det[(size_t)b * A + a];
    sbox[q] = make_float4(d.bbox[0], d.bbox[1], d.bbox[2], d.bbox[3]);
    keep[q] = 1;
  }
  __syncthreads();
  // greedy suppression per class, one wave per class (taken in turn)
  for (;;) {
    int c = 0;
    if (lane == 0) c = atomicAdd(&sn[1], 1);
    c = __shfl(c, 0);
    if (c >= ncls) break;
    const int s0 = soff[c], e0 = s0 + scnt[c];
    for (int i = s0; i < e0; ++i) {
      if (!keep[i]) continue;
      const float4 bi = sbox[i];
      const float ai = box_area(bi);
      for (int j = i + 1 + lane; j < e0; j += 64)
        if (keep[j] && box_iou(bi, ai, sbox[j]) > p.iou) keep[j] = 0;
    }
  }
  __syncthreads();
  for (int q = tid; q < n; q += kNmsThreads)
    if (keep[q]) {
      const int sp = p.part_pos[(size_t)b * nmax + q];
      atomicOr(&kbits[sp >> 5], 1u << (sp & 31));
    }
  __syncthreads();
  // kept detections in sorted order: contiguous ranges per thread, block scan
  const int per = (n + kNmsThreads - 1) / kNmsThreads;
  const int q0 = tid * per, q1 = min(n, q0 + per);
  int mine = 0;
  for (int q = q0; q < q1; ++q) mine += (kbits[q >> 5] >> (q & 31)) & 1;
  scnt[tid] = mine;
  __syncthreads();
  for (int d = 1; d < 1024; d <<= 1) {
    const int add = tid >= d ? scnt[tid - d] : 0;
    __syncthreads();
    scnt[tid] += add;
    __syncthreads();
  }
  int k = scnt[tid] - mine;
  for (int q = q0; q < q1; ++q)
    if ((kbits[q >> 5] >> (q & 31)) & 1) {
      const int a = p.sorted_anchor[(size_t)b * nmax + q];
      p.out_det[(size_t)b * nmax + k] = p.det[(size_t)b * A + a];
      p.out_pos[(size_t)b * nmax + k] = q;
      ++k;
    }
  if (tid == kNmsThreads - 1) {
    cnt[0] = n;
    cnt[1] = scnt[tid];
    cnt[2] = 0;
  }
}

}  // namespace

void launch_detect_tail(hipStream_t st, int dtype, const DetectTailArgs& t, float* out, int n) {
  TailLevels L{};
  if (t.levels < 1 || t.levels > 4) fail(-2, "detect tail: 1 to 4 levels");
  int a = 0;
  for (int s = 0; s < t.levels; ++s) {
    L.x[s] = t.x[s];
    L.h[s] = t.h[s];
    L.w[s] = t.w[s];
    L.pix[s] = t.pix[s];
    L.stride[s] = t.stride[s];
    L.start[s] = a;
    a += t.h[s] * t.w[s];
  }
  L.levels = t.levels;
  L.A = a;
  const dim3 g((unsigned)((a + 255) / 256), (unsigned)n);
  if (dtype == F16)
    hipLaunchKernelGGL(detect_tail_kernel<true>, g, dim3(256), 0, st, L, out, t.nc, t.reg_max);
  else if (dtype == F32)
    hipLaunchKernelGGL(detect_tail_kernel<false>, g, dim3(256), 0, st, L, out, t.nc, t.reg_max);
  else
    fail(-2, "detect tail: f16 or f32 inputs");
  DW_HIP(hipGetLastError());
}

size_t pp_nms_lds_bytes(int nmax) { return nms_lds_bytes(nmax); }

void launch_yolo_postprocess(hipStream_t st, const PostprocessArgs& a) {
  PPArgs p{};
  p.raw = a.raw;
  p.nc = a.nc;
  p.A = a.A;
  p.sx = a.sx;
  p.sy = a.sy;
  p.img_w = a.img_w;
  p.img_h = a.img_h;
  p.conf = a.conf;
  p.iou = a.iou;
  p.agnostic = a.agnostic;
  p.nmax = a.nmax;
  int s = 1;
  while (s < a.A) s <<= 1;
  p.sort_n = s;
  if ((size_t)s * 8 > (size_t)16 * a.nmax) fail(-2, "postprocess: too many anchors to sort");
  if (a.nmax > kPPMaxCandidates) fail(-1, "postprocess: capacity");
  p.keys = a.keys;
  p.det = a.det;
  p.sorted_anchor = a.sorted_anchor;
  p.part_pos = a.part_pos;
  p.out_det = a.out_det;
  p.out_pos = a.out_pos;
  p.counts = a.counts;
  hipLaunchKernelGGL(pp_candidates_kernel, dim3((unsigned)((a.A + 255) / 256), (unsigned)a.n), dim3(256), 0, st,
                     p);
  DW_HIP(hipGetLastError());
  hipLaunchKernelGGL(pp_nms_kernel, dim3((unsigned)a.n), dim3(kNmsThreads), nms_lds_bytes(a.nmax), st, p);
  DW_HIP(hipGetLastError());
}

}  // namespace dw
