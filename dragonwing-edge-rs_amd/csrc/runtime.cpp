// HipGraphRuntime: VulkanGraphRuntime's API
// (crates/dragonwing-onnx/src/vulkan_runtime.rs:115-469, :2113-2141) on the
// HIP backend.  At creation the graph is lowered once:
//
//  1. fusion groups — Conv(+bias) with its activation (Relu, Sigmoid*Mul,
//     SiLU) and a following residual Add; QLinearConv with its activation
//     table and QLinearAdd; DequantizeLinear -> fp16 Conv and fp16 Conv ->
//     QuantizeLinear -> table for the fp16 layers of a u8 graph; three
//     cascaded SPPF max pools.  Intermediates inside a group never touch
//     memory.
//  2. placement — a Concat's inputs are written straight into channel
//     slices of the concat buffer, and Split outputs are channel slices of
//     their input, so neither op moves data (a copy is emitted only when a
//     tensor cannot be placed).
//  3. allocation of every remaining root tensor, weight packing for the
//     MFMA kernels, per-channel requant tables.
//  4. a launch list replayed by run(); optionally captured once into a HIP
//     graph (the analogue of OpsRecorder's single command buffer).
//
// Every op runs on the GPU; an op without a kernel is an error at creation.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <exception>
#include <functional>
#include <map>
#include <memory>
#include <set>
#include <sstream>

#include "backend.h"
#include "graph.h"

namespace dw {

struct RtTensor {
  int dtype = 0;
  int64_t n = 1, h = 1, w = 1, c = 1;
  bool rank4 = false;
  bool materialized = true;
  std::string parent;  // storage parent ("" = own storage)
  int c_off = 0;       // channel offset inside parent
  void* base = nullptr;
  int pix_stride = 0;
  int abs_off = 0;
  int rid = -1;                   // storage root (index), set by allocate()
  uintptr_t ra0 = 0, ra1 = 0;     // the root's bytes in the activation arena
  float scale = 1.0f;
  int zp = 0;
  int64_t pixels() const { return n * h * w; }
  View view() const { return {base, pix_stride, abs_off}; }
  size_t bytes() const { return (size_t)(n * h * w * c) * dtype_size(dtype); }
};

// Channels [lo, hi) of every pixel of storage root `rid`, which occupies
// bytes [a0, a1): what a launch reads or writes (every activation is a
// channel slice of a root).  Roots whose lifetimes do not overlap may share
// bytes, so two regions of different roots overlap when their bytes do.
struct Region {
  int rid;
  int lo, hi;
  uintptr_t a0, a1;
  bool overlaps(const Region& o) const {
    return rid == o.rid ? (lo < o.hi && o.lo < hi) : (a0 < o.a1 && o.a0 < a1);
  }
};

struct Launch {
  std::string kernel;
  std::string op;
  double work = 0;   // algorithmic ops (MAC = 2)
  double bytes = 0;  // algorithmic bytes moved
  std::function<void(hipStream_t)> fn;
  // implicit-GEMM launches: their arguments, shared with `fn`, so the tuner
  // can change the tile shape after the launch list is built
  std::shared_ptr<IgemmArgs> ig;
  // direct-conv launches: their arguments, shared with `fn`, so an input
  // can be switched to the NCHW f32 loader after the list is built
  std::shared_ptr<DirectArgs> da;
  std::shared_ptr<StemF16Args> sa;  // the same for the fp16 MFMA stem
  // nearest-resize launches: their arguments and element type, so the pass
  // that folds a 2x upsample into its producer can find them
  std::shared_ptr<ResizeArgs> ra;
  int rdtype = 0;
  // band-tile depthwise launches: their output rows per band, chosen by the tuner
  std::shared_ptr<int> dw_band;  // units * 100 + band rows
  std::shared_ptr<DwArgs> dwa;
  int esize = 0;
  // QLinearConv launches: the group's input and final output tensors (the
  // pass that chains two convs into one launch matches them), and the
  // tuner's time for 4 launches of the chosen tile (ms; 0 when untimed)
  std::string t_in, t_out;
  float tuned_ms = 0;
  // u8 -> f16 1x1 launches (conv1x1_u8_f16): their arguments, so the pass
  // that fuses them into the conv before can take them over
  std::shared_ptr<Conv1x1F16Args> c1a;
  // schedule over several streams: the storage this launch touches, its
  // stream, the launches on other streams it waits for, and whether a
  // later launch on another stream waits for it
  int group = -1;
  std::vector<Region> reads, writes;
  int stream = 0;
  std::vector<int> waits;
  bool record = false;
};

struct Group {
  std::string kind;  // conv, qconv, pool3, pool, resize, concat, split, ew, noop
  std::vector<int> ops;
  // conv / qconv fusion details
  int act = ACT_NONE;
  std::string in, out, res;  // input, final output, residual tensors
  int in_kind = 0;           // direct conv input: 0 f32, 1 f16, 2 u8 dequant
  float in_scale = 1; int in_zp = 0;
  int out_kind = 0;          // direct conv output: 0 f32, 1 f16, 2 u8 quant
  std::string pre;           // QLinearConv output (pre-table) tensor
  bool lut = false;
  std::string lut_out;       // tensor after the table (QLinearLUT output)
  int conv = -1;             // index of the conv op
  // reference-form INT8 conv (s8 x s8): requantized to s8 with one scale
  // (Requantize / Conv2dRequantReluI8Nhwc) or the raw int32 accumulator
  bool requant = false;
  float requant_scale = 1.0f;
};

struct Runtime {
  Backend* be = nullptr;
  GraphIR g;
  std::map<std::string, RtTensor> ts;
  std::vector<void*> allocs;
  size_t act_bytes = 0;           // the activation arena
  size_t act_bytes_unshared = 0;  // what the roots would take without reuse
  std::vector<Launch> launches;
  // the sibling fusions in the order made: the fused launch's position, the
  // two launches it replaced and the second one's former position (undone
  // last first, they restore the list)
  struct SibUndo {
    size_t pos, jpos;
    Launch a, b;
  };
  std::vector<SibUndo> sib_undo;
  std::vector<std::string> info;
  bool capture = false;
  hipGraph_t hgraph = nullptr;
  hipGraphExec_t hexec = nullptr;
  // independent launches (no shared storage along any path of the launch
  // list) go to different streams, forked from and joined back into the
  // backend's stream; a captured graph keeps them as parallel branches
  int nstreams = 1;
  std::vector<hipStream_t> side;  // streams 1 .. nstreams - 1
  std::vector<hipEvent_t> evs;    // per launch (recorded ones only), then fork
  bool stats = false;
  // DW_RT_EXACT_U8_F16_CONV: convs that read u8 (dequantized to f16) and
  // write f16 run in the reference's accumulation order (bit-identical to
  // the CPU) instead of on the fp16 matrix cores
  bool exact_u8_f16 = false;
  // DW_RT_EXACT_F16_DEPTHWISE: fp16 depthwise convs in the reference's
  // accumulation order instead of the packed-f16 band kernel
  bool exact_f16_dw = false;
  // graph inputs given in NCHW f32 (the layout before convert_nchw_to_nhwc):
  // the one stem conv that reads such an input loads the NCHW planes itself
  // (rounding to f16 in its loader); any other input is converted by a
  // transpose launch at the head of every run
  struct NchwIn {
    int launch = -2;        // the stem launch reading the input, -1 none, -2 not looked up
    DirectArgs orig{};      // its arguments for the NHWC input
    StemF16Args orig_s{};   // the same when it is the fp16 MFMA stem
    void* stage = nullptr;  // owned device copy of host NCHW data
    size_t stage_bytes = 0;
    const void* src = nullptr;  // NCHW data the runs read (stage or a bound buffer)
    bool active = false;
  };
  std::map<std::string, NchwIn> nchw;
  void set_input_nchw(const std::string& name, const void* src);
  void reset_input_layout(const std::string& name);
  void drop_capture();
  float* stats_dev = nullptr;
  std::vector<std::string> stats_names;

  ~Runtime() {
    if (be) (void)hipSetDevice(be->device);
    if (be && be->stream) (void)hipStreamSynchronize(be->stream);
    if (hexec) (void)hipGraphExecDestroy(hexec);
    if (hgraph) (void)hipGraphDestroy(hgraph);
    for (hipStream_t s : side) {
      (void)hipStreamSynchronize(s);
      (void)hipStreamDestroy(s);
    }
    for (hipEvent_t e : evs)
      if (e) (void)hipEventDestroy(e);
    for (void* p : allocs) (void)hipFree(p);
    for (auto& kv : nchw)
      if (kv.second.stage) (void)hipFree(kv.second.stage);
  }

  void* dalloc(size_t bytes) {
    void* p = nullptr;
    DW_HIP(hipMalloc(&p, std::max<size_t>(bytes, 256)));
    allocs.push_back(p);
    return p;
  }
  void* upload(const void* src, size_t bytes) {
    void* p = dalloc(bytes);
    DW_HIP(hipMemcpy(p, src, bytes, hipMemcpyHostToDevice));
    return p;
  }

  RtTensor& T(const std::string& n) {
    auto it = ts.find(n);
    if (it == ts.end()) fail(DW_ERR_RUNTIME, "runtime: unknown tensor '" + n + "'");
    return it->second;
  }

  void build(Backend* b, const GraphIR& graph, bool stats_mode);
  void lower(std::vector<Group>& groups);
  void place(const std::vector<Group>& groups);
  void allocate(const std::vector<Group>& groups);
  void emit(const Group& gr);
  void emit_conv(const Group& gr);
  void emit_qconv(const Group& gr);
  void emit_ew(const OpNode& op);
  void emit_iconv(const Group& gr);
  void emit_shape(const Group& gr);
  // a tensor as a rank-4 index space (its dims padded with leading 1s) with
  // the element strides and offset of its storage
  struct Addr4 {
    void* base = nullptr;
    long long d[4] = {1, 1, 1, 1};
    long long st[4] = {0, 0, 0, 1};
    long long off = 0;
    int es = 1;
    int rank = 0;
  };
  Addr4 addr4(const std::string& name);
  void normalize();
  void push_igemm(Launch& L, const IgemmArgs& a, int esize);
  void autotune();
  void fuse_pairs();
  void fuse_heads();
  void tag_group(const Group& gr, size_t first, int gid);
  void plan_streams(int n);
  float time_graph();
  void fuse_c2f();
  void fuse_resize();
  void fuse_siblings();
  void enqueue(hipStream_t st);
  void run();
};

// F16::to_f32_soft (dtype.rs:226-263), used by get_output_f32 as the
// reference's runtime does.
float f16_to_f32_ref(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  uint32_t out;
  if (e == 0) {
    if (m == 0) {
      out = sign;
    } else {
      uint32_t mm = m;
      int sh = 0;
      while ((mm & 0x400u) == 0) { mm <<= 1; ++sh; }
      out = sign | ((uint32_t)(127 - 15 - sh) << 23) | ((mm & 0x3FFu) << 13);
    }
  } else if (e == 31) {
    out = m == 0 ? (sign | 0x7F800000u) : (sign | 0x7FC00000u | (m << 13));
  } else {
    out = sign | ((e + 112) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &out, 4);
  return f;
}

namespace {

// Whether rint(x / s), for every finite f16 value x widened with the
// reference decode, equals rint of the reciprocal quotient with one FMA
// correction: q0 = x * (1/s); q = fma(fma(-q0, s, x), 1/s, q0).  Checked
// exhaustively (65,536 inputs), so the kernels may use it bit-exactly.
bool fast_quant_ok(float s, float rcp) {
  for (uint32_t h = 0; h < 65536; ++h) {
    const float x = f16_to_f32_ref((uint16_t)h);
    if (!(fabsf(x) <= 65504.0f)) continue;  // non-finite: the kernels divide
    const float q0 = x * rcp;
    const float q = fmaf(fmaf(-q0, s, x), rcp, q0);
    if (rintf(q) != rintf(x / s)) return false;
  }
  return true;
}

// Whether rint(x * (1/s)) equals rint(x / s) for every finite f16 value x
// (IEEE decode) whose quotient is not clamped either way (|x / s| < 512;
// x * (1/s) is within two ulps of x / s), so the fast epilogue may leave out
// the FMA correction.
bool plain_quant_ok(float s, float rcp) {
  for (uint32_t h = 0; h < 65536; ++h) {
    if ((h & 0x7C00u) == 0x7C00u) continue;  // inf, NaN
    uint16_t hb = (uint16_t)h;
    _Float16 hv;
    memcpy(&hv, &hb, 2);
    const float x = (float)hv;
    if (fabsf(x / s) >= 512.0f) continue;  // clamped to 0 or 255 either way
    if (rintf(x * rcp) != rintf(x / s)) return false;
  }
  return true;
}

// Whether an f16 bias holds no subnormal value (then the bias pass on f16
// values is the IEEE f16 sum).
bool bias_plain_f16(const GraphIR& g, const OpNode& op, bool has_bias) {
  if (!has_bias) return true;
  const TensorInfo& B = g.t.at(op.in[2]);
  if (B.dtype != DW_DTYPE_F16) return false;
  const uint16_t* bh = (const uint16_t*)B.data.data();
  for (size_t c = 0; c < B.data.size() / 2; ++c) {
    const uint16_t m = bh[c] & 0x7fff;
    if (m != 0 && m < 0x400) return false;
  }
  return true;
}

// Whether the exact-conv epilogue may widen its f16 values as IEEE f16
// instead of the reference decode (which halves subnormals) and use the
// reciprocal quotient: true when no f16 subnormal can change an output.
//  * bias pass F16(f32(y) + b): checked for every subnormal y and every
//    channel's bias;
//  * QuantizeLinear: a subnormal |y| < 2^-14 gives |y / s| < 0.5 either way
//    when s >= 2^-13, so it quantizes to the zero point both ways; and the
//    reciprocal quotient must be exact (out_fast).
bool fast_epi_ok(const GraphIR& g, const OpNode& op, bool has_bias, int out_kind, const DirectArgs& a) {
  if (out_kind == 2 && (!a.out_fast || !(a.out_scale >= 1.220703125e-04f))) return false;
  if (!has_bias) return true;
  const TensorInfo& B = g.t.at(op.in[2]);
  if (B.dtype != DW_DTYPE_F16) return false;
  const uint16_t* bh = (const uint16_t*)B.data.data();
  for (size_t c = 0; c < B.data.size() / 2; ++c) {
    const float b = f16_to_f32_ref(bh[c]);
    for (uint32_t m = 1; m < 0x400; ++m)
      for (uint32_t sign : {0u, 0x8000u}) {
        const float ieee = ldexpf((float)m, -24) * (sign ? -1.0f : 1.0f);
        const float ref = f16_to_f32_ref((uint16_t)(sign | m));
        if (f16_bits_from_f32(ref + b) != f16_bits_from_f32(ieee + b)) return false;
      }
  }
  return true;
}

}  // namespace

void Runtime::build(Backend* b, const GraphIR& graph, bool stats_mode) {
  be = b;
  g = graph;
  stats = stats_mode;
  for (auto& kv : g.t) {
    RtTensor r;
    const TensorInfo& ti = kv.second;
    r.dtype = ti.dtype;
    if (ti.dims.size() == 4) {
      r.rank4 = true;
      r.n = ti.dims[0]; r.h = ti.dims[1]; r.w = ti.dims[2]; r.c = ti.dims[3];
    } else if (!ti.is_init && !ti.dims.empty()) {
      // other ranks (Gemm, Flatten, Reshape, Softmax operands): rows of the
      // last dimension, as rows pixels of cols channels
      r.rank4 = true;
      r.c = ti.dims.back();
      r.n = ti.numel() / std::max<int64_t>(1, r.c); r.h = 1; r.w = 1;
    } else {
      r.c = ti.numel();
    }
    r.scale = ti.scale;
    r.zp = ti.zp;
    ts[kv.first] = r;
  }
  for (auto& op : g.ops) {
    if (op.type == "BatchNormalization")
      fail(DW_ERR_UNSUPPORTED, "BatchNormalization must be folded (dw_graph_fold_batchnorm) first");
    for (auto& o : op.out)
      if (!T(o).rank4) fail(DW_ERR_UNSUPPORTED, "runtime: activations must be 4-D NHWC (" + o + ")");
  }
  normalize();
  std::vector<Group> groups;
  lower(groups);
  place(groups);
  allocate(groups);
  if (stats) {
    for (auto& kv : ts)
      if (kv.second.rank4 && !g.t[kv.first].is_init && kv.second.dtype == F32) stats_names.push_back(kv.first);
    stats_dev = (float*)dalloc(stats_names.size() * 2 * sizeof(float));
  }
  for (size_t gi = 0; gi < groups.size(); ++gi) {
    const Group& gr = groups[gi];
    const size_t first = launches.size();
    emit(gr);
    tag_group(gr, first, (int)gi);
    if (!stats) continue;
    // calibration: min/max of every f32 activation an op writes
    for (int oi : gr.ops)
      for (auto& on : g.ops[oi].out) {
        auto it = std::find(stats_names.begin(), stats_names.end(), on);
        if (it == stats_names.end()) continue;
        RtTensor& y = T(on);
        float* dst = stats_dev + 2 * (it - stats_names.begin());
        const View v = y.view();
        const int px = (int)y.pixels(), ch = (int)y.c;
        Launch S;
        S.kernel = "minmax";
        S.op = on;
        S.fn = [=](hipStream_t st) { launch_minmax(st, v, px, ch, dst); };
        launches.push_back(S);
      }
  }
  if (!stats) {
    autotune();
    fuse_c2f();
    fuse_pairs();
    fuse_heads();
    fuse_resize();
    fuse_siblings();
  }
  // streams: the schedule over 4 streams, or one stream, whichever runs the
  // whole graph faster (the cross-stream waits cost more than the overlap
  // gains when the layers already fill the GPU); DW_GRAPH_STREAMS=<n> fixes
  // the count
  int ns = 4;
  const char* senv = getenv("DW_GRAPH_STREAMS");
  if (senv) ns = atoi(senv);
  ns = stats ? 1 : std::max(1, std::min(ns, 8));
  plan_streams(ns);
  const char* tune_env = getenv("DW_AUTOTUNE");
  const bool tuned = !((tune_env && tune_env[0] == '0') || getenv("DW_IGEMM_TILE"));
  if (!senv && !stats && tuned && nstreams > 1) {
    const float t_multi = time_graph();
    plan_streams(1);
    const float t_one = time_graph();
    if (t_multi < t_one) plan_streams(ns);
    if (const char* lp = getenv("DW_AUTOTUNE_LOG"))
      if (FILE* log = fopen(lp, "a")) {
        fprintf(log, "graph\t%d streams\t%.2f\ngraph\t1 stream\t%.2f\n", ns, t_multi * 1e3f, t_one * 1e3f);
        fclose(log);
      }
  }
  // sibling GEMMs were kept by timing each alone; on several streams the two
  // convs they replace may already run concurrently, so the whole graph is
  // timed with them and without them (on the chosen stream count), and the
  // faster list kept
  if (!sib_undo.empty() && !stats && tuned) {
    const int nsel = nstreams;
    const float t_sib = time_graph();
    std::vector<Launch> fused = launches;
    for (auto it = sib_undo.rbegin(); it != sib_undo.rend(); ++it) {
      launches[it->pos] = it->a;
      launches.insert(launches.begin() + (long)it->jpos, it->b);
    }
    plan_streams(nsel);
    const float t_apart = time_graph();
    if (t_sib <= t_apart) {
      launches = fused;
      plan_streams(nsel);
    }
    if (const char* lp = getenv("DW_AUTOTUNE_LOG"))
      if (FILE* log = fopen(lp, "a")) {
        fprintf(log, "graph\tsibling GEMMs\t%.2f\ngraph\tsiblings apart\t%.2f\n", t_sib * 1e3f, t_apart * 1e3f);
        fclose(log);
      }
  }
}

// Milliseconds of one graph run on the current stream schedule (the best of
// 3 timings of 4 runs back to back; the activations hold whatever the last
// run left, which the timing does not depend on).
float Runtime::time_graph() {
  hipStream_t st = be->stream;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  DW_HIP(hipEventCreate(&e0));
  DW_HIP(hipEventCreate(&e1));
  enqueue(st);
  float best = 1e30f;
  for (int r = 0; r < 3; ++r) {
    DW_HIP(hipEventRecord(e0, st));
    for (int k = 0; k < 4; ++k) enqueue(st);
    DW_HIP(hipEventRecord(e1, st));
    DW_HIP(hipEventSynchronize(e1));
    float ms = 0;
    DW_HIP(hipEventElapsedTime(&ms, e0, e1));
    best = std::min(best, ms / 4);
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return best;
}

namespace {
// Concat / Split along channels: whether the operand shapes are those of a
// channel concatenation (every input agrees with the output on N, H, W and
// the channel counts add up).  convert_nchw_to_nhwc leaves these ops'
// axis attribute in NCHW numbering (graph.rs:248-290: axis 1 for channels),
// so a graph that went through the reference's passes carries axis 1 on
// NHWC data; the shapes decide.
bool channel_join(const std::vector<const RtTensor*>& parts, const RtTensor& whole) {
  int64_t c = 0;
  for (const RtTensor* t : parts) {
    if (t->n != whole.n || t->h != whole.h || t->w != whole.w) return false;
    c += t->c;
  }
  return c == whole.c;
}
}  // namespace

// Graph forms normalised before lowering:
//  * the reference's INT8 form names a conv's int32 accumulator "<t>_i32"
//    without any op writing it: Conv writes t, then Requantize reads
//    "<t>_i32" and writes t again (QuantizedGraphCompiler::create_requant_op,
//    quantize.rs:205-223).  The Conv is given the accumulator as its output,
//    so every tensor has one writer;
//  * Concat / Split with an NCHW-numbered channel axis (1) on NHWC tensors
//    are renumbered to axis 3 when the shapes are a channel join.
void Runtime::normalize() {
  for (size_t i = 0; i < g.ops.size(); ++i) {
    OpNode& rq = g.ops[i];
    if (rq.type != "Requantize" || rq.in.empty() || rq.out.empty()) continue;
    bool written = false;
    for (size_t k = 0; k < i; ++k)
      for (auto& o : g.ops[k].out) written |= o == rq.in[0];
    if (written) continue;
    for (int k = (int)i - 1; k >= 0; --k) {
      OpNode& cv = g.ops[k];
      if (cv.type == "Conv" && !cv.out.empty() && cv.out[0] == rq.out[0]) {
        if (T(rq.in[0]).dtype != I32) fail(DW_ERR_RUNTIME, "Requantize input " + rq.in[0] + " must be int32");
        cv.out[0] = rq.in[0];
        break;
      }
    }
  }
  for (auto& op : g.ops) {
    if (op.type != "Concat" && op.type != "Split") continue;
    if (op.in.empty() || op.out.empty()) continue;
    const bool cat = op.type == "Concat";
    const std::string& whole = cat ? op.out[0] : op.in[0];
    const int rank = (int)g.t[whole].dims.size();
    if (op.p.axis < 0) op.p.axis += rank;
    if (rank == 4 && op.p.axis == 3) continue;
    std::vector<const RtTensor*> parts;
    for (auto& n : cat ? op.in : op.out) parts.push_back(&T(n));
    // axis 3 below means the channel (last) axis of the rows x channels
    // view; other axes are joined by copies
    const bool last = rank != 4 && op.p.axis == rank - 1;
    if ((last || (rank == 4 && op.p.axis == 1)) && channel_join(parts, T(whole))) op.p.axis = 3;
    else if (rank != 4) op.p.axis += 4 - rank;  // as an axis of the rank-4 index space
  }
}

// The storage a group's launches touch: every materialized activation its
// ops read or write, as channel ranges of their roots (a superset of what
// each launch touches, which only adds dependencies).
void Runtime::tag_group(const Group& gr, size_t first, int gid) {
  std::vector<Region> rd, wr;
  auto add = [&](std::vector<Region>& v, const std::string& name) {
    auto it = ts.find(name);
    if (it == ts.end() || g.t[name].is_init) return;
    const RtTensor& r = it->second;
    if (!r.rank4 || !r.base) return;
    v.push_back({r.rid, r.abs_off, r.abs_off + (int)r.c, r.ra0, r.ra1});
  };
  for (int oi : gr.ops) {
    for (auto& n : g.ops[oi].in) add(rd, n);
    for (auto& n : g.ops[oi].out) add(wr, n);
  }
  for (size_t k = first; k < launches.size(); ++k) {
    launches[k].group = gid;
    launches[k].reads = rd;
    launches[k].writes = wr;
  }
}

// Stream schedule.  Launch j depends on an earlier launch i when one writes
// storage the other reads or writes, or when both belong to the same group
// (launches of one group run in list order).  j continues the stream whose
// last launch is its latest dependency; otherwise (no dependency at a
// stream's tail) it takes the stream whose last launch is oldest.  It then
// waits for the latest dependency on every other stream.
void Runtime::plan_streams(int n) {
  // a previous schedule's events (nothing in flight uses them once the
  // streams are idle)
  if (!evs.empty()) {
    DW_HIP(hipStreamSynchronize(be->stream));
    for (hipStream_t s : side) DW_HIP(hipStreamSynchronize(s));
    for (hipEvent_t e : evs)
      if (e) (void)hipEventDestroy(e);
    evs.clear();
  }
  nstreams = n;
  for (auto& L : launches) {
    L.stream = 0;
    L.waits.clear();
    L.record = false;
  }
  if (n <= 1) return;
  auto depends = [](const Launch& a, const Launch& b) {
    if (a.group == b.group) return true;
    for (const Region& w : a.writes) {
      for (const Region& r : b.reads) if (w.overlaps(r)) return true;
      for (const Region& r : b.writes) if (w.overlaps(r)) return true;
    }
    for (const Region& r : a.reads)
      for (const Region& w : b.writes) if (r.overlaps(w)) return true;
    return false;
  };
  std::vector<int> last(n, -1);
  for (int j = 0; j < (int)launches.size(); ++j) {
    Launch& J = launches[j];
    std::vector<int> dep(n, -1);
    for (int i = 0; i < j; ++i)
      if (depends(launches[i], J)) dep[launches[i].stream] = i;
    int s = -1;
    for (int k = 0; k < n; ++k)
      if (dep[k] >= 0 && dep[k] == last[k] && (s < 0 || dep[k] > dep[s])) s = k;
    if (s < 0) {
      s = 0;
      for (int k = 1; k < n; ++k)
        if (last[k] < last[s]) s = k;
    }
    for (int k = 0; k < n; ++k)
      if (k != s && dep[k] >= 0) {
        J.waits.push_back(dep[k]);
        launches[dep[k]].record = true;
      }
    J.stream = s;
    last[s] = j;
  }
  // one stream after all (a chain, or a single launch): no fork or join
  bool side_used = false;
  for (int k = 1; k < n; ++k) side_used |= last[k] >= 0;
  if (!side_used) {
    nstreams = 1;
    for (auto& L : launches) {
      L.waits.clear();
      L.record = false;
    }
    return;
  }
  // the backend's stream joins every other stream's last launch
  for (int k = 1; k < n; ++k)
    if (last[k] >= 0) launches[last[k]].record = true;
  while ((int)side.size() < n - 1) {
    hipStream_t st = nullptr;
    DW_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    side.push_back(st);
  }
  evs.assign(launches.size() + 1, nullptr);
  for (size_t i = 0; i <= launches.size(); ++i)
    if (i == launches.size() || launches[i].record)
      DW_HIP(hipEventCreateWithFlags(&evs[i], hipEventDisableTiming));
}

void Runtime::enqueue(hipStream_t st) {
  for (auto& kv : nchw) {
    const NchwIn& e = kv.second;
    if (!e.active || e.launch >= 0) continue;
    const RtTensor& t = T(kv.first);
    launch_nchw_f32_to_nhwc(st, (const float*)e.src, t.base, (int)t.n, (int)t.c, (int)(t.h * t.w), t.dtype,
                            t.pix_stride, t.abs_off);
  }
  if (nstreams <= 1 || stats) {
    for (auto& L : launches) L.fn(st);
    return;
  }
  auto sk = [&](int k) { return k == 0 ? st : side[k - 1]; };
  hipEvent_t fork = evs.back();
  DW_HIP(hipEventRecord(fork, st));
  std::vector<bool> forked(nstreams, false);
  std::vector<int> last(nstreams, -1);
  for (size_t j = 0; j < launches.size(); ++j) {
    const Launch& L = launches[j];
    const hipStream_t s = sk(L.stream);
    if (L.stream != 0 && !forked[L.stream]) {
      DW_HIP(hipStreamWaitEvent(s, fork, 0));
      forked[L.stream] = true;
    }
    for (int w : L.waits) DW_HIP(hipStreamWaitEvent(s, evs[w], 0));
    L.fn(s);
    if (L.record) DW_HIP(hipEventRecord(evs[j], s));
    last[L.stream] = (int)j;
  }
  for (int k = 1; k < nstreams; ++k)
    if (last[k] >= 0) DW_HIP(hipStreamWaitEvent(st, evs[last[k]], 0));
}

// ---------------------------------------------------------------------------
// 1. fusion groups
// ---------------------------------------------------------------------------
void Runtime::lower(std::vector<Group>& groups) {
  const int nops = (int)g.ops.size();
  std::vector<bool> used(nops, false);
  auto single = [&](const std::string& t) -> int {
    if (stats || g.is_output(t)) return -1;
    auto cs = g.consumers(t);
    return cs.size() == 1 ? cs[0] : -1;
  };
  auto computed_before = [&](const std::string& t, int idx) {
    if (g.t[t].is_init) return false;
    const int p = g.producer(t);
    return p < idx;  // graph inputs have no producer (-1)
  };
  // DequantizeLinear absorbed into the fp16 conv that is its only consumer.
  std::map<int, int> dq_into;  // conv op -> dq op
  if (!stats) {
    for (int i = 0; i < nops; ++i)
      if (g.ops[i].type == "DequantizeLinear") {
        const int c = single(g.ops[i].out[0]);
        if (c >= 0 && g.ops[c].type == "Conv") {
          dq_into[c] = i;
          used[i] = true;
        }
      }
  }

  for (int i = 0; i < nops; ++i) {
    if (used[i]) continue;
    const OpNode& op = g.ops[i];
    Group gr;
    gr.ops = {i};
    used[i] = true;
    if (op.type == "Conv" && op.p.group > 1) {
      // CpuGraphRuntime::dispatch_conv2d: depthwise when group == c_in
      // (runtime.rs:1412-1421); other groupings are an error there too.
      if (op.p.group != T(op.in[0]).c || T(op.out[0]).c != T(op.in[0]).c)
        fail(DW_ERR_UNSUPPORTED, "runtime: general grouped convolution (" + op.name + ")");
      gr.kind = "dwconv";
      gr.conv = i;
      gr.in = op.in[0];
      std::string cur = op.out[0];
      int c = op.p.has_relu ? -1 : single(cur);
      if (op.p.has_relu) {
        gr.act = ACT_RELU;  // Conv + Relu fused by apply_fusion_passes
      } else if (c >= 0 && (g.ops[c].type == "Relu" || g.ops[c].type == "SiLU")) {
        gr.act = g.ops[c].type == "Relu" ? ACT_RELU : ACT_SILU;
      } else if (!stats && !g.is_output(cur)) {
        auto cs = g.consumers(cur);
        if (cs.size() == 2) {
          int s = -1, m = -1;
          for (int k : cs) {
            if (g.ops[k].type == "Sigmoid") s = k;
            if (g.ops[k].type == "Mul") m = k;
          }
          if (s >= 0 && m >= 0 && single(g.ops[s].out[0]) == m) {
            gr.act = ACT_SILU;
            used[s] = true;
            gr.ops.push_back(s);
            T(g.ops[s].out[0]).materialized = false;
            c = m;
          }
        }
      }
      if (gr.act != ACT_NONE && c >= 0) {
        used[c] = true;
        gr.ops.push_back(c);
        T(cur).materialized = false;
        cur = g.ops[c].out[0];
      }
      gr.out = cur;
      groups.push_back(gr);
      continue;
    }
    if (op.type == "Conv2dRequantReluI8" || (op.type == "Conv" && T(op.in[0]).dtype == I8)) {
      // the reference's INT8 conv: s8 x s8 -> int32, then (fused, or as the
      // following Requantize [+ Relu]) requantize_i32_to_i8 with one scale
      gr.kind = "iconv";
      gr.conv = i;
      gr.in = op.in[0];
      std::string cur = op.out[0];
      if (op.type == "Conv2dRequantReluI8") {
        gr.requant = true;
        gr.requant_scale = op.p.scale;
        gr.act = op.p.has_relu ? ACT_RELU : ACT_NONE;
      } else {
        const int rq = single(cur);
        if (rq >= 0 && g.ops[rq].type == "Requantize" && T(g.ops[rq].out[0]).dtype == I8) {
          used[rq] = true;
          gr.ops.push_back(rq);
          T(cur).materialized = false;
          cur = g.ops[rq].out[0];
          gr.requant = true;
          gr.requant_scale = g.ops[rq].p.scale;
          const int rl = single(cur);
          if (rl >= 0 && g.ops[rl].type == "Relu" && T(g.ops[rl].out[0]).dtype == I8) {
            used[rl] = true;
            gr.ops.push_back(rl);
            T(cur).materialized = false;
            cur = g.ops[rl].out[0];
            gr.act = ACT_RELU;
          }
        }
      }
      gr.out = cur;
      groups.push_back(gr);
      continue;
    }
    if (op.type == "Conv") {
      const dw_op_params& p = op.p;
      if ((p.dilations[0] > 1) || (p.dilations[1] > 1)) fail(DW_ERR_UNSUPPORTED, "runtime: dilation != 1");
      gr.kind = "conv";
      gr.conv = i;
      gr.in = op.in[0];
      gr.out = op.out[0];
      const int xdt = T(op.in[0]).dtype;
      gr.in_kind = xdt == F32 ? 0 : 1;
      auto dq = dq_into.find(i);
      if (dq != dq_into.end()) {
        const OpNode& d = g.ops[dq->second];
        gr.in = d.in[0];
        gr.in_kind = 2;
        gr.in_scale = T(d.in[0]).scale;
        gr.in_zp = T(d.in[0]).zp;
        gr.ops.insert(gr.ops.begin(), dq->second);
        T(d.out[0]).materialized = false;
      }
      gr.out_kind = T(op.out[0]).dtype == F32 ? 0 : 1;
      std::string cur = op.out[0];
      int c = op.p.has_relu ? -1 : single(cur);
      if (op.p.has_relu) {
        gr.act = ACT_RELU;  // Conv + Relu fused by apply_fusion_passes
      } else if (c >= 0 && g.ops[c].type == "Relu") {
        gr.act = ACT_RELU;
      } else if (c >= 0 && g.ops[c].type == "SiLU") {
        gr.act = ACT_SILU;
      } else if (!stats && !g.is_output(cur)) {
        auto cs = g.consumers(cur);
        if (cs.size() == 2) {
          int s = -1, m = -1;
          for (int k : cs) {
            if (g.ops[k].type == "Sigmoid") s = k;
            if (g.ops[k].type == "Mul") m = k;
          }
          if (s >= 0 && m >= 0 && single(g.ops[s].out[0]) == m) {
            const OpNode& mul = g.ops[m];
            if ((mul.in[0] == cur && mul.in[1] == g.ops[s].out[0]) ||
                (mul.in[1] == cur && mul.in[0] == g.ops[s].out[0])) {
              gr.act = ACT_SILU;
              used[s] = true;
              gr.ops.push_back(s);
              T(g.ops[s].out[0]).materialized = false;
              c = m;
            }
          }
        }
      }
      if (gr.act != ACT_NONE && c >= 0) {
        used[c] = true;
        gr.ops.push_back(c);
        T(cur).materialized = false;
        cur = g.ops[c].out[0];
      }
      // fp16 conv of a u8 graph feeding QuantizeLinear (+ table)
      int qc = single(cur);
      if (qc >= 0 && g.ops[qc].type == "QuantizeLinear") {
        used[qc] = true;
        gr.ops.push_back(qc);
        T(cur).materialized = false;
        cur = g.ops[qc].out[0];
        gr.out_kind = 2;
        int lc = single(cur);
        if (lc >= 0 && g.ops[lc].type == "QLinearLUT") {
          used[lc] = true;
          gr.ops.push_back(lc);
          gr.lut = true;
          gr.pre = cur;
          T(cur).materialized = false;
          cur = g.ops[lc].out[0];
        }
      }
      // residual add (f16 MFMA path only)
      int ac = single(cur);
      const bool mfma = g.dtype == DW_GRAPH_F16 && gr.in_kind == 1 && gr.out_kind == 1 &&
                        (T(gr.in).c * 2) % 16 == 0 && T(gr.out).c % 4 == 0;
      if (mfma && ac >= 0 && g.ops[ac].type == "Add") {
        const OpNode& add = g.ops[ac];
        const std::string other = add.in[0] == cur ? add.in[1] : add.in[0];
        if (other != cur && computed_before(other, i) && T(other).rank4 &&
            T(other).dtype == F16 && T(other).c == T(cur).c) {
          used[ac] = true;
          gr.ops.push_back(ac);
          gr.res = other;
          T(cur).materialized = false;
          cur = add.out[0];
        }
      }
      gr.out = cur;
      groups.push_back(gr);
      continue;
    }
    if (op.type == "QLinearConv" || op.type == "QGemm") {
      // QGemm is the QLinearConv definition on a 1x1 kernel over the rows
      // of A (its weights are stored as [1][1][k][n])
      gr.kind = "qconv";
      gr.conv = i;
      gr.in = op.in[0];
      gr.pre = op.out[0];
      std::string cur = op.out[0];
      int lc = single(cur);
      if (lc >= 0 && g.ops[lc].type == "QLinearLUT") {
        used[lc] = true;
        gr.ops.push_back(lc);
        gr.lut = true;
        T(cur).materialized = false;
        cur = g.ops[lc].out[0];
        gr.lut_out = cur;
      }
      int ac = single(cur);
      if (ac >= 0 && g.ops[ac].type == "QLinearAdd") {
        const OpNode& add = g.ops[ac];
        const std::string other = add.in[0] == cur ? add.in[1] : add.in[0];
        if (other != cur && computed_before(other, i) && T(other).rank4 && T(other).c == T(cur).c) {
          used[ac] = true;
          gr.ops.push_back(ac);
          gr.res = other;
          T(cur).materialized = false;
          cur = add.out[0];
        }
      }
      gr.out = cur;
      groups.push_back(gr);
      continue;
    }
    if (op.type == "MaxPool") {
      const dw_op_params& p = op.p;
      const int k = p.kernel_shape[0];
      auto cascade_ok = [&](const OpNode& o) {
        const dw_op_params& q = o.p;
        return o.type == "MaxPool" && q.kernel_shape[0] == k && q.kernel_shape[1] == k && q.strides[0] == 1 &&
               q.strides[1] == 1 && q.pads[0] == k / 2 && q.pads[1] == k / 2 && q.pads[2] == k / 2 &&
               q.pads[3] == k / 2 && (k % 2) == 1;
      };
      if (!stats && cascade_ok(op)) {
        int j2 = -1, j3 = -1;
        for (int cidx : g.consumers(op.out[0]))
          if (!used[cidx] && cascade_ok(g.ops[cidx])) j2 = cidx;
        if (j2 >= 0)
          for (int cidx : g.consumers(g.ops[j2].out[0]))
            if (!used[cidx] && cascade_ok(g.ops[cidx])) j3 = cidx;
        if (j2 >= 0 && j3 >= 0) {
          gr.kind = "pool3";
          gr.ops = {i, j2, j3};
          used[j2] = used[j3] = true;
          groups.push_back(gr);
          continue;
        }
      }
      gr.kind = "pool";
      groups.push_back(gr);
      continue;
    }
    if (op.type == "GlobalAveragePool" || op.type == "QLinearGlobalAveragePool") {
      gr.kind = "gap";
    } else if (op.type == "Gemm" || op.type == "MatMul") {
      gr.kind = "gemm";
    } else if (op.type == "Flatten" || op.type == "Reshape") {
      gr.kind = "flatten";
    } else if (op.type == "Softmax") {
      gr.kind = "softmax";
    } else if (op.type == "YoloDetect") {
      gr.kind = "detect";
    } else if (op.type == "Resize") {
      if (!op.p.mode_nearest) fail(DW_ERR_UNSUPPORTED, "runtime: only nearest Resize is implemented");
      gr.kind = "resize";
    } else if (op.type == "Concat") {
      gr.kind = op.p.axis == 3 ? "concat" : "concat_copy";
    } else if (op.type == "Split") {
      gr.kind = op.p.axis == 3 ? "split" : "split_copy";
    } else if (op.type == "Transpose" || op.type == "LayoutTranspose") {
      gr.kind = "transpose";
    } else if (op.type == "Slice") {
      gr.kind = "slice";
    } else if (op.type == "AveragePool") {
      gr.kind = "avgpool";
    } else if (op.type == "Sub" || op.type == "Div" ||
               ((op.type == "Add" || op.type == "Mul") && op.in.size() == 2 &&
                (g.t[op.in[0]].is_init || g.t[op.in[1]].is_init || g.t[op.in[0]].dims != g.t[op.in[1]].dims))) {
      gr.kind = "bin";
    } else if (op.type == "Relu" || op.type == "Sigmoid" || op.type == "Mul" || op.type == "Add" ||
               op.type == "SiLU" || op.type == "QLinearLUT" || op.type == "QLinearAdd" ||
               op.type == "QuantizeLinear" || op.type == "DequantizeLinear" || op.type == "Requantize" ||
               op.type == "AddQuantized" || op.type == "Quantize" || op.type == "Dequantize" ||
               op.type == "Clip") {
      gr.kind = "ew";
    } else {
      fail(DW_ERR_UNSUPPORTED, "runtime: no kernel for op type '" + op.type + "' (" + op.name + ")");
    }
    groups.push_back(gr);
  }
}

// ---------------------------------------------------------------------------
// 2. placement of concat inputs and split outputs
// ---------------------------------------------------------------------------
void Runtime::place(const std::vector<Group>& groups) {
  std::set<std::string> protect(g.inputs.begin(), g.inputs.end());
  for (auto& o : g.outputs) protect.insert(o);
  // Split outputs: slices of the input.
  for (auto& gr : groups) {
    if (gr.kind != "split") continue;
    const OpNode& op = g.ops[gr.ops[0]];
    if (op.p.axis != 3) fail(DW_ERR_UNSUPPORTED, "runtime: Split only along channels");
    int off = 0;
    for (size_t k = 0; k < op.out.size(); ++k) {
      RtTensor& o = T(op.out[k]);
      if (protect.count(op.out[k])) fail(DW_ERR_UNSUPPORTED, "runtime: split output as graph output");
      o.parent = op.in[0];
      o.c_off = off;
      off += (int)o.c;
    }
  }
  // Walks split parents up to the storage root; returns "" if the tensor
  // already lives inside another concat's buffer.
  std::set<std::string> concat_placed;
  auto root_of = [&](std::string t, int& off) -> std::string {
    off = 0;
    while (!T(t).parent.empty()) {
      if (concat_placed.count(t)) return "";
      off += T(t).c_off;
      t = T(t).parent;
    }
    return t;
  };
  // Producers that write dense tensors only (no channel-strided output
  // view): their outputs are copied into a concat buffer, not placed in it.
  std::set<std::string> dense_only;
  for (auto& gr : groups)
    if (gr.kind == "flatten" || gr.kind == "softmax" || gr.kind == "gemm" || gr.kind == "gap" ||
        gr.kind == "avgpool" || gr.kind == "detect")
      for (int oi : gr.ops)
        for (auto& o : g.ops[oi].out) dense_only.insert(o);
  // Concats, last first, so nested placements resolve through parents.
  for (auto it = groups.rbegin(); it != groups.rend(); ++it) {
    if (it->kind != "concat") continue;
    const OpNode& op = g.ops[it->ops[0]];
    if (op.p.axis != 3) fail(DW_ERR_UNSUPPORTED, "runtime: Concat only along channels");
    const std::string out = op.out[0];
    const int total = (int)T(out).c;
    int off = 0;
    std::map<std::string, int> want;  // root -> offset inside `out`
    std::set<std::string> bad;
    std::vector<std::pair<std::string, int>> ins;
    for (auto& in : op.in) {
      ins.push_back({in, off});
      off += (int)T(in).c;
    }
    for (auto& pr : ins) {
      int roff = 0;
      const std::string r = root_of(pr.first, roff);
      if (r.empty()) continue;
      const int d = pr.second - roff;
      if (protect.count(r) || g.t[r].is_init || !T(r).parent.empty() || r == out || dense_only.count(r) ||
          T(r).dtype != T(out).dtype || d < 0 || d + T(r).c > total || (d % 16) != 0 || (total % 16) != 0 ||
          T(r).pixels() != T(out).pixels()) {
        bad.insert(r);
        continue;
      }
      auto w = want.find(r);
      if (w != want.end() && w->second != d) bad.insert(r);
      want[r] = d;
    }
    for (auto& kv : want) {
      if (bad.count(kv.first)) continue;
      T(kv.first).parent = out;
      T(kv.first).c_off = kv.second;
      concat_placed.insert(kv.first);
    }
  }
}

// Activation storage.  Every storage root (a materialized tensor without a
// parent, or a concat buffer its inputs are placed in) is touched by a set
// of groups; graph inputs and outputs are kept apart.  Roots are placed in
// one arena, largest first, each at the lowest 256-byte-aligned offset that
// no placed root it may not share with occupies (the liveness reuse of the
// reference's slab allocator, slab.rs:228-367).  Two roots share only when
// the data dependencies already order every use of one before every use of
// the other, so independent branches (the detect heads) keep running
// concurrently.  The stream schedule orders launches by the bytes they
// touch (Region) in any case.  DW_ACT_REUSE=0 gives every root its own
// bytes.
void Runtime::allocate(const std::vector<Group>& groups) {
  auto root_of = [&](std::string t) {
    while (!T(t).parent.empty()) t = T(t).parent;
    return t;
  };
  auto is_io = [&](const std::string& n) {
    return g.is_output(n) || std::find(g.inputs.begin(), g.inputs.end(), n) != g.inputs.end();
  };
  // roots that need storage: graph inputs, outputs and every materialized
  // tensor without a parent, and the roots of placed tensors
  std::vector<std::string> roots;
  std::map<std::string, int> rid;
  auto add_root = [&](const std::string& r) {
    if (rid.count(r)) return;
    rid[r] = (int)roots.size();
    roots.push_back(r);
  };
  for (auto& kv : ts) {
    const RtTensor& r = kv.second;
    if (!r.rank4 || g.t[kv.first].is_init) continue;
    if (!r.parent.empty()) {
      add_root(root_of(kv.first));
      continue;
    }
    if (r.materialized || is_io(kv.first)) add_root(kv.first);
  }
  // the groups touching each root, and each group's storage as (root,
  // channels) regions, read and written
  auto root_off = [&](std::string t, int& o) {
    o = 0;
    while (!T(t).parent.empty()) {
      o += T(t).c_off;
      t = T(t).parent;
    }
    return t;
  };
  const int ng = (int)groups.size();
  std::vector<std::vector<int>> touch(roots.size());
  std::vector<std::vector<Region>> grd(ng), gwr(ng);
  for (int gi = 0; gi < ng; ++gi)
    for (int oi : groups[gi].ops) {
      const OpNode& op = g.ops[oi];
      for (int w = 0; w < 2; ++w)
        for (const auto& n : w ? op.out : op.in) {
          auto it = ts.find(n);
          if (it == ts.end() || !it->second.rank4 || g.t[n].is_init) continue;
          int o = 0;
          auto r = rid.find(root_off(n, o));
          if (r == rid.end()) continue;
          auto& tv = touch[r->second];
          if (tv.empty() || tv.back() != gi) tv.push_back(gi);
          (w ? gwr : grd)[gi].push_back({r->second, o, o + (int)it->second.c, 0, 0});
        }
    }
  // ancestors of each group along data dependencies (one group writes
  // storage the other reads or writes): the order every stream schedule
  // keeps whatever the placement
  std::vector<std::vector<char>> anc(ng, std::vector<char>(ng, 0));
  auto dep = [&](int i, int j) {
    for (const Region& w : gwr[i]) {
      for (const Region& r : grd[j]) if (w.overlaps(r)) return true;
      for (const Region& r : gwr[j]) if (w.overlaps(r)) return true;
    }
    for (const Region& r : grd[i])
      for (const Region& w : gwr[j]) if (r.overlaps(w)) return true;
    return false;
  };
  for (int j = 0; j < ng; ++j)
    for (int i = 0; i < j; ++i)
      if (!anc[j][i] && dep(i, j)) {
        anc[j][i] = 1;
        for (int k = 0; k < i; ++k) anc[j][k] |= anc[i][k];
      }
  bool reuse = true;
  if (const char* e = getenv("DW_ACT_REUSE")) reuse = atoi(e) != 0;
  std::vector<char> pinned(roots.size(), 0);
  for (size_t i = 0; i < roots.size(); ++i) {
    pinned[i] = !reuse || touch[i].empty() || is_io(roots[i]);
    for (auto& kv : ts)  // a root holding a graph input or output
      if (!pinned[i] && kv.second.rank4 && is_io(kv.first) && !kv.second.parent.empty() &&
          root_of(kv.first) == roots[i])
        pinned[i] = 1;
  }
  // Two roots may share bytes when every group touching one is an ancestor
  // of every group touching the other: the data dependencies then already
  // order all uses of the first before any use of the second, so sharing
  // adds no wait to the stream schedule.
  auto before = [&](int a, int b) {
    for (int gb : touch[b])
      for (int ga : touch[a])
        if (ga >= gb || !anc[gb][ga]) return false;
    return true;
  };
  auto conflict = [&](int a, int b) { return pinned[a] || pinned[b] || !(before(a, b) || before(b, a)); };
  auto align = [](size_t v) { return (v + 255) & ~(size_t)255; };
  std::vector<size_t> size(roots.size()), off(roots.size(), 0);
  for (size_t i = 0; i < roots.size(); ++i) size[i] = align(std::max<size_t>(T(roots[i]).bytes(), 256));
  std::vector<int> order(roots.size());
  for (size_t i = 0; i < order.size(); ++i) order[i] = (int)i;
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return size[a] > size[b]; });
  std::vector<int> placed;
  size_t total = 0;
  for (int i : order) {
    // occupied byte ranges of the placed roots it may not share with
    std::vector<std::pair<size_t, size_t>> busy;
    for (int j : placed)
      if (conflict(i, j)) busy.push_back({off[j], off[j] + size[j]});
    std::sort(busy.begin(), busy.end());
    size_t o = 0;
    for (auto& b : busy) {
      if (o + size[i] <= b.first) break;
      o = std::max(o, b.second);
    }
    off[i] = o;
    placed.push_back(i);
    total = std::max(total, o + size[i]);
  }
  uint8_t* arena = (uint8_t*)dalloc(total);
  act_bytes = total;
  act_bytes_unshared = 0;
  for (size_t i = 0; i < roots.size(); ++i) {
    act_bytes_unshared += size[i];
    RtTensor& r = T(roots[i]);
    r.base = arena + off[i];
    r.pix_stride = (int)r.c;
    r.abs_off = 0;
    r.rid = (int)i;
    r.ra0 = (uintptr_t)r.base;
    r.ra1 = r.ra0 + size[i];
  }
  for (auto& kv : ts) {
    RtTensor& r = kv.second;
    if (r.parent.empty()) continue;
    int o = 0;
    std::string t = kv.first;
    while (!T(t).parent.empty()) {
      o += T(t).c_off;
      t = T(t).parent;
    }
    const RtTensor& root = T(t);
    r.base = root.base;
    r.pix_stride = root.pix_stride;
    r.abs_off = o;
    r.rid = root.rid;
    r.ra0 = root.ra0;
    r.ra1 = root.ra1;
  }
}

// ---------------------------------------------------------------------------
// 4. launches
// ---------------------------------------------------------------------------
namespace {
std::string join_names(const GraphIR& g, const std::vector<int>& ops) {
  std::string s;
  for (int i : ops) s += (s.empty() ? "" : "+") + g.ops[i].name;
  return s;
}
}  // namespace

void Runtime::emit(const Group& gr) {
  if (gr.kind == "conv") return emit_conv(gr);
  if (gr.kind == "dwconv") {
    const OpNode& op = g.ops[gr.conv];
    const TensorInfo& W = g.t[op.in[1]];
    RtTensor& x = T(gr.in);
    RtTensor& y = T(gr.out);
    // weights [kh][kw][c][1] (HWIO with one output per group)
    if (W.dims.size() != 4 || W.dims[2] != 1 || W.dims[3] != x.c)
      fail(DW_ERR_UNSUPPORTED, "runtime: depthwise weights must be [kh,kw,1,C] after NHWC conversion");
    if (x.c % 8 != 0 || x.pix_stride % 8 != 0 || x.abs_off % 8 != 0 || y.pix_stride % 8 != 0 ||
        y.abs_off % 8 != 0)
      fail(DW_ERR_UNSUPPORTED, "runtime: depthwise needs 8-channel aligned views (" + op.name + ")");
    if (x.dtype != F16 && x.dtype != F32) fail(DW_ERR_UNSUPPORTED, "runtime: depthwise dtype");
    DwArgs a{};
    a.x = x.base;
    a.y = y.base;
    a.wt = upload(W.data.data(), W.data.size());
    if (op.in.size() > 2 && !op.in[2].empty()) a.bias = upload(g.t[op.in[2]].data.data(), g.t[op.in[2]].data.size());
    if (x.dtype == F16) {
      a.w_plain = 1;
      const uint16_t* wh = (const uint16_t*)W.data.data();
      for (size_t i = 0; i < W.data.size() / 2; ++i)
        if ((wh[i] & 0x7C00u) == 0 && (wh[i] & 0x03FFu) != 0) a.w_plain = 0;
    }
    a.n = (int)x.n; a.h = (int)x.h; a.w = (int)x.w; a.c = (int)x.c;
    a.kh = (int)W.dims[0]; a.kw = (int)W.dims[1];
    a.sh = std::max(1, op.p.strides[0]); a.sw = std::max(1, op.p.strides[1]);
    a.pt = op.p.pads[0]; a.pl = op.p.pads[1]; a.ho = (int)y.h; a.wo = (int)y.w;
    a.act = gr.act;
    a.x_pix_stride = x.pix_stride; a.x_c_off = x.abs_off;
    a.y_pix_stride = y.pix_stride; a.y_c_off = y.abs_off;
    const int dt = x.dtype;
    Launch L;
    L.kernel = dt == F16 ? "dwconv_f16" : "dwconv_f32";
    L.op = join_names(g, gr.ops);
    L.work = 2.0 * (double)y.pixels() * y.c * a.kh * a.kw;
    L.bytes = (double)x.bytes() + (double)y.bytes() + W.data.size() + (a.bias ? y.c * dtype_size(dt) : 0);
    if (dt == F16 && !exact_f16_dw && (dwconv3_tile_cfg_ok(a, 8, 4) || dwconv3_tile_cfg_ok(a, 4, 4))) {
      // packed-f16 band kernel (fp16 tolerance); the tuner picks the band height
      L.kernel = "dwconv3_tile";
      L.dwa = std::make_shared<DwArgs>(a);
      L.dw_band = std::make_shared<int>(dwconv3_tile_cfg_ok(a, 8, 4) ? 804 : 404);
      L.fn = [a, cfg = L.dw_band](hipStream_t st) { launch_dwconv3_tile(st, a, *cfg / 100, *cfg % 100); };
      launches.push_back(L);
      return;
    }
    L.fn = [=](hipStream_t st) { launch_dwconv(st, a, dt); };
    launches.push_back(L);
    return;
  }
  if (gr.kind == "qconv") return emit_qconv(gr);
  if (gr.kind == "iconv") return emit_iconv(gr);
  if (gr.kind == "split") return;
  if (gr.kind == "concat") {
    const OpNode& op = g.ops[gr.ops[0]];
    RtTensor& out = T(op.out[0]);
    int off = 0;
    for (auto& in : op.in) {
      RtTensor& ti = T(in);
      int roff = 0;
      std::string t = in;
      while (!T(t).parent.empty()) {
        roff += T(t).c_off;
        t = T(t).parent;
      }
      const bool placed = ti.base == out.base && ti.abs_off == out.abs_off + off;
      if (!placed) {
        View src = ti.view(), dst = out.view();
        dst.c_off += off;
        const int px = (int)ti.pixels(), ch = (int)ti.c, es = dtype_size(ti.dtype);
        Launch L;
        L.kernel = "copy_channels";
        L.op = op.name + ":" + in;
        L.bytes = 2.0 * px * ch * es;
        L.fn = [=](hipStream_t st) { launch_copy_channels(st, src, dst, px, ch, es); };
        launches.push_back(L);
      }
      off += (int)ti.c;
    }
    return;
  }
  if (gr.kind == "pool" || gr.kind == "pool3") {
    const OpNode& op = g.ops[gr.ops[0]];
    RtTensor& x = T(op.in[0]);
    RtTensor& y = T(op.out[0]);
    PoolArgs a{};
    a.x = x.view();
    a.y = y.view();
    a.n = (int)x.n; a.h = (int)x.h; a.w = (int)x.w; a.c = (int)x.c;
    a.kh = op.p.kernel_shape[0]; a.kw = op.p.kernel_shape[1];
    a.sh = std::max(1, op.p.strides[0]); a.sw = std::max(1, op.p.strides[1]);
    a.pt = op.p.pads[0]; a.pl = op.p.pads[1];
    a.ho = (int)y.h; a.wo = (int)y.w;
    const int dt = x.dtype;
    Launch L;
    L.op = join_names(g, gr.ops);
    if (gr.kind == "pool3") {
      View y2 = T(g.ops[gr.ops[1]].out[0]).view(), y3 = T(g.ops[gr.ops[2]].out[0]).view();
      L.kernel = "maxpool_cascade3";
      L.bytes = 4.0 * x.bytes();
      L.fn = [=](hipStream_t st) { launch_maxpool_cascade3(st, a, y2, y3, dt); };
    } else {
      L.kernel = "maxpool";
      L.bytes = (double)x.bytes() + y.bytes();
      L.fn = [=](hipStream_t st) { launch_maxpool(st, a, dt); };
    }
    launches.push_back(L);
    return;
  }
  if (gr.kind == "resize") {
    const OpNode& op = g.ops[gr.ops[0]];
    RtTensor& x = T(op.in[0]);
    RtTensor& y = T(op.out[0]);
    ResizeArgs a{};
    a.x = x.view();
    a.y = y.view();
    a.n = (int)x.n; a.h = (int)x.h; a.w = (int)x.w; a.c = (int)x.c; a.ho = (int)y.h; a.wo = (int)y.w;
    const int dt = x.dtype;
    Launch L;
    L.kernel = "resize_nearest";
    L.op = op.name;
    L.bytes = (double)x.bytes() + y.bytes();
    L.ra = std::make_shared<ResizeArgs>(a);
    L.rdtype = dt;
    L.t_in = op.in[0];
    L.t_out = op.out[0];
    L.fn = [ra = L.ra, dt](hipStream_t st) { launch_resize_nearest(st, *ra, dt); };
    launches.push_back(L);
    return;
  }
  if (gr.kind == "transpose" || gr.kind == "slice" || gr.kind == "bin" || gr.kind == "avgpool" ||
      gr.kind == "concat_copy" || gr.kind == "split_copy")
    return emit_shape(gr);
  if (gr.kind == "flatten") {
    // Reshape / Flatten: the row-major order of the elements is kept; a
    // dense input is one copy, a channel view a strided one
    const OpNode& op = g.ops[gr.ops[0]];
    RtTensor& x = T(op.in[0]);
    RtTensor& y = T(op.out[0]);
    if (x.bytes() != y.bytes() || x.dtype != y.dtype) fail(DW_ERR_RUNTIME, op.type + " " + op.name + ": element count");
    Launch L;
    L.op = op.name;
    L.bytes = (double)x.bytes() + y.bytes();
    if (y.pix_stride != y.c || y.abs_off != 0) fail(DW_ERR_RUNTIME, op.type + " " + op.name + ": output view");
    if (x.pix_stride == x.c && x.abs_off == 0) {
      const void* xb = x.base;
      void* yb = y.base;
      const size_t nb = x.bytes();
      L.kernel = "copy";
      L.fn = [=](hipStream_t st) { DW_HIP(hipMemcpyAsync(yb, xb, nb, hipMemcpyDeviceToDevice, st)); };
    } else {
      StridedCopyArgs c{};
      c.x = x.base;
      c.y = y.base;
      c.esize = dtype_size(x.dtype);
      c.dims[0] = c.dims[1] = 1;
      c.dims[2] = x.pixels();
      c.dims[3] = x.c;
      c.xs[2] = x.pix_stride; c.xs[3] = 1;
      c.ys[2] = x.c; c.ys[3] = 1;
      c.x_off = x.abs_off;
      L.kernel = "strided_copy";
      L.fn = [=](hipStream_t st) { launch_strided_copy(st, c); };
    }
    launches.push_back(L);
    return;
  }
  if (gr.kind == "gap" || gr.kind == "gemm" || gr.kind == "softmax") {
    // classifier-head ops: dense tensors only
    const OpNode& op = g.ops[gr.ops[0]];
    RtTensor& x = T(op.in[0]);
    RtTensor& y = T(op.out[0]);
    auto dense = [](const RtTensor& t) { return t.rank4 && t.pix_stride == t.c && t.abs_off == 0; };
    if (!dense(x) || !dense(y)) fail(DW_ERR_UNSUPPORTED, "runtime: " + op.type + " on a channel slice");
    Launch L;
    L.op = op.name;
    L.bytes = (double)x.bytes() + y.bytes();
    const int dt = x.dtype;
    if (dt != F32 && dt != F16 && gr.kind != "flatten" && !(gr.kind == "gap" && dt == U8))
      fail(DW_ERR_UNSUPPORTED, "runtime: " + op.type + " needs f32 or f16");
    const void* xb = x.base;
    void* yb = y.base;
    if (gr.kind == "softmax") {
      // CpuGraphRuntime::dispatch_softmax (runtime.rs:1288-1326): along the
      // last dimension; an axis other than the last is refused (after
      // convert_nchw_to_nhwc, a 4-D tensor's axes are NHWC positions)
      const int rank = (int)g.t[op.in[0]].dims.size();
      const int ax = op.p.axis < 0 ? op.p.axis + rank : op.p.axis;
      if (ax != rank - 1) fail(DW_ERR_UNSUPPORTED, "Softmax " + op.name + ": only along the last axis");
      if (y.dtype != dt || x.bytes() != y.bytes()) fail(DW_ERR_RUNTIME, "Softmax: output shape or dtype");
      const int rows = (int)x.pixels(), n = (int)x.c;
      L.kernel = "softmax";
      L.fn = [=](hipStream_t st) { launch_softmax_rows_t(st, dt, xb, yb, rows, n); };
    } else if (gr.kind == "gap") {
      if (y.pixels() != x.n || y.c != x.c) fail(DW_ERR_RUNTIME, "GlobalAveragePool: output shape");
      const int n = (int)x.n, hw = (int)(x.h * x.w), c = (int)x.c;
      L.kernel = "global_avg_pool";
      if (dt == U8) {
        // QLinearGlobalAveragePool
        if (y.dtype != U8) fail(DW_ERR_RUNTIME, "QLinearGlobalAveragePool: u8 output");
        const float m = (x.scale / y.scale) / (float)hw;
        const int xz = x.zp, yz = y.zp;
        L.fn = [=](hipStream_t st) {
          launch_qlinear_gap(st, (const uint8_t*)xb, (uint8_t*)yb, n, hw, c, xz, m, yz);
        };
      } else {
        L.fn = [=](hipStream_t st) { launch_global_avg_pool(st, dt, xb, yb, n, hw, c); };
      }
    } else {
      // Gemm / MatMul (dispatch_gemm, onnx runtime.rs:1178-1275): A [m][k]
      // activation, B an initializer ([k][n], or [n][k] with trans_b),
      // optional bias over the columns
      const bool tb = op.type == "Gemm" && op.p.trans_b;
      if (op.type == "Gemm" && op.p.trans_a) fail(DW_ERR_UNSUPPORTED, "Gemm: transA");
      const TensorInfo& B = g.t.at(op.in[1]);
      if (!B.is_init || B.dims.size() != 2) fail(DW_ERR_UNSUPPORTED, "Gemm: B must be a 2-D initializer");
      const int m = (int)x.n, k = (int)x.c;
      const int n = (int)(tb ? B.dims[0] : B.dims[1]);
      if ((tb ? B.dims[1] : B.dims[0]) != k) fail(DW_ERR_RUNTIME, "Gemm: inner dimensions differ");
      if (y.pixels() != m || y.c != n) fail(DW_ERR_RUNTIME, "Gemm: output shape");
      if (B.dtype != dt) fail(DW_ERR_UNSUPPORTED, "Gemm: A and B element types differ");
      const void* wb = upload(B.data.data(), B.data.size());
      const void* bb = nullptr;
      int blen = 0;
      if (op.in.size() > 2 && !op.in[2].empty()) {
        const TensorInfo& Bi = g.t.at(op.in[2]);
        if (!Bi.is_init || Bi.dtype != dt) fail(DW_ERR_UNSUPPORTED, "Gemm: bias must be an initializer of A's type");
        bb = upload(Bi.data.data(), Bi.data.size());
        blen = (int)Bi.numel();
        if (blen <= 0) fail(DW_ERR_RUNTIME, "Gemm: empty bias");
      }
      L.kernel = "gemm";
      L.bytes += (double)B.data.size();
      L.fn = [=](hipStream_t st) { launch_gemm_ex(st, dt, xb, wb, yb, m, n, k, tb, bb, blen); };
    }
    launches.push_back(L);
    return;
  }
  if (gr.kind == "detect") {
    // YOLOv8 detect tail (k_detect.hip): the per-level head outputs, each a
    // dense or channel-strided NHWC tensor, into [n][4 + nc][A] f32
    const OpNode& op = g.ops[gr.ops[0]];
    const int levels = (int)op.in.size();
    if (levels < 1 || levels > 4) fail(DW_ERR_UNSUPPORTED, "YoloDetect: 1 to 4 inputs");
    const int reg_max = op.p.reg_max;
    if (reg_max < 1) fail(DW_ERR_RUNTIME, "YoloDetect: reg_max");
    DetectTailArgs t{};
    const RtTensor& x0 = T(op.in[0]);
    const int dt = x0.dtype;
    if (dt != F16 && dt != F32) fail(DW_ERR_UNSUPPORTED, "YoloDetect: f16 or f32 inputs");
    const int nc = (int)x0.c - 4 * reg_max;
    if (nc < 1) fail(DW_ERR_RUNTIME, "YoloDetect: fewer channels than 4 * reg_max + 1");
    int64_t A = 0;
    Launch L;
    L.op = op.name;
    L.kernel = "detect_tail";
    for (int s = 0; s < levels; ++s) {
      const RtTensor& x = T(op.in[s]);
      if (x.dtype != dt || x.c != x0.c || x.n != x0.n) fail(DW_ERR_RUNTIME, "YoloDetect: inputs differ");
      t.x[s] = (const uint8_t*)x.base + (size_t)x.abs_off * dtype_size(dt);
      t.h[s] = (int)x.h;
      t.w[s] = (int)x.w;
      t.pix[s] = x.pix_stride;
      t.stride[s] = op.p.level_strides[s];
      A += x.h * x.w;
      L.bytes += (double)x.bytes();
    }
    const RtTensor& y = T(op.out[0]);
    if (y.dtype != F32 || y.pixels() * y.c != x0.n * (4 + nc) * A)
      fail(DW_ERR_RUNTIME, "YoloDetect: output must be f32 [n][4 + nc][A]");
    t.levels = levels;
    t.nc = nc;
    t.reg_max = reg_max;
    float* yb = (float*)y.base;
    const int n = (int)x0.n;
    L.bytes += (double)y.bytes();
    L.fn = [=](hipStream_t st) { launch_detect_tail(st, dt, t, yb, n); };
    launches.push_back(L);
    return;
  }
  if (gr.kind == "ew") return emit_ew(g.ops[gr.ops[0]]);
  fail(DW_ERR_RUNTIME, "runtime: unhandled group " + gr.kind);
}

Runtime::Addr4 Runtime::addr4(const std::string& name) {
  const TensorInfo& ti = g.t.at(name);
  Addr4 a;
  a.rank = (int)ti.dims.size();
  if (a.rank > 4) fail(DW_ERR_UNSUPPORTED, "runtime: '" + name + "' above rank 4");
  for (int k = 0; k < a.rank; ++k) a.d[4 - a.rank + k] = ti.dims[k];
  a.es = dtype_size(ti.dtype);
  if (ti.is_init) {
    a.base = upload(ti.data.data(), ti.data.size());
    a.st[3] = 1;
    for (int k = 2; k >= 0; --k) a.st[k] = a.st[k + 1] * a.d[k + 1];
    return a;
  }
  const RtTensor& r = T(name);
  if (a.d[3] != r.c) fail(DW_ERR_RUNTIME, "runtime: '" + name + "' layout");
  // rows of the last dimension, pix_stride elements apart
  a.base = r.base;
  a.off = r.abs_off;
  a.st[3] = 1;
  a.st[2] = r.pix_stride;
  a.st[1] = a.d[2] * a.st[2];
  a.st[0] = a.d[1] * a.st[1];
  return a;
}

// Transpose, Slice, broadcasting Add / Sub / Mul / Div, AveragePool, and
// Concat / Split along a non-channel axis (k_shape.hip).
void Runtime::emit_shape(const Group& gr) {
  const OpNode& op = g.ops[gr.ops[0]];
  Launch L;
  L.op = op.name;
  auto copy_launch = [&](const StridedCopyArgs& c, const std::string& what) {
    Launch C = L;
    C.op = what;
    C.kernel = "strided_copy";
    C.bytes = 2.0 * c.dims[0] * c.dims[1] * c.dims[2] * c.dims[3] * c.esize;
    C.fn = [c](hipStream_t st) { launch_strided_copy(st, c); };
    launches.push_back(C);
  };
  if (gr.kind == "transpose" || gr.kind == "slice") {
    const Addr4 x = addr4(op.in[0]), y = addr4(op.out[0]);
    if (x.es != y.es || x.rank != y.rank) fail(DW_ERR_RUNTIME, op.type + " " + op.name + ": operand types");
    StridedCopyArgs c{};
    c.x = x.base;
    c.y = y.base;
    c.esize = x.es;
    // the reference's f16 Transpose / Slice go through f32 (runtime.rs:2073-2084, :2130-2140)
    c.f16_round_trip = op.type != "LayoutTranspose" && T(op.in[0]).dtype == F16;
    c.x_off = x.off;
    c.y_off = y.off;
    for (int k = 0; k < 4; ++k) {
      c.dims[k] = y.d[k];
      c.ys[k] = y.st[k];
    }
    const int lead = 4 - x.rank;
    if (gr.kind == "transpose") {
      for (int k = 0; k < 4; ++k) {
        const int src = k < lead ? k : lead + op.p.perm[k - lead];
        if (src < 0 || src > 3 || x.d[src] != y.d[k]) fail(DW_ERR_RUNTIME, "Transpose " + op.name + ": perm");
        c.xs[k] = x.st[src];
      }
    } else {
      for (int k = 0; k < 4; ++k) c.xs[k] = x.st[k];
      for (int i = 0; i < op.p.num_slice_axes; ++i) {
        const int ax = lead + op.p.slice_axes[i];
        if (ax < 0 || ax > 3) fail(DW_ERR_RUNTIME, "Slice " + op.name + ": axis");
        c.x_off += (long long)op.p.slice_starts[i] * x.st[ax];
        c.xs[ax] *= op.p.slice_steps[i];
      }
    }
    copy_launch(c, op.name);
    return;
  }
  if (gr.kind == "concat_copy" || gr.kind == "split_copy") {
    const bool cat = gr.kind == "concat_copy";
    const std::string& whole = cat ? op.out[0] : op.in[0];
    const Addr4 w = addr4(whole);
    const int ax = op.p.axis;
    if (ax < 0 || ax > 3) fail(DW_ERR_RUNTIME, op.type + " " + op.name + ": axis");
    long long off = 0;
    for (auto& part : cat ? op.in : op.out) {
      const Addr4 pa = addr4(part);
      StridedCopyArgs c{};
      c.esize = pa.es;
      for (int k = 0; k < 4; ++k) c.dims[k] = pa.d[k];
      if (cat) {
        c.x = pa.base; c.y = w.base;
        c.x_off = pa.off;
        c.y_off = w.off + off * w.st[ax];
        for (int k = 0; k < 4; ++k) { c.xs[k] = pa.st[k]; c.ys[k] = w.st[k]; }
      } else {
        c.x = w.base; c.y = pa.base;
        c.x_off = w.off + off * w.st[ax];
        c.y_off = pa.off;
        for (int k = 0; k < 4; ++k) { c.xs[k] = w.st[k]; c.ys[k] = pa.st[k]; }
      }
      off += pa.d[ax];
      copy_launch(c, op.name + ":" + part);
    }
    if (off != w.d[ax]) fail(DW_ERR_RUNTIME, op.type + " " + op.name + ": sizes along the axis");
    return;
  }
  if (gr.kind == "bin") {
    const Addr4 a = addr4(op.in[0]), b = addr4(op.in[1]), y = addr4(op.out[0]);
    const int dt = T(op.out[0]).dtype;
    if (dt != F32 && dt != F16) fail(DW_ERR_UNSUPPORTED, op.type + " " + op.name + " needs f32 or f16");
    if (g.t[op.in[0]].dtype != dt || g.t[op.in[1]].dtype != dt)
      fail(DW_ERR_RUNTIME, op.type + " " + op.name + ": operand element types");
    BinaryArgs e{};
    e.a = a.base; e.b = b.base; e.y = y.base;
    e.a_off = a.off; e.b_off = b.off; e.y_off = y.off;
    e.f16 = dt == F16;
    e.op = op.type == "Add" ? BIN_ADD : op.type == "Sub" ? BIN_SUB : op.type == "Mul" ? BIN_MUL : BIN_DIV;
    for (int k = 0; k < 4; ++k) {
      e.dims[k] = y.d[k];
      e.ys[k] = y.st[k];
      // a size-1 axis broadcasts (stride 0)
      if ((a.d[k] != y.d[k] && a.d[k] != 1) || (b.d[k] != y.d[k] && b.d[k] != 1))
        fail(DW_ERR_RUNTIME, op.type + " " + op.name + ": operands do not broadcast to the output");
      e.as[k] = a.d[k] == 1 ? 0 : a.st[k];
      e.bs[k] = b.d[k] == 1 ? 0 : b.st[k];
    }
    L.kernel = "broadcast_binary";
    L.bytes = (double)(y.d[0] * y.d[1] * y.d[2] * y.d[3]) * y.es * 3.0;
    L.fn = [e](hipStream_t st) { launch_broadcast_binary(st, e); };
    launches.push_back(L);
    return;
  }
  // avgpool
  RtTensor& x = T(op.in[0]);
  RtTensor& y = T(op.out[0]);
  if (x.dtype != y.dtype || (x.dtype != F32 && x.dtype != F16))
    fail(DW_ERR_UNSUPPORTED, "AveragePool " + op.name + " needs f32 or f16");
  if (x.pix_stride != x.c || x.abs_off != 0 || y.pix_stride != y.c || y.abs_off != 0)
    fail(DW_ERR_RUNTIME, "AveragePool " + op.name + ": channel views");
  AvgPoolArgs a{};
  a.x = x.base; a.y = y.base;
  a.n = (int)x.n; a.h = (int)x.h; a.w = (int)x.w; a.c = (int)x.c;
  a.kh = op.p.kernel_shape[0]; a.kw = op.p.kernel_shape[1];
  a.sh = std::max(1, op.p.strides[0]); a.sw = std::max(1, op.p.strides[1]);
  a.ho = (int)y.h; a.wo = (int)y.w;
  a.f16 = x.dtype == F16;
  if (a.ho != (a.h - a.kh) / a.sh + 1 || a.wo != (a.w - a.kw) / a.sw + 1 || y.c != x.c || y.n != x.n)
    fail(DW_ERR_RUNTIME, "AveragePool " + op.name + ": output shape");
  L.kernel = "avgpool";
  L.bytes = (double)x.bytes() + y.bytes();
  L.fn = [a](hipStream_t st) { launch_avgpool(st, a); };
  launches.push_back(L);
}

void Runtime::emit_ew(const OpNode& op) {
  Ew2Args e{};
  RtTensor& a = T(op.in[0]);
  RtTensor& y = T(op.out[0]);
  e.a = a.view();
  e.y = y.view();
  e.pixels = (int)y.pixels();
  e.channels = (int)y.c;
  e.dtype = a.dtype;
  double bytes = (double)a.bytes() + y.bytes();
  if (op.in.size() > 1) {
    RtTensor& b = T(op.in[1]);
    if (b.pixels() != a.pixels() || b.c != a.c)
      fail(DW_ERR_UNSUPPORTED, "runtime: broadcasting elementwise op " + op.name);
    e.b = b.view();
    bytes += b.bytes();
  }
  const bool fl = a.dtype == F32 || a.dtype == F16;
  auto need_dt = [&](const RtTensor& t, int dt) {
    if (t.dtype != dt) fail(DW_ERR_RUNTIME, "runtime: " + op.type + " " + op.name + ": operand element type");
  };
  if (op.type == "Relu" && a.dtype == I8) {
    need_dt(y, I8);
    e.op = EW_RELU_I8;  // relu_i8 (ops.rs:3301-3320)
  } else if (op.type == "Requantize") {  // requantize_i32_to_i8 (ops.rs:3380-3386)
    need_dt(a, I32);
    need_dt(y, I8);
    e.op = EW_REQUANT_I32_I8;
    e.s0 = op.p.scale;
  } else if (op.type == "AddQuantized") {  // add_i8 (ops.rs:3176-3209)
    need_dt(a, I8);
    need_dt(T(op.in[1]), I8);
    need_dt(y, I8);
    e.op = EW_ADD_I8;
    e.s0 = op.p.scale_a_over_out;
    e.s1 = op.p.scale_b_over_out;
  } else if (op.type == "Quantize") {  // quantize_f32_to_i8 (ops.rs:3503-3516): x * (1 / scale)
    need_dt(a, F32);
    need_dt(y, I8);
    e.op = EW_QUANT_F32_I8;
    e.s0 = 1.0f / op.p.scale;
  } else if (op.type == "Dequantize") {  // dequantize_i8_to_f32 (ops.rs:3439-3457)
    need_dt(a, I8);
    need_dt(y, F32);
    e.op = EW_DEQUANT_I8_F32;
    e.s0 = op.p.scale;
  } else if (op.type == "Clip") {
    if (!fl) fail(DW_ERR_UNSUPPORTED, "runtime: Clip needs f32 or f16");
    need_dt(y, a.dtype);
    e.op = EW_CLIP;
    e.s0 = op.p.clip_min;
    e.s1 = op.p.clip_max;
  } else if (!fl && (op.type == "Relu" || op.type == "Sigmoid" || op.type == "Mul" || op.type == "Add" ||
                     op.type == "SiLU")) {
    fail(DW_ERR_UNSUPPORTED, "runtime: " + op.type + " " + op.name + " needs f32 or f16 operands");
  } else if (op.type == "Relu") e.op = EW_RELU;
  else if (op.type == "Sigmoid") e.op = EW_SIGMOID;
  else if (op.type == "Mul") e.op = EW_MUL;
  else if (op.type == "Add") e.op = EW_ADD;
  else if (op.type == "SiLU") e.op = EW_SILU;
  else if (op.type == "QLinearAdd") {
    RtTensor& b = T(op.in[1]);
    e.op = EW_QADD_U8;
    e.s0 = a.scale / y.scale; e.s1 = b.scale / y.scale;
    e.z0 = a.zp; e.z1 = b.zp; e.z2 = y.zp;
  } else if (op.type == "QLinearLUT") {
    e.op = EW_LUT_U8;
    uint8_t lut[256];
    build_silu_lut(lut, a.scale, a.zp, y.scale, y.zp);
    e.lut = (const uint8_t*)upload(lut, 256);
  } else if (op.type == "QuantizeLinear") {
    e.op = EW_QUANT_LINEAR_F16_U8;
    e.s0 = y.scale; e.z0 = y.zp;
  } else if (op.type == "DequantizeLinear") {
    e.op = EW_DEQUANT_LINEAR_U8_F16;
    e.s0 = a.scale; e.z0 = a.zp;
  } else {
    fail(DW_ERR_UNSUPPORTED, "runtime: elementwise " + op.type);
  }
  Launch L;
  L.kernel = "elementwise";
  L.op = op.name;
  L.bytes = bytes;
  L.fn = [=](hipStream_t st) { launch_elementwise2d(st, e); };
  launches.push_back(L);
}

void Runtime::emit_conv(const Group& gr) {
  const OpNode& op = g.ops[gr.conv];
  const TensorInfo& W = g.t[op.in[1]];
  if (W.dims.size() != 4) fail(DW_ERR_UNSUPPORTED, "runtime: conv weight must be HWIO 4-D (run convert_nchw_to_nhwc)");
  RtTensor& x = T(gr.in);
  RtTensor& y = T(gr.out);
  const int kh = (int)W.dims[0], kw = (int)W.dims[1], ci = (int)W.dims[2], co = (int)W.dims[3];
  if (ci != x.c || co != y.c) fail(DW_ERR_RUNTIME, "runtime: conv " + op.name + " channel mismatch");
  const bool has_bias = op.in.size() > 2 && !op.in[2].empty();
  const int pt = op.p.pads[0], pl = op.p.pads[1];
  const int sh = std::max(1, op.p.strides[0]), sw = std::max(1, op.p.strides[1]);
  const double macs = (double)y.pixels() * co * kh * kw * ci;
  Launch L;
  L.op = join_names(g, gr.ops);
  L.work = 2.0 * macs;

  const bool mfma = g.dtype == DW_GRAPH_F16 && gr.in_kind == 1 && gr.out_kind == 1 && (ci * 2) % 16 == 0 &&
                    co % 4 == 0 && kh * kw <= 31 && (x.pix_stride * 2) % 16 == 0 && (x.abs_off * 2) % 16 == 0 &&
                    (y.pix_stride % 4) == 0 && (y.abs_off % 4) == 0;
  if (mfma) {
    IgemmArgs a{};
    a.x = (const uint8_t*)x.base;
    a.y = y.base;
    a.n = (int)x.n; a.h = (int)x.h; a.w = (int)x.w; a.cin = ci; a.cout = co; a.kh = kh; a.kw = kw;
    a.sh = sh; a.sw = sw; a.pt = pt; a.pl = pl; a.ho = (int)y.h; a.wo = (int)y.w;
    a.m = (int)y.pixels();
    a.ksteps = (kh * kw * ci * 2 + 63) / 64;
    const int bc = igemm_channel_tile(co);
    a.cout_pad = (co + bc - 1) / bc * bc;
    a.x_pix_stride = x.pix_stride; a.x_c_off = x.abs_off;
    a.y_pix_stride = y.pix_stride; a.y_c_off = y.abs_off;
    void* whwio = upload(W.data.data(), W.data.size());
    void* wpk = dalloc((size_t)a.ksteps * a.cout_pad * 64);
    launch_pack_weights(be->stream, whwio, wpk, kh * kw * ci, co, a.cout_pad, a.ksteps, 2);
    a.wpk = (const uint8_t*)wpk;
    a.epi = EPI_F16;
    a.act = gr.act;
    if (has_bias) a.bias_h = (const uint16_t*)upload(g.t[op.in[2]].data.data(), g.t[op.in[2]].data.size());
    if (!gr.res.empty()) {
      RtTensor& r = T(gr.res);
      if (r.pix_stride % 4 != 0 || r.abs_off % 4 != 0)
        fail(DW_ERR_RUNTIME, "runtime: misaligned residual view for " + op.name);
      a.res = r.base;
      a.r_pix_stride = r.pix_stride;
      a.r_c_off = r.abs_off;
      L.bytes += r.bytes();
    }
    L.bytes += (double)x.bytes() + W.data.size() + y.pixels() * co * 2.0;
    L.t_in = gr.in;
    L.t_out = gr.out;
    DW_HIP(hipStreamSynchronize(be->stream));
    push_igemm(L, a, 2);
    return;
  }
  // the fp16 graphs' three-channel stem (all of K in one fp16 k-step) on
  // the fp16 matrix cores, held to the fp16 tolerance like the other MFMA
  // convs of those graphs
  const bool stem_mfma = g.dtype == DW_GRAPH_F16 && gr.in_kind == 1 && gr.out_kind == 1 && gr.res.empty() &&
                         stem_f16_supported(ci, kh, kw, co, (int)y.w, sh, sw) && op.p.group <= 1 && op.p.dilations[0] <= 1 &&
                         op.p.dilations[1] <= 1 && W.dtype == DW_DTYPE_F16 &&
                         (!has_bias || g.t[op.in[2]].dtype == DW_DTYPE_F16) && y.pix_stride % 4 == 0 &&
                         y.abs_off % 4 == 0;
  if (stem_mfma) {
    // fragment order [cb][lane][j] = W[k = 8 (lane / 16) + j][c = 16 cb + lane % 16],
    // zero past K (the HWIO weights flattened over kh, kw, c_in)
    const int K = kh * kw * ci;
    std::vector<uint16_t> frag((size_t)(co / 16) * 64 * 8, 0);
    for (int cb = 0; cb < co / 16; ++cb)
      for (int l = 0; l < 64; ++l)
        for (int j = 0; j < 8; ++j) {
          const int k = 8 * (l / 16) + j, c = 16 * cb + l % 16;
          if (k < K) frag[((size_t)cb * 64 + l) * 8 + j] = ((const uint16_t*)W.data.data())[(size_t)k * co + c];
        }
    StemF16Args a{};
    a.x = (const uint16_t*)x.base;
    a.in_kind = 1;
    a.wfrag = (const uint16_t*)upload(frag.data(), frag.size() * 2);
    a.bias = has_bias ? (const uint16_t*)upload(g.t[op.in[2]].data.data(), g.t[op.in[2]].data.size()) : nullptr;
    a.y = (uint16_t*)y.base;
    a.n = (int)x.n; a.h = (int)x.h; a.w = (int)x.w; a.cin = ci; a.ho = (int)y.h; a.wo = (int)y.w;
    a.kh = kh; a.kw = kw; a.sh = sh; a.sw = sw; a.pt = pt; a.pl = pl; a.cout = co;
    a.m = (int)y.pixels();
    a.x_pix_stride = x.pix_stride; a.x_c_off = x.abs_off;
    a.y_pix_stride = y.pix_stride; a.y_c_off = y.abs_off;
    a.act = gr.act;
    L.kernel = "stem_f16_mfma";
    L.bytes += (double)x.bytes() + frag.size() * 2.0 + (double)y.bytes();
    L.sa = std::make_shared<StemF16Args>(a);
    L.fn = [sa = L.sa](hipStream_t st) { launch_stem_f16(st, *sa); };
    launches.push_back(L);
    return;
  }
  // u8 -> f16 1x1 on the fp16 matrix cores (the dequantized fp16 layers of a
  // quantized graph), held to the fp16 tolerance like the other MFMA convs
  const bool head_mfma = !exact_u8_f16 && gr.in_kind == 2 && gr.out_kind == 1 && gr.res.empty() && kh == 1 &&
                         kw == 1 && sh == 1 && sw == 1 && pt == 0 && pl == 0 && op.p.pads[2] == 0 &&
                         op.p.pads[3] == 0 && conv1x1_u8_f16_supported(ci, co) && x.pix_stride % 8 == 0 &&
                         x.abs_off % 8 == 0 && y.pix_stride % 4 == 0 && y.abs_off % 4 == 0 &&
                         (W.dtype == DW_DTYPE_F16 || W.dtype == DW_DTYPE_F32) &&
                         (!has_bias || g.t[op.in[2]].dtype == DW_DTYPE_F16);
  if (head_mfma) {
    // weights widened as the reference does (subnormals at half value) and
    // re-encoded to f16, in fragment order: [cb][ks][lane][j] =
    // W[k = 32 ks + 8 (lane / 16) + j][c = 16 cb + lane % 16], zero past K or c_out
    const int cbn = (co + 15) / 16, ksn = (ci + 31) / 32;
    std::vector<uint16_t> frag((size_t)cbn * ksn * 64 * 8, 0);
    for (int cb = 0; cb < cbn; ++cb)
      for (int ks = 0; ks < ksn; ++ks)
        for (int l = 0; l < 64; ++l)
          for (int j = 0; j < 8; ++j) {
            const int k = 32 * ks + 8 * (l / 16) + j, c = 16 * cb + l % 16;
            if (k >= ci || c >= co) continue;
            const size_t src = (size_t)k * co + c;
            const float v = W.dtype == DW_DTYPE_F16 ? f16_to_f32_ref(((const uint16_t*)W.data.data())[src])
                                                    : ((const float*)W.data.data())[src];
            frag[(((size_t)cb * ksn + ks) * 64 + l) * 8 + j] = f16_bits_from_f32(v);
          }
    Conv1x1F16Args a{};
    a.x = (const uint8_t*)x.base;
    a.wfrag = (const uint16_t*)upload(frag.data(), frag.size() * 2);
    a.bias = has_bias ? (const uint16_t*)upload(g.t[op.in[2]].data.data(), g.t[op.in[2]].data.size()) : nullptr;
    a.y = (uint16_t*)y.base;
    a.m = (int)y.pixels();
    a.cin = ci;
    a.cout = co;
    a.x_pix_stride = x.pix_stride; a.x_c_off = x.abs_off;
    a.y_pix_stride = y.pix_stride; a.y_c_off = y.abs_off;
    a.in_scale = gr.in_scale;
    a.in_zp = gr.in_zp;
    a.zp_bytes = (uint32_t)(gr.in_zp & 0xff) * 0x01010101u;
    a.act = gr.act;
    L.kernel = "conv1x1_u8_f16";
    L.bytes += (double)x.bytes() + frag.size() * 2.0 + (double)y.bytes();
    L.fn = [a](hipStream_t st) { launch_conv1x1_u8_f16(st, a); };
    L.c1a = std::make_shared<Conv1x1F16Args>(a);
    L.t_in = gr.in;
    L.t_out = gr.out;
    launches.push_back(L);
    return;
  }
  // direct (reference accumulation order)
  DirectArgs a{};
  a.x = x.base;
  a.y = y.base;
  a.n = (int)x.n; a.h = (int)x.h; a.w = (int)x.w; a.cin = ci; a.cout = co; a.kh = kh; a.kw = kw;
  a.sh = sh; a.sw = sw; a.pt = pt; a.pl = pl; a.ho = (int)y.h; a.wo = (int)y.w;
  a.m = (int)y.pixels();
  a.x_pix_stride = x.pix_stride; a.x_c_off = x.abs_off;
  a.y_pix_stride = y.pix_stride; a.y_c_off = y.abs_off;
  a.in_kind = gr.in_kind;
  a.in_scale = gr.in_scale;
  a.in_zp = gr.in_zp;
  a.out_kind = gr.out_kind;
  a.act = gr.act;
  // weights as f32 (exact widening of f16 weights with the reference decode)
  std::vector<float> wf(W.numel());
  if (W.dtype == DW_DTYPE_F32) {
    memcpy(wf.data(), W.data.data(), wf.size() * 4);
  } else if (W.dtype == DW_DTYPE_F16) {
    void* wh = upload(W.data.data(), W.data.size());
    float* wdev = (float*)dalloc(wf.size() * 4);
    EwArgs e{};
    e.op = EW_F16_TO_F32; e.a = wh; e.y = wdev; e.count = wf.size();
    launch_elementwise(be->stream, e);
    DW_HIP(hipStreamSynchronize(be->stream));
    a.wf = wdev;
  } else {
    fail(DW_ERR_UNSUPPORTED, "runtime: conv weight dtype");
  }
  if (!a.wf) a.wf = (const float*)upload(wf.data(), wf.size() * 4);
  {
    bool fin = true;
    if (W.dtype == DW_DTYPE_F32)
      for (size_t i = 0; i < wf.size() && fin; ++i) fin = std::isfinite(wf[i]);
    else
      for (size_t i = 0; i < W.numel() && fin; ++i) fin = (((const uint16_t*)W.data.data())[i] & 0x7c00) != 0x7c00;
    a.w_finite = fin ? 1 : 0;
  }
  if (kh == 1 && kw == 1 && co % 16 == 0 && (W.dtype == DW_DTYPE_F32 || W.dtype == DW_DTYPE_F16)) {
    // the 1x1 kernel's layout: [co / 16][ci][16] (each 16-channel group's
    // weight rows contiguous)
    std::vector<float> w(W.numel());
    if (W.dtype == DW_DTYPE_F32)
      memcpy(w.data(), W.data.data(), w.size() * 4);
    else
      for (size_t i = 0; i < w.size(); ++i) w[i] = f16_to_f32_ref(((const uint16_t*)W.data.data())[i]);
    std::vector<float> wq(w.size());
    for (int g16 = 0; g16 < co / 16; ++g16)
      for (int r = 0; r < ci; ++r)
        for (int j = 0; j < 16; ++j) wq[((size_t)g16 * ci + r) * 16 + j] = w[(size_t)r * co + 16 * g16 + j];
    a.wq16 = (const float*)upload(wq.data(), wq.size() * 4);
  }
  if (a.in_kind == 0 && W.dtype == DW_DTYPE_F32 && ci % 16 == 0 && co % 4 == 0) {
    // the tiled kernel's layout: [co / 4][kh * kw * ci][4]
    const size_t rows = (size_t)kh * kw * ci;
    std::vector<float> wq(wf.size());
    for (int g4 = 0; g4 < co / 4; ++g4)
      for (size_t r = 0; r < rows; ++r)
        for (int j = 0; j < 4; ++j) wq[((size_t)g4 * rows + r) * 4 + j] = wf[r * co + 4 * g4 + j];
    a.wq = (const float*)upload(wq.data(), wq.size() * 4);
  }
  if (has_bias) {
    const TensorInfo& B = g.t[op.in[2]];
    if (gr.out_kind == 0) {
      a.bias_f = (const float*)upload(B.data.data(), B.data.size());
    } else {
      a.bias_h = (const uint16_t*)upload(B.data.data(), B.data.size());
      if (B.dtype == DW_DTYPE_F16) {  // widen once here, as every f16 operand is widened
        std::vector<float> bf(B.data.size() / 2);
        for (size_t i = 0; i < bf.size(); ++i) bf[i] = f16_to_f32_ref(((const uint16_t*)B.data.data())[i]);
        a.bias_hf = (const float*)upload(bf.data(), bf.size() * 4);
      }
    }
  }
  if (gr.out_kind == 2) {
    const RtTensor& q = T(gr.lut ? gr.pre : gr.out);
    a.out_scale = q.scale;
    a.out_zp = q.zp;
    a.out_rcp = 1.0f / q.scale;
    a.out_fast = fast_quant_ok(q.scale, a.out_rcp) ? 1 : 0;
    if (gr.lut) {
      uint8_t lut[256];
      build_silu_lut(lut, q.scale, q.zp, y.scale, y.zp);
      a.lut = (const uint8_t*)upload(lut, 256);
    }
  }
  if (gr.out_kind != 0) a.fast_epi = fast_epi_ok(g, op, has_bias, gr.out_kind, a) ? 1 : 0;
  if (gr.out_kind == 1) a.epi_pk = bias_plain_f16(g, op, has_bias) ? 1 : 0;
  if (gr.out_kind == 2 && a.out_fast && a.out_scale >= 1.220703125e-04f) {
    a.epi_pk = bias_plain_f16(g, op, has_bias) ? 1 : 0;
    a.out_plain = plain_quant_ok(a.out_scale, a.out_rcp) ? 1 : 0;
    // test override: the quotient with the FMA correction everywhere
    if (const char* e = getenv("DW_QUANT_CORRECTED"))
      if (atoi(e) != 0) a.out_plain = 0;
  }
  L.kernel = stem_pad_ok(a) ? "stem_pad_u8" : "direct_conv";
  L.bytes += (double)x.bytes() + W.numel() * 4.0 + (double)y.bytes();
  L.da = std::make_shared<DirectArgs>(a);
  L.fn = [da = L.da](hipStream_t st) { launch_direct_conv(st, *da); };
  launches.push_back(L);
}

void Runtime::emit_qconv(const Group& gr) {
  const OpNode& op = g.ops[gr.conv];
  const TensorInfo& W = g.t[op.in[1]];
  RtTensor& x = T(gr.in);
  RtTensor& pre = T(gr.pre);
  RtTensor& y = T(gr.out);
  const int kh = (int)W.dims[0], kw = (int)W.dims[1], ci = (int)W.dims[2], co = (int)W.dims[3];
  if (x.dtype != U8 || y.dtype != U8) fail(DW_ERR_RUNTIME, "runtime: QLinearConv needs u8 tensors");
  if (ci % 16 != 0 || co % 4 != 0 || kh * kw > 31)
    fail(DW_ERR_UNSUPPORTED, "runtime: QLinearConv needs c_in % 16 == 0, c_out % 4 == 0 and at most 31 taps (" +
                                 op.name + ")");
  if (x.pix_stride % 16 != 0 || x.abs_off % 16 != 0 || y.pix_stride % 4 != 0 || y.abs_off % 4 != 0)
    fail(DW_ERR_RUNTIME, "runtime: misaligned view for " + op.name);
  IgemmArgs a{};
  a.x = (const uint8_t*)x.base;
  a.y = y.base;
  a.n = (int)x.n; a.h = (int)x.h; a.w = (int)x.w; a.cin = ci; a.cout = co; a.kh = kh; a.kw = kw;
  a.sh = std::max(1, op.p.strides[0]); a.sw = std::max(1, op.p.strides[1]);
  a.pt = op.p.pads[0]; a.pl = op.p.pads[1]; a.ho = (int)y.h; a.wo = (int)y.w;
  a.m = (int)y.pixels();
  a.ksteps = (kh * kw * ci + 63) / 64;
  const int bc = igemm_channel_tile(co);
  a.cout_pad = (co + bc - 1) / bc * bc;
  a.x_pix_stride = x.pix_stride; a.x_c_off = x.abs_off;
  a.y_pix_stride = y.pix_stride; a.y_c_off = y.abs_off;
  // weights, bias' = bias + (128 - x_zp) * sum_k w, M[c] = xs*ws[c]/ys
  void* whwio = upload(W.data.data(), W.data.size());
  void* wpk = dalloc((size_t)a.ksteps * a.cout_pad * 64);
  launch_pack_weights(be->stream, whwio, wpk, kh * kw * ci, co, a.cout_pad, a.ksteps, 1);
  std::vector<int64_t> bias(co, 0);
  if (op.in.size() > 2 && !op.in[2].empty()) {
    const TensorInfo& B = g.t[op.in[2]];
    if (B.dtype != DW_DTYPE_I32) fail(DW_ERR_RUNTIME, "runtime: QLinearConv bias must be int32");
    for (int c = 0; c < co; ++c) bias[c] = ((const int32_t*)B.data.data())[c];
  }
  std::vector<int32_t> bi(co);
  std::vector<float> ms(co);
  const int8_t* wq = (const int8_t*)W.data.data();
  for (int c = 0; c < co; ++c) {
    int64_t s = 0;
    for (int k = 0; k < kh * kw * ci; ++k) s += wq[(size_t)k * co + c];
    const int64_t v = bias[c] + (int64_t)(128 - x.zp) * s;
    if (v < INT32_MIN || v > INT32_MAX) fail(DW_ERR_RUNTIME, "runtime: bias overflow in " + op.name);
    bi[c] = (int32_t)v;
    if (W.ch_scales.size() != (size_t)co) fail(DW_ERR_RUNTIME, "runtime: missing weight scales");
    ms[c] = (x.scale * W.ch_scales[c]) / pre.scale;
  }
  a.wpk = (const uint8_t*)wpk;
  a.bias_i = (const int*)upload(bi.data(), bi.size() * 4);
  a.mscale = (const float*)upload(ms.data(), ms.size() * 4);
  a.epi = EPI_QU8;
  a.xxor = 0x80808080u;
  a.xpad = (uint32_t)((x.zp ^ 0x80) & 0xff) * 0x01010101u;
  a.y_zp = pre.zp;
  Launch L;
  L.op = join_names(g, gr.ops);
  L.work = 2.0 * (double)y.pixels() * co * kh * kw * ci;
  L.bytes = (double)x.bytes() + W.data.size() + (double)y.pixels() * co;
  uint8_t lut[256];
  if (gr.lut) {
    const RtTensor& lo = T(gr.lut_out);
    build_silu_lut(lut, pre.scale, pre.zp, lo.scale, lo.zp);
    a.lut = (const uint8_t*)upload(lut, 256);
  }
  if (!gr.res.empty()) {
    RtTensor& r = T(gr.res);
    const RtTensor& av = T(gr.lut ? gr.lut_out : gr.pre);
    if (r.pix_stride % 4 != 0 || r.abs_off % 4 != 0)
      fail(DW_ERR_RUNTIME, "runtime: misaligned residual view for " + op.name);
    a.res = r.base;
    a.r_pix_stride = r.pix_stride;
    a.r_c_off = r.abs_off;
    a.ra = av.scale / y.scale;
    a.rb = r.scale / y.scale;
    a.za = av.zp;
    a.zb = r.zp;
    a.zy = y.zp;
    L.bytes += r.bytes();
    // the QLinearAdd's rounded products as tables (the kernels that take
    // them add two entries instead of converting and multiplying): the same
    // f32 products qadd_u8 forms, kept when every sum of two entries stays
    // below 2^21 in magnitude; DW_QADD_TABLES=0 keeps qadd_u8
    const char* qt = getenv("DW_QADD_TABLES");
    if (gr.lut && !(qt && qt[0] == '0')) {
      float rt[512];
      float ma = 0.0f, mb = 0.0f;
      for (int q = 0; q < 256; ++q) {
        rt[q] = (float)((int)lut[q] - a.za) * a.ra;
        rt[256 + q] = (float)(q - a.zb) * a.rb;
        ma = std::max(ma, std::fabs(rt[q]));
        mb = std::max(mb, std::fabs(rt[256 + q]));
      }
      if (std::isfinite(ma) && std::isfinite(mb) && ma + mb < 2097152.0f)
        a.rtab = (const float*)upload(rt, sizeof rt);
    }
  }
  DW_HIP(hipStreamSynchronize(be->stream));
  L.t_in = gr.in;
  L.t_out = gr.out;
  push_igemm(L, a, 1);
}

namespace {
// Whether the first op name of a launch (its op string up to the first '+')
// is in a comma-separated list.
bool listed(const char* csv, const std::string& ops) {
  const std::string first = ops.substr(0, ops.find('+'));
  std::string list = std::string(",") + csv + ",";
  return list.find("," + first + ",") != std::string::npos;
}
}  // namespace

// Chained QLinearConv pairs in one launch (igemm_pair.h): a 3x3 conv whose
// output only the next launch's 3x3 conv reads (the bottleneck of a C2f
// block, c = 16, 32 or 64 channels) may run with it, the intermediate kept
// in LDS.  The outputs are those of the two launches.  After the tile
// tuner, each candidate pair is timed at every valid band height, as the
// tuner times a tile, and kept (at its fastest height) only if it beats the
// two tuned launches.  DW_PAIR=1 keeps every candidate pair, DW_PAIR=0
// none; untuned plans (DW_AUTOTUNE=0, DW_IGEMM_TILE) keep none unless
// DW_PAIR=1, which then takes the tallest band that leaves two workgroups
// a CU their LDS (or the tallest).  Each height is timed in both
// workgroup forms (4 waves, and 16 waves with smaller register chunks).
// DW_PAIR_ROWS=<r> forces band height r wherever it is valid (tests),
// DW_PAIR_WAVES=4|16 forces the form; DW_PAIR_KEEP=<op,op,..> keeps exactly
// the pairs whose first conv is listed (another process reproducing a plan).
void Runtime::fuse_pairs() {
  const char* env = getenv("DW_PAIR");
  if (env && env[0] == '0') return;
  const char* keep = getenv("DW_PAIR_KEEP");
  const bool force = (env && env[0] == '1') || keep;
  const char* tune_env = getenv("DW_AUTOTUNE");
  const bool tuned = !((tune_env && tune_env[0] == '0') || getenv("DW_IGEMM_TILE"));
  if (!force && !tuned) return;
  auto readers = [&](const std::string& t) {
    int k = 0;
    for (auto& op : g.ops)
      for (auto& i : op.in) k += i == t;
    return k;
  };
  FILE* log = nullptr;
  if (const char* lp = getenv("DW_AUTOTUNE_LOG")) log = fopen(lp, "a");
  hipStream_t st = be->stream;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  DW_HIP(hipEventCreate(&e0));
  DW_HIP(hipEventCreate(&e1));
  auto time4 = [&](const IgemmArgs& a1, const IgemmArgs& a2, int rows, int waves) {
    launch_igemm_pair(st, a1, a2, rows, waves);
    float t_min = 1e30f;
    for (int r = 0; r < 3; ++r) {
      DW_HIP(hipEventRecord(e0, st));
      for (int k = 0; k < 4; ++k) launch_igemm_pair(st, a1, a2, rows, waves);
      DW_HIP(hipEventRecord(e1, st));
      DW_HIP(hipEventSynchronize(e1));
      float ms = 0;
      DW_HIP(hipEventElapsedTime(&ms, e0, e1));
      t_min = std::min(t_min, ms);
    }
    return t_min;
  };
  for (size_t i = 0; i + 1 < launches.size(); ++i) {
    Launch& L1 = launches[i];
    Launch& L2 = launches[i + 1];
    if (!L1.ig || !L2.ig || L1.esize != 1 || L2.esize != 1 || L1.t_out.empty() || L2.t_in != L1.t_out) continue;
    if (readers(L1.t_out) != 1 || std::find(g.outputs.begin(), g.outputs.end(), L1.t_out) != g.outputs.end())
      continue;
    if (keep && !listed(keep, L1.op)) continue;
    int cand[16];
    const int nc = igemm_pair_rows(*L1.ig, *L2.ig, cand, 16);
    if (nc == 0) continue;
    int rows = cand[0], waves = 4;
    if (tuned) {
      if (L1.tuned_ms <= 0 || L2.tuned_ms <= 0) continue;
      float best = 1e30f;
      for (int k = 0; k < nc; ++k)
        for (int wv : {4, 16}) {
          const float t = time4(*L1.ig, *L2.ig, cand[k], wv);
          if (log)
            fprintf(log, "%s\tigemm_i8_pair_c%d_r%d_w%d\t%.2f\n", L1.op.c_str(), L1.ig->cin, cand[k], wv, t * 1e3f / 4);
          if (t < best) {
            best = t;
            rows = cand[k];
            waves = wv;
          }
        }
      if (log) fprintf(log, "%s\ttwo launches\t%.2f\n", L1.op.c_str(), (L1.tuned_ms + L2.tuned_ms) * 1e3f / 4);
      if (!force && best >= L1.tuned_ms + L2.tuned_ms) continue;
    } else {
      for (int k = 0; k < nc; ++k)
        if (igemm_pair_lds_two_per_cu(*L1.ig, cand[k])) {
          rows = cand[k];
          break;
        }
    }
    if (const char* fr = getenv("DW_PAIR_ROWS")) {
      const int r = atoi(fr);
      if (igemm_pair_ok(*L1.ig, *L2.ig, r)) rows = r;
    }
    Launch P;
    if (const char* fw = getenv("DW_PAIR_WAVES")) waves = atoi(fw) == 16 ? 16 : 4;
    P.kernel = "igemm_i8_pair_c" + std::to_string(L1.ig->cin) + (waves == 16 ? "_w16" : "");
    P.op = L1.op + "+" + L2.op;
    P.work = L1.work + L2.work;
    // the intermediate neither written nor read back
    P.bytes = L1.bytes + L2.bytes - 2.0 * (double)T(L1.t_out).pixels() * T(L1.t_out).c;
    auto a1 = L1.ig, a2 = L2.ig;
    P.fn = [a1, a2, rows, waves](hipStream_t s) { launch_igemm_pair(s, *a1, *a2, rows, waves); };
    P.esize = 1;
    P.group = L1.group;
    P.reads = L1.reads;
    P.reads.insert(P.reads.end(), L2.reads.begin(), L2.reads.end());
    P.writes = L1.writes;
    P.writes.insert(P.writes.end(), L2.writes.begin(), L2.writes.end());
    P.t_in = L1.t_in;
    P.t_out = L2.t_out;
    launches[i] = P;
    launches.erase(launches.begin() + (long)i + 1);
  }
  if (log) fclose(log);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
}

// Sibling convs in one launch: two convs that read the same input tensor
// with the same geometry, each with the u8 table epilogue (QLinearConv) or
// the same f16 epilogue (fp16 Conv) and no residual (the box0 and cls0 convs
// of a detect scale), as one GEMM over both channel sets: the second conv's
// channels after the first's (packed weights, bias' and multipliers
// concatenated on the device), each channel tile writing its own conv's
// output view (u8: with its own table).  Every output is computed as
// its own conv computes it, so the bytes are the two launches'.  Both orders
// and every staged, streamed-weight and band tile whose channel tiles do not
// straddle the first conv's channels are timed; the fastest is kept if it
// beats the two tuned launches.  DW_SIB=0 fuses none, =1 every candidate;
// DW_SIB_KEEP=<op,op,..> keeps exactly the pairs whose first conv is listed.
void Runtime::fuse_siblings() {
  const char* env = getenv("DW_SIB");
  if (env && env[0] == '0') return;
  const char* keep = getenv("DW_SIB_KEEP");
  const bool force = (env && env[0] == '1') || keep;
  const char* tune_env = getenv("DW_AUTOTUNE");
  const bool tuned = !((tune_env && tune_env[0] == '0') || getenv("DW_IGEMM_TILE"));
  if (!force && !tuned) return;
  FILE* log = nullptr;
  if (const char* lp = getenv("DW_AUTOTUNE_LOG")) log = fopen(lp, "a");
  hipStream_t st = be->stream;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  DW_HIP(hipEventCreate(&e0));
  DW_HIP(hipEventCreate(&e1));
  // u8: the table epilogue; fp16: the f16 epilogue with its bias (the two
  // convs' activations compared below)
  auto alone = [](const IgemmArgs& a, int esize) {
    const bool base = !a.res && !a.y_up && !a.h_wfrag && !a.y2 && a.cout % 16 == 0;
    return esize == 1 ? base && a.epi == EPI_QU8 && a.lut && a.bias_i && a.mscale
                      : base && a.epi == EPI_F16 && a.bias_h;
  };
  auto same_input = [](const IgemmArgs& a, const IgemmArgs& b) {
    return a.x == b.x && a.x_pix_stride == b.x_pix_stride && a.x_c_off == b.x_c_off && a.n == b.n && a.h == b.h &&
           a.w == b.w && a.cin == b.cin && a.kh == b.kh && a.kw == b.kw && a.sh == b.sh && a.sw == b.sw &&
           a.pt == b.pt && a.pl == b.pl && a.ho == b.ho && a.wo == b.wo && a.ksteps == b.ksteps &&
           a.xpad == b.xpad && a.xxor == b.xxor && a.y_zp == b.y_zp;
  };
  auto time4 = [&](const IgemmArgs& a, int esize) {
    launch_igemm(st, a, esize);
    float t_min = 1e30f;
    for (int r = 0; r < 3; ++r) {
      DW_HIP(hipEventRecord(e0, st));
      for (int k = 0; k < 4; ++k) launch_igemm(st, a, esize);
      DW_HIP(hipEventRecord(e1, st));
      DW_HIP(hipEventSynchronize(e1));
      float ms = 0;
      DW_HIP(hipEventElapsedTime(&ms, e0, e1));
      t_min = std::min(t_min, ms);
    }
    return t_min;
  };
  // F's channels, then S's, at channel tile width bc: the combined
  // arguments (packed weights zero-padded to a whole tile)
  auto combine = [&](const IgemmArgs& F, const IgemmArgs& S, int bc, int esize) {
    IgemmArgs C = F;
    C.cout = F.cout + S.cout;
    C.split = F.cout;
    C.cout_pad = (C.cout + bc - 1) / bc * bc;
    const size_t row = 64, ks = (size_t)F.ksteps;
    uint8_t* wpk = (uint8_t*)dalloc(ks * C.cout_pad * row);
    DW_HIP(hipMemsetAsync(wpk, 0, ks * C.cout_pad * row, st));
    DW_HIP(hipMemcpy2DAsync(wpk, C.cout_pad * row, F.wpk, F.cout_pad * row, F.cout * row, ks,
                            hipMemcpyDeviceToDevice, st));
    DW_HIP(hipMemcpy2DAsync(wpk + F.cout * row, C.cout_pad * row, S.wpk, S.cout_pad * row, S.cout * row, ks,
                            hipMemcpyDeviceToDevice, st));
    if (esize == 1) {
      int* bias = (int*)dalloc(C.cout_pad * sizeof(int));
      float* ms = (float*)dalloc(C.cout_pad * sizeof(float));
      DW_HIP(hipMemcpyAsync(bias, F.bias_i, F.cout * sizeof(int), hipMemcpyDeviceToDevice, st));
      DW_HIP(hipMemcpyAsync(bias + F.cout, S.bias_i, S.cout * sizeof(int), hipMemcpyDeviceToDevice, st));
      DW_HIP(hipMemcpyAsync(ms, F.mscale, F.cout * sizeof(float), hipMemcpyDeviceToDevice, st));
      DW_HIP(hipMemcpyAsync(ms + F.cout, S.mscale, S.cout * sizeof(float), hipMemcpyDeviceToDevice, st));
      C.bias_i = bias;
      C.mscale = ms;
    } else {
      uint16_t* bh = (uint16_t*)dalloc(C.cout_pad * sizeof(uint16_t));
      DW_HIP(hipMemcpyAsync(bh, F.bias_h, F.cout * sizeof(uint16_t), hipMemcpyDeviceToDevice, st));
      DW_HIP(hipMemcpyAsync(bh + F.cout, S.bias_h, S.cout * sizeof(uint16_t), hipMemcpyDeviceToDevice, st));
      C.bias_h = bh;
    }
    DW_HIP(hipStreamSynchronize(st));
    C.wpk = wpk;
    C.y2 = S.y;
    C.y2_pix_stride = S.y_pix_stride;
    C.y2_c_off = S.y_c_off;
    C.lut2 = S.lut;
    C.tile_bc = C.tile_pb = C.tile_tpw = 0;
    return C;
  };
  for (size_t i = 0; i < launches.size(); ++i) {
    for (size_t j = i + 1; j < launches.size(); ++j) {
      Launch& LA = launches[i];
      Launch& LB = launches[j];
      const int es = LA.esize;
      if (!LA.ig || !LB.ig || (es != 1 && es != 2) || LB.esize != es) continue;
      const IgemmArgs A = *LA.ig, B = *LB.ig;
      // the same input tensor (not only the same bytes: activations that
      // are never live together share arena bytes)
      if (LA.t_in.empty() || LA.t_in != LB.t_in) continue;
      if (!alone(A, es) || !alone(B, es) || !same_input(A, B) || A.act != B.act) continue;
      if (!tuned && !force) continue;
      if (tuned && (LA.tuned_ms <= 0 || LB.tuned_ms <= 0)) continue;
      float best = 1e30f;
      IgemmArgs bestC{};
      bool first_a = true;
      for (int order = 0; order < 2; ++order) {
        const IgemmArgs& F = order == 0 ? A : B;
        const IgemmArgs& S = order == 0 ? B : A;
        const Launch& LF = order == 0 ? LA : LB;
        if (keep && !listed(keep, LF.op)) continue;
        for (int bw : {128, 96, 80, 64, 48, 32, 16}) {
          if (F.cout % bw != 0) continue;
          IgemmArgs C = combine(F, S, bw, es);
          int bc[64], pb[64], tpw[64];
          const int n = igemm_candidates(C, bc, pb, tpw, 64);
          for (int k = 0; k < n; ++k) {
            if (bc[k] != bw || !igemm_sibling_tile_ok(C, bc[k], tpw[k], es)) continue;
            C.tile_bc = bc[k];
            C.tile_pb = pb[k];
            C.tile_tpw = tpw[k];
            const float t = tuned ? time4(C, es) : 0.0f;
            if (log)
              fprintf(log, "%s+%s\t%s\t%.2f\n", LF.op.c_str(), (order == 0 ? LB : LA).op.c_str(),
                      igemm_tile_name(C, es), t * 1e3f / 4);
            if (t < best) {
              best = t;
              bestC = C;
              first_a = order == 0;
            }
          }
        }
      }
      if (best >= 1e30f) continue;
      if (log) fprintf(log, "%s+%s\ttwo launches\t%.2f\n", LA.op.c_str(), LB.op.c_str(),
                       (LA.tuned_ms + LB.tuned_ms) * 1e3f / 4);
      if (!force && best >= LA.tuned_ms + LB.tuned_ms) continue;
      const Launch& LF = first_a ? LA : LB;
      const Launch& LS = first_a ? LB : LA;
      Launch P;
      P.ig = std::make_shared<IgemmArgs>(bestC);
      P.kernel = igemm_tile_name(bestC, es);
      P.op = LF.op + "+" + LS.op;
      P.work = LA.work + LB.work;
      // the input read once
      P.bytes = LA.bytes + LB.bytes - (double)A.n * A.h * A.w * A.cin * es;
      auto ig = P.ig;
      P.fn = [ig, es](hipStream_t s) { launch_igemm(s, *ig, es); };
      P.esize = es;
      P.group = LA.group;
      P.reads = LA.reads;
      P.reads.insert(P.reads.end(), LB.reads.begin(), LB.reads.end());
      P.writes = LA.writes;
      P.writes.insert(P.writes.end(), LB.writes.begin(), LB.writes.end());
      P.t_in = LA.t_in;
      P.tuned_ms = best;
      if (!force) sib_undo.push_back({i, j, LA, LB});
      launches[i] = P;
      launches.erase(launches.begin() + (long)j);
      break;
    }
  }
  if (log) fclose(log);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
}

// A C2f block with one bottleneck (cv1, m.cv1, m.cv2, cv2: four
// consecutive QLinearConv launches over the block's concat buffer) in one
// launch (igemm_c2f.h), when nothing else reads or writes the storage of
// the block's intermediates (y, t, z and their concat) and none of it is a
// graph output.  Timed over its band heights against the four tuned
// launches and kept only if faster; DW_C2F=1 keeps every candidate, =0
// none; DW_C2F_KEEP=<op,op,..> keeps exactly the blocks whose cv1 is
// listed, DW_C2F_ROWS=<r> forces a band height.
void Runtime::fuse_c2f() {
  const char* env = getenv("DW_C2F");
  if (env && env[0] == '0') return;
  const char* keep = getenv("DW_C2F_KEEP");
  const bool force = (env && env[0] == '1') || keep;
  const char* tune_env = getenv("DW_AUTOTUNE");
  const bool tuned = !((tune_env && tune_env[0] == '0') || getenv("DW_IGEMM_TILE"));
  if (!force && !tuned) return;
  FILE* log = nullptr;
  if (const char* lp = getenv("DW_AUTOTUNE_LOG")) log = fopen(lp, "a");
  hipStream_t st = be->stream;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  DW_HIP(hipEventCreate(&e0));
  DW_HIP(hipEventCreate(&e1));
  for (size_t i = 0; i + 3 < launches.size(); ++i) {
    Launch* Ls[4] = {&launches[i], &launches[i + 1], &launches[i + 2], &launches[i + 3]};
    bool ok = true;
    for (Launch* L : Ls) ok = ok && L->ig && L->esize == 1;
    if (!ok || !igemm_c2f_shapes_ok(*Ls[0]->ig, *Ls[1]->ig, *Ls[2]->ig, *Ls[3]->ig)) continue;
    // the intermediates' storage roots: written by cv1, m.cv1 and m.cv2
    std::set<int> roots;
    for (int k = 0; k < 3; ++k)
      for (const Region& r : Ls[k]->writes) roots.insert(r.rid);
    for (size_t j = 0; j < launches.size() && ok; ++j) {
      if (j >= i && j < i + 4) continue;
      for (const Region& r : launches[j].reads) ok = ok && !roots.count(r.rid);
      for (const Region& r : launches[j].writes) ok = ok && !roots.count(r.rid);
    }
    for (const std::string& o : g.outputs) ok = ok && !roots.count(T(o).rid);
    if (!ok) continue;
    if (keep && !listed(keep, Ls[0]->op)) continue;
    const IgemmArgs &a0 = *Ls[0]->ig, &a1 = *Ls[1]->ig, &a2 = *Ls[2]->ig, &a3 = *Ls[3]->ig;
    int cand[16];
    const int nc = igemm_c2f_rows(a0, a1, a2, a3, cand, 16);
    if (nc == 0) continue;
    int rows = cand[0];
    if (tuned) {
      float sum = 0;
      for (Launch* L : Ls) sum += L->tuned_ms;
      float best = 1e30f;
      for (int k = 0; k < nc; ++k) {
        launch_igemm_c2f(st, a0, a1, a2, a3, cand[k]);
        float t_min = 1e30f;
        for (int r = 0; r < 3; ++r) {
          DW_HIP(hipEventRecord(e0, st));
          for (int q = 0; q < 4; ++q) launch_igemm_c2f(st, a0, a1, a2, a3, cand[k]);
          DW_HIP(hipEventRecord(e1, st));
          DW_HIP(hipEventSynchronize(e1));
          float ms = 0;
          DW_HIP(hipEventElapsedTime(&ms, e0, e1));
          t_min = std::min(t_min, ms);
        }
        if (log) fprintf(log, "%s\tigemm_i8_c2f_c%d_r%d\t%.2f\n", Ls[0]->op.c_str(), a1.cin, cand[k], t_min * 1e3f / 4);
        if (t_min < best) {
          best = t_min;
          rows = cand[k];
        }
      }
      if (log) fprintf(log, "%s\tfour launches\t%.2f\n", Ls[0]->op.c_str(), sum * 1e3f / 4);
      bool timed = true;
      for (Launch* L : Ls) timed = timed && L->tuned_ms > 0;
      if (!force && (!timed || best >= sum)) continue;
    }
    if (const char* fr = getenv("DW_C2F_ROWS")) {
      const int r = atoi(fr);
      if (igemm_c2f_ok(a0, a1, a2, a3, r)) rows = r;
    }
    Launch F;
    F.kernel = "igemm_i8_c2f_c" + std::to_string(a1.cin);
    F.op = Ls[0]->op + "+" + Ls[1]->op + "+" + Ls[2]->op + "+" + Ls[3]->op;
    F.work = 0;
    for (Launch* L : Ls) F.work += L->work;
    // x in, the block output out, the four weight sets
    F.bytes = (double)a0.m * (a0.cin + a3.cout);
    for (const IgemmArgs* a : {&a0, &a1, &a2, &a3}) F.bytes += (double)a->ksteps * a->cout_pad * 64;
    auto p0 = Ls[0]->ig, p1 = Ls[1]->ig, p2 = Ls[2]->ig, p3 = Ls[3]->ig;
    F.fn = [p0, p1, p2, p3, rows](hipStream_t s) { launch_igemm_c2f(s, *p0, *p1, *p2, *p3, rows); };
    F.esize = 1;
    F.group = Ls[0]->group;
    for (Launch* L : Ls) {
      F.reads.insert(F.reads.end(), L->reads.begin(), L->reads.end());
      F.writes.insert(F.writes.end(), L->writes.begin(), L->writes.end());
    }
    F.t_in = Ls[0]->t_in;
    F.t_out = Ls[3]->t_out;
    launches[i] = F;
    launches.erase(launches.begin() + (long)i + 1, launches.begin() + (long)i + 4);
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (log) fclose(log);
}

// A nearest 2x upsample (resize) of a u8 or f16 tensor folded into the
// implicit GEMM that writes that tensor: its epilogue stores every output
// pixel's values at the pixel's four pixels of the resize's output view as well
// (igemm_store, IgemmArgs::y_up), and the resize's launch goes.  The bytes
// are the resize's.  Timed against the two launches and kept only if
// faster; DW_RESIZE_FUSE=1 keeps every candidate, =0 none;
// DW_RESIZE_KEEP=<op,op,..> keeps exactly the listed resizes.
void Runtime::fuse_resize() {
  const char* env = getenv("DW_RESIZE_FUSE");
  if (env && env[0] == '0') return;
  const char* keep = getenv("DW_RESIZE_KEEP");
  const bool force = (env && env[0] == '1') || keep;
  const char* tune_env = getenv("DW_AUTOTUNE");
  const bool tuned = !((tune_env && tune_env[0] == '0') || getenv("DW_IGEMM_TILE"));
  if (!force && !tuned) return;
  hipStream_t st = be->stream;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  DW_HIP(hipEventCreate(&e0));
  DW_HIP(hipEventCreate(&e1));
  auto time4 = [&](const std::function<void(hipStream_t)>& fn) {
    fn(st);
    float t_min = 1e30f;
    for (int r = 0; r < 3; ++r) {
      DW_HIP(hipEventRecord(e0, st));
      for (int k = 0; k < 4; ++k) fn(st);
      DW_HIP(hipEventRecord(e1, st));
      DW_HIP(hipEventSynchronize(e1));
      float ms = 0;
      DW_HIP(hipEventElapsedTime(&ms, e0, e1));
      t_min = std::min(t_min, ms);
    }
    return t_min;
  };
  for (size_t j = 0; j < launches.size(); ++j) {
    Launch& R = launches[j];
    if (!R.ra || (R.rdtype != U8 && R.rdtype != F16)) continue;
    if (keep && !listed(keep, R.op)) continue;
    const ResizeArgs& ra = *R.ra;
    if (ra.ho != 2 * ra.h || ra.wo != 2 * ra.w || ra.y.pix_stride % 4 != 0 || ra.y.c_off % 4 != 0) continue;
    const int es = R.rdtype == U8 ? 1 : 2;
    // the launch that writes the resize's input
    int pi = -1;
    for (int i = (int)j - 1; i >= 0 && pi < 0; --i)
      if (launches[i].t_out == R.t_in) pi = i;
    if (pi < 0) continue;
    Launch& L = launches[pi];
    if (!L.ig || L.esize != es) continue;
    const IgemmArgs& a = *L.ig;
    if (es == 1 ? (a.epi != EPI_QU8 || a.h_wfrag || (a.res && !a.lut)) : a.epi != EPI_F16) continue;
    if (a.y_up) continue;
    if (a.y != ra.x.base || a.y_pix_stride != ra.x.pix_stride || a.y_c_off != ra.x.c_off || a.cout != ra.c ||
        a.n != ra.n || a.ho != ra.h || a.wo != ra.w)
      continue;
    // the upsample is now written at the producer's place in the list: no
    // launch in between may touch its storage (arena bytes shared with a
    // tensor still in use there)
    bool clear = true;
    for (int k = pi + 1; k < (int)j && clear; ++k)
      for (const Region& w : R.writes) {
        for (const Region& r : launches[k].reads) clear = clear && !w.overlaps(r);
        for (const Region& r : launches[k].writes) clear = clear && !w.overlaps(r);
      }
    if (!clear) continue;
    IgemmArgs f = a;
    f.y_up = ra.y.base;
    f.up_pix_stride = ra.y.pix_stride;
    f.up_c_off = ra.y.c_off;
    if (tuned) {
      const float both = time4([&a, es](hipStream_t s) { launch_igemm(s, a, es); }) + time4(R.fn);
      const float one = time4([&f, es](hipStream_t s) { launch_igemm(s, f, es); });
      if (!force && one >= both) continue;
    }
    *L.ig = f;
    L.kernel = igemm_tile_name(f, es);
    L.op += "+" + R.op;
    L.bytes += (double)R.bytes - (double)ra.n * ra.h * ra.w * ra.c * es;  // the resize's read goes
    L.writes.insert(L.writes.end(), R.writes.begin(), R.writes.end());
    L.tuned_ms = 0;
    launches.erase(launches.begin() + (long)j);
    --j;
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
}

// A detect head's u8 -> f16 1x1 conv (conv1x1_u8_f16) fused into the
// epilogue of the QLinearConv before it, when that conv's u8 output (all of
// its 64 or 80 channels in one tile) feeds only the 1x1: the u8 results are
// regrouped in LDS and go straight to the fp16 matrix cores
// (EPV_QU8_LUT_HEAD), so the intermediate is neither stored nor read back
// and the 1x1's launch goes.  The 1x1's arithmetic is conv1x1_u8_f16's, so
// its outputs are the same.  Each candidate is timed over the head tiles
// (the staged, row-tile and band-tile kernels with one tile of every
// channel; a DW_IGEMM_TILE row- or band-tile override wins) and kept
// only if it beats the two launches; DW_HEAD_FUSE=1 keeps every candidate,
// =0 none; untuned plans keep none unless DW_HEAD_FUSE=1.  DW_HEAD_KEEP=
// <op,op,..> keeps exactly the fusions whose 3x3 conv is listed.
void Runtime::fuse_heads() {
  const char* env = getenv("DW_HEAD_FUSE");
  if (env && env[0] == '0') return;
  const char* keep = getenv("DW_HEAD_KEEP");
  const bool force = (env && env[0] == '1') || keep;
  const char* tune_env = getenv("DW_AUTOTUNE");
  const bool tuned = !((tune_env && tune_env[0] == '0') || getenv("DW_IGEMM_TILE"));
  if (!force && !tuned) return;
  auto readers = [&](const std::string& t) {
    int k = 0;
    for (auto& op : g.ops)
      for (auto& i : op.in) k += i == t;
    return k;
  };
  hipStream_t st = be->stream;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  DW_HIP(hipEventCreate(&e0));
  DW_HIP(hipEventCreate(&e1));
  auto time4 = [&](const std::function<void(hipStream_t)>& fn) {
    fn(st);
    float t_min = 1e30f;
    for (int r = 0; r < 3; ++r) {
      DW_HIP(hipEventRecord(e0, st));
      for (int k = 0; k < 4; ++k) fn(st);
      DW_HIP(hipEventRecord(e1, st));
      DW_HIP(hipEventSynchronize(e1));
      float ms = 0;
      DW_HIP(hipEventElapsedTime(&ms, e0, e1));
      t_min = std::min(t_min, ms);
    }
    return t_min;
  };
  for (size_t i = 0; i + 1 < launches.size(); ++i) {
    Launch& L1 = launches[i];
    Launch& L2 = launches[i + 1];
    if (!L1.ig || L1.esize != 1 || !L2.c1a || L1.t_out.empty() || L2.t_in != L1.t_out) continue;
    const IgemmArgs& a = *L1.ig;
    const Conv1x1F16Args& c = *L2.c1a;
    if (a.epi != EPI_QU8 || !a.lut || a.res || a.h_wfrag || !(a.cout == 64 || a.cout == 80) || a.cout_pad != a.cout)
      continue;
    if (c.cin != a.cout || c.cout > a.cout || c.x != (const uint8_t*)a.y || c.x_pix_stride != a.y_pix_stride ||
        c.x_c_off != a.y_c_off || c.m != a.m)
      continue;
    if (readers(L1.t_out) != 1 || std::find(g.outputs.begin(), g.outputs.end(), L1.t_out) != g.outputs.end())
      continue;
    if (keep && !listed(keep, L1.op)) continue;
    IgemmArgs h = a;
    h.h_wfrag = c.wfrag;
    h.h_bias = c.bias;
    h.h_y = c.y;
    h.h_cout = c.cout;
    h.h_y_pix_stride = c.y_pix_stride;
    h.h_y_c_off = c.y_c_off;
    h.h_act = c.act;
    h.h_scale = c.in_scale;
    h.h_zp = c.in_zp;
    int bc[16], pb[16], tpw[16];
    const int n = igemm_candidates(h, bc, pb, tpw, 16);
    if (n == 0) continue;
    h.tile_bc = bc[0];
    h.tile_pb = pb[0];
    h.tile_tpw = tpw[0];
    if (tuned) {
      float best = 1e30f;
      int bi = 0;
      for (int k = 0; k < n; ++k) {
        IgemmArgs hk = h;
        hk.tile_bc = bc[k];
        hk.tile_pb = pb[k];
        hk.tile_tpw = tpw[k];
        const float t = time4([&hk](hipStream_t s) { launch_igemm(s, hk, 1); });
        if (t < best) {
          best = t;
          bi = k;
        }
      }
      h.tile_bc = bc[bi];
      h.tile_pb = pb[bi];
      h.tile_tpw = tpw[bi];
      if (!force && (L1.tuned_ms <= 0 || best >= L1.tuned_ms + time4(L2.fn))) continue;
    }
    auto hp = std::make_shared<IgemmArgs>(h);
    L1.ig = hp;
    L1.kernel = igemm_tile_name(h, 1);
    L1.fn = [hp](hipStream_t s) { launch_igemm(s, *hp, 1); };
    L1.op += "+" + L2.op;
    L1.work += L2.work;
    L1.bytes = L1.bytes + L2.bytes - 2.0 * (double)T(L1.t_out).pixels() * T(L1.t_out).c;
    L1.reads.insert(L1.reads.end(), L2.reads.begin(), L2.reads.end());
    L1.writes.insert(L1.writes.end(), L2.writes.begin(), L2.writes.end());
    L1.t_out = L2.t_out;
    L1.tuned_ms = 0;
    launches.erase(launches.begin() + (long)i + 1);
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
}

// The reference's INT8 conv (s8 activations, s8 HWIO weights, zero padding):
// conv2d_i8_nhwc (ops.rs:3086-3142) to the int32 accumulator, or with
// requantize_i32_to_i8 (ops.rs:3380-3386) and relu_i8 fused, which is
// conv2d_requant_relu_i8_packed (dragonwing-vulkan ops.rs:2294-2430).
void Runtime::emit_iconv(const Group& gr) {
  const OpNode& op = g.ops[gr.conv];
  const TensorInfo& W = g.t[op.in[1]];
  RtTensor& x = T(gr.in);
  RtTensor& y = T(gr.out);
  if (!W.is_init || W.dims.size() != 4 || W.dtype != DW_DTYPE_I8)
    fail(DW_ERR_UNSUPPORTED, "runtime: INT8 conv " + op.name + " needs HWIO int8 weights");
  const int kh = (int)W.dims[0], kw = (int)W.dims[1], ci = (int)W.dims[2], co = (int)W.dims[3];
  if (ci != x.c || co != y.c) fail(DW_ERR_RUNTIME, "runtime: conv " + op.name + " channel mismatch");
  if (x.dtype != I8) fail(DW_ERR_RUNTIME, "runtime: INT8 conv " + op.name + " needs an int8 input");
  if (gr.requant ? y.dtype != I8 : y.dtype != I32)
    fail(DW_ERR_RUNTIME, "runtime: INT8 conv " + op.name +
                             (gr.requant ? " must requantize to int8" : " without Requantize must write int32"));
  if (op.in.size() > 2 && !op.in[2].empty())
    fail(DW_ERR_UNSUPPORTED, "runtime: INT8 conv " + op.name +
                                 " has a bias (the reference's INT8 convs take none: fusion.rs:303-309)");
  if (op.p.group > 1) fail(DW_ERR_UNSUPPORTED, "runtime: grouped INT8 conv " + op.name);
  if (op.p.dilations[0] > 1 || op.p.dilations[1] > 1) fail(DW_ERR_UNSUPPORTED, "runtime: dilation != 1");
  if (ci % 16 != 0 || co % 4 != 0 || kh * kw > 31)
    fail(DW_ERR_UNSUPPORTED, "runtime: INT8 conv needs c_in % 16 == 0, c_out % 4 == 0 and at most 31 taps (" +
                                 op.name + ")");
  if (x.pix_stride % 16 != 0 || x.abs_off % 16 != 0 || y.pix_stride % 4 != 0 || y.abs_off % 4 != 0)
    fail(DW_ERR_RUNTIME, "runtime: misaligned view for " + op.name);
  IgemmArgs a{};
  a.x = (const uint8_t*)x.base;
  a.y = y.base;
  a.n = (int)x.n; a.h = (int)x.h; a.w = (int)x.w; a.cin = ci; a.cout = co; a.kh = kh; a.kw = kw;
  a.sh = std::max(1, op.p.strides[0]); a.sw = std::max(1, op.p.strides[1]);
  a.pt = op.p.pads[0]; a.pl = op.p.pads[1]; a.ho = (int)y.h; a.wo = (int)y.w;
  a.m = (int)y.pixels();
  a.ksteps = (kh * kw * ci + 63) / 64;
  const int bc = igemm_channel_tile(co);
  a.cout_pad = (co + bc - 1) / bc * bc;
  a.x_pix_stride = x.pix_stride; a.x_c_off = x.abs_off;
  a.y_pix_stride = y.pix_stride; a.y_c_off = y.abs_off;
  void* whwio = upload(W.data.data(), W.data.size());
  void* wpk = dalloc((size_t)a.ksteps * a.cout_pad * 64);
  launch_pack_weights(be->stream, whwio, wpk, kh * kw * ci, co, a.cout_pad, a.ksteps, 1);
  a.wpk = (const uint8_t*)wpk;
  a.epi = gr.requant ? EPI_QS8_REF : EPI_I32;
  a.tscale = gr.requant_scale;
  a.act = gr.act;
  a.xxor = 0;  // s8 operands as they are; padding taps read 0
  a.xpad = 0;
  Launch L;
  L.op = join_names(g, gr.ops);
  L.work = 2.0 * (double)y.pixels() * co * kh * kw * ci;
  L.bytes = (double)x.bytes() + W.data.size() + (double)y.bytes();
  DW_HIP(hipStreamSynchronize(be->stream));
  push_igemm(L, a, 1);
}

void Runtime::push_igemm(Launch& L, const IgemmArgs& a, int esize) {
  auto ig = std::make_shared<IgemmArgs>(a);
  L.ig = ig;
  L.esize = esize;
  L.kernel = igemm_tile_name(*ig, esize);
  L.fn = [ig, esize](hipStream_t st) { launch_igemm(st, *ig, esize); };
  launches.push_back(L);
}

// Plan-time tuning of the implicit-GEMM tile shapes: every candidate shape
// of every MFMA convolution is timed on the runtime's own buffers (one
// warm-up launch, then the best of three), and the fastest is kept.  The
// tile shape changes only the work split, never the order of the k-steps a
// result is accumulated over, so outputs are identical for every choice.
// The launches write only buffers the next run() rewrites.  Set
// DW_AUTOTUNE=0 to keep the built-in heuristic (DW_IGEMM_TILE, which forces
// a shape, also disables it).  DW_AUTOTUNE_LOG=<file> appends every
// candidate's time per launch (op, kernel, microseconds) to that file.
void Runtime::autotune() {
  const char* env = getenv("DW_AUTOTUNE");
  if ((env && env[0] == '0') || getenv("DW_IGEMM_TILE")) return;
  FILE* log = nullptr;
  if (const char* lp = getenv("DW_AUTOTUNE_LOG")) log = fopen(lp, "a");
  hipStream_t st = be->stream;
  hipEvent_t e0, e1;
  DW_HIP(hipEventCreate(&e0));
  DW_HIP(hipEventCreate(&e1));
  for (auto& L : launches) {
    if (!L.dw_band) continue;
    // band heights whose tile fits LDS (two workgroups a CU where possible)
    float best = 1e30f;
    int bb = *L.dw_band;
    for (int cand : {404, 408, 410, 420, 804, 808, 810}) {
      if (!dwconv3_tile_cfg_ok(*L.dwa, cand / 100, cand % 100)) continue;
      const int band = cand;
      *L.dw_band = band;
      L.fn(st);
      float t_min = 1e30f;
      for (int r = 0; r < 3; ++r) {
        DW_HIP(hipEventRecord(e0, st));
        for (int k = 0; k < 4; ++k) L.fn(st);
        DW_HIP(hipEventRecord(e1, st));
        DW_HIP(hipEventSynchronize(e1));
        float ms = 0;
        DW_HIP(hipEventElapsedTime(&ms, e0, e1));
        t_min = std::min(t_min, ms);
      }
      if (t_min < best) {
        best = t_min;
        bb = band;
      }
    }
    *L.dw_band = bb;
    L.kernel = "dwconv3_tile_u" + std::to_string(bb / 100) + "r" + std::to_string(bb % 100);
  }
  for (auto& L : launches) {
    if (!L.ig) continue;
    IgemmArgs& a = *L.ig;
    int bc[64], pb[64], tpw[64];
    const int n = igemm_candidates(a, bc, pb, tpw, 64);
    float best = 1e30f;
    int bi = -1;
    for (int i = 0; i < n; ++i) {
      a.tile_bc = bc[i];
      a.tile_pb = pb[i];
      a.tile_tpw = tpw[i];
      if (log) fprintf(log, "%s\t%s\t", L.op.c_str(), igemm_tile_name(a, L.esize));
      launch_igemm(st, a, L.esize);
      // back-to-back launches between the events: the event overhead is
      // spread over several kernels, so close candidates are told apart
      float t_min = 1e30f;
      for (int r = 0; r < 3; ++r) {
        DW_HIP(hipEventRecord(e0, st));
        for (int k = 0; k < 4; ++k) launch_igemm(st, a, L.esize);
        DW_HIP(hipEventRecord(e1, st));
        DW_HIP(hipEventSynchronize(e1));
        float ms = 0;
        DW_HIP(hipEventElapsedTime(&ms, e0, e1));
        t_min = std::min(t_min, ms);
      }
      if (log) fprintf(log, "%.2f\n", t_min * 1e3f / 4);
      if (t_min < best) {
        best = t_min;
        bi = i;
      }
    }
    if (bi >= 0) {
      a.tile_bc = bc[bi];
      a.tile_pb = pb[bi];
      a.tile_tpw = tpw[bi];
      L.tuned_ms = best;
    }
    L.kernel = igemm_tile_name(a, L.esize);
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (log) fclose(log);
  info.clear();
}

void Runtime::drop_capture() {
  if (hexec) {
    DW_HIP(hipStreamSynchronize(be->stream));
    (void)hipGraphExecDestroy(hexec);
    hexec = nullptr;
  }
  if (hgraph) {
    (void)hipGraphDestroy(hgraph);
    hgraph = nullptr;
  }
}

void Runtime::set_input_nchw(const std::string& name, const void* src) {
  RtTensor& t = T(name);
  if (t.dtype != F32 && t.dtype != F16) fail(DW_ERR_UNSUPPORTED, "NCHW input: the input must be f32 or f16");
  NchwIn& e = nchw[name];
  if (e.launch == -2) {
    // the stem that can read NCHW itself: the only launch reading the
    // input, a 3x3 three-channel direct conv on the dense f16 tensor
    int found = -1, count = 0;
    for (size_t k = 0; k < launches.size(); ++k)
      for (const Region& r : launches[k].reads)
        if (r.rid == t.rid) {
          ++count;
          found = (int)k;
          break;
        }
    e.launch = -1;
    if (count == 1 && launches[found].da) {
      const DirectArgs& a = *launches[found].da;
      if (a.in_kind == 1 && a.x == t.base && a.kh == 3 && a.kw == 3 && a.cin == 3 && a.cout % 16 == 0 &&
          a.x_pix_stride == 3 && a.x_c_off == 0 && t.pix_stride == 3 && t.abs_off == 0) {
        e.launch = found;
        e.orig = a;
      }
    } else if (count == 1 && launches[found].sa) {
      // the fp16 MFMA stem reads any dense f16 input of up to 4 channels
      const StemF16Args& a = *launches[found].sa;
      if (t.dtype == F16 && a.in_kind == 1 && (const void*)a.x == t.base && a.x_pix_stride == a.cin &&
          a.x_c_off == 0 && t.pix_stride == (int)t.c && t.abs_off == 0) {
        e.launch = found;
        e.orig_s = a;
      }
    }
  }
  e.src = src;
  e.active = true;
  if (e.launch >= 0 && launches[e.launch].da) {
    DirectArgs& a = *launches[e.launch].da;
    a = e.orig;
    a.x = src;
    a.in_kind = 3;
  } else if (e.launch >= 0) {
    StemF16Args& a = *launches[e.launch].sa;
    a = e.orig_s;
    a.x_nchw = (const float*)src;
    a.in_kind = 3;
  }
  drop_capture();
}

void Runtime::reset_input_layout(const std::string& name) {
  auto it = nchw.find(name);
  if (it == nchw.end() || !it->second.active) return;
  NchwIn& e = it->second;
  if (e.launch >= 0 && launches[e.launch].da) *launches[e.launch].da = e.orig;
  else if (e.launch >= 0) *launches[e.launch].sa = e.orig_s;
  e.active = false;
  e.src = nullptr;
  drop_capture();
}

void Runtime::run() {
  hipStream_t st = be->stream;
  if (stats) {
    for (size_t i = 0; i < stats_names.size(); ++i) launch_minmax_init(st, stats_dev + 2 * i);
    // graph inputs are not produced by any op: record them first
    for (auto& in : g.inputs) {
      auto it = std::find(stats_names.begin(), stats_names.end(), in);
      if (it != stats_names.end()) {
        RtTensor& t = T(in);
        launch_minmax(st, t.view(), (int)t.pixels(), (int)t.c, stats_dev + 2 * (it - stats_names.begin()));
      }
    }
  }
  if (capture && !stats) {
    if (!hexec) {
      DW_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
      enqueue(st);
      DW_HIP(hipStreamEndCapture(st, &hgraph));
      DW_HIP(hipGraphInstantiate(&hexec, hgraph, nullptr, nullptr, 0));
    }
    DW_HIP(hipGraphLaunch(hexec, st));
    return;
  }
  enqueue(st);
}

}  // namespace dw

// ===========================================================================
// C ABI
// ===========================================================================
struct dw_hip_graph_runtime {
  dw::Runtime rt;
};

#define API_BEGIN try {
#define API_END                           \
  }                                       \
  catch (const dw::Error& e) {            \
    dw::set_last_error(e.msg);            \
    return e.code;                        \
  }                                       \
  catch (const std::exception& e) {       \
    dw::set_last_error(e.what());         \
    return DW_ERR_BACKEND;                \
  }                                       \
  return DW_OK;

namespace {
dw::Runtime& R(dw_hip_graph_runtime* rt) {
  if (!rt) dw::fail(DW_ERR_INVALID, "null runtime");
  DW_HIP(hipSetDevice(rt->rt.be->device));
  return rt->rt;
}
dw::Backend* Bk(dw_hip_backend* be) {
  if (!be) dw::fail(DW_ERR_INVALID, "null backend");
  dw::Backend* b = reinterpret_cast<dw::Backend*>(be);
  DW_HIP(hipSetDevice(b->device));
  return b;
}

using dw::f16_to_f32_ref;
}  // namespace

extern "C" {

int dw_hip_graph_runtime_create(dw_hip_backend* be, const dw_graph* g, dw_hip_graph_runtime** out) {
  return dw_hip_graph_runtime_create_ex(be, g, 0u, out);
}

int dw_hip_graph_runtime_create_ex(dw_hip_backend* be, const dw_graph* g, unsigned flags,
                                   dw_hip_graph_runtime** out) {
  API_BEGIN
  if (!g || !out) dw::fail(DW_ERR_INVALID, "null argument");
  if (flags & ~(unsigned)(DW_RT_EXACT_U8_F16_CONV | DW_RT_EXACT_F16_DEPTHWISE))
    dw::fail(DW_ERR_INVALID, "unknown runtime flags");
  dw::Backend* b = Bk(be);
  std::lock_guard<std::mutex> lock(b->mu);
  auto* rt = new dw_hip_graph_runtime();
  rt->rt.exact_u8_f16 = (flags & DW_RT_EXACT_U8_F16_CONV) != 0;
  rt->rt.exact_f16_dw = (flags & DW_RT_EXACT_F16_DEPTHWISE) != 0;
  dw::hold(b);  // released with the runtime
  try {
    rt->rt.build(b, g->g, false);
  } catch (...) {
    delete rt;
    dw::release(b);
    throw;
  }
  *out = rt;
  API_END
}

void dw_hip_graph_runtime_destroy(dw_hip_graph_runtime* rt) {
  if (!rt) return;
  dw::Backend* b = rt->rt.be;
  delete rt;
  if (b) dw::release(b);
}

int dw_hip_graph_set_input_bytes(dw_hip_graph_runtime* rth, const char* name, const void* data, size_t len) {
  API_BEGIN
  dw::Runtime& rt = R(rth);
  std::lock_guard<std::mutex> lock(rt.be->mu);
  if (!name || std::find(rt.g.inputs.begin(), rt.g.inputs.end(), std::string(name)) == rt.g.inputs.end())
    dw::fail(DW_ERR_RUNTIME, std::string("input not found: ") + (name ? name : "(null)"));
  dw::RtTensor& t = rt.T(name);
  rt.reset_input_layout(name);
  if (len != t.bytes())
    dw::fail(DW_ERR_RUNTIME, "input size mismatch: expected " + std::to_string(t.bytes()) + ", got " +
                                 std::to_string(len));
  DW_HIP(hipMemcpyAsync(t.base, data, len, hipMemcpyHostToDevice, rt.be->stream));
  DW_HIP(hipStreamSynchronize(rt.be->stream));
  API_END
}

int dw_hip_graph_set_input_f32(dw_hip_graph_runtime* rth, const char* name, const float* data, size_t count) {
  API_BEGIN
  dw::Runtime& rt = R(rth);
  std::lock_guard<std::mutex> lock(rt.be->mu);
  if (!name || std::find(rt.g.inputs.begin(), rt.g.inputs.end(), std::string(name)) == rt.g.inputs.end())
    dw::fail(DW_ERR_RUNTIME, std::string("input not found: ") + (name ? name : "(null)"));
  dw::RtTensor& t = rt.T(name);
  rt.reset_input_layout(name);
  const size_t n = (size_t)(t.pixels() * t.c);
  if (count != n)
    dw::fail(DW_ERR_RUNTIME, "input size mismatch: expected " + std::to_string(n) + ", got " + std::to_string(count));
  if (t.dtype == dw::F32) {
    DW_HIP(hipMemcpyAsync(t.base, data, n * 4, hipMemcpyHostToDevice, rt.be->stream));
  } else if (t.dtype == dw::F16) {
    std::vector<uint16_t> h(n);
    for (size_t i = 0; i < n; ++i) h[i] = dw::f16_bits_from_f32(data[i]);
    DW_HIP(hipMemcpyAsync(t.base, h.data(), n * 2, hipMemcpyHostToDevice, rt.be->stream));
    DW_HIP(hipStreamSynchronize(rt.be->stream));
  } else {
    dw::fail(DW_ERR_RUNTIME, "unsupported dtype for set_input_f32");
  }
  DW_HIP(hipStreamSynchronize(rt.be->stream));
  API_END
}

int dw_hip_graph_set_input_nchw_f32(dw_hip_graph_runtime* rth, const char* name, const float* data, size_t count) {
  API_BEGIN
  dw::Runtime& rt = R(rth);
  std::lock_guard<std::mutex> lock(rt.be->mu);
  if (!name || std::find(rt.g.inputs.begin(), rt.g.inputs.end(), std::string(name)) == rt.g.inputs.end())
    dw::fail(DW_ERR_RUNTIME, std::string("input not found: ") + (name ? name : "(null)"));
  if (!data) dw::fail(DW_ERR_INVALID, "null data");
  dw::RtTensor& t = rt.T(name);
  const size_t n = (size_t)(t.pixels() * t.c);
  if (count != n)
    dw::fail(DW_ERR_RUNTIME, "input size mismatch: expected " + std::to_string(n) + ", got " + std::to_string(count));
  auto& e = rt.nchw[name];
  if (e.stage_bytes != n * 4) {
    if (e.stage) DW_HIP(hipFree(e.stage));
    e.stage = nullptr;
    e.stage_bytes = 0;
    DW_HIP(hipMalloc(&e.stage, n * 4));
    e.stage_bytes = n * 4;
  }
  DW_HIP(hipMemcpyAsync(e.stage, data, n * 4, hipMemcpyHostToDevice, rt.be->stream));
  DW_HIP(hipStreamSynchronize(rt.be->stream));
  rt.set_input_nchw(name, e.stage);
  API_END
}

int dw_hip_graph_bind_input_nchw_f32(dw_hip_graph_runtime* rth, const char* name, const dw_hip_buffer* buf) {
  API_BEGIN
  dw::Runtime& rt = R(rth);
  std::lock_guard<std::mutex> lock(rt.be->mu);
  if (!name || std::find(rt.g.inputs.begin(), rt.g.inputs.end(), std::string(name)) == rt.g.inputs.end())
    dw::fail(DW_ERR_RUNTIME, std::string("input not found: ") + (name ? name : "(null)"));
  if (!buf) dw::fail(DW_ERR_INVALID, "null buffer");
  dw::RtTensor& t = rt.T(name);
  const size_t n = (size_t)(t.pixels() * t.c);
  if (dw_hip_buffer_len_bytes(buf) != n * 4)
    dw::fail(DW_ERR_RUNTIME, "input size mismatch: expected " + std::to_string(n * 4) + " bytes");
  rt.set_input_nchw(name, dw_hip_buffer_device_ptr(buf));
  API_END
}

int dw_hip_graph_run(dw_hip_graph_runtime* rth) {
  API_BEGIN
  dw::Runtime& rt = R(rth);
  std::lock_guard<std::mutex> lock(rt.be->mu);
  rt.run();
  API_END
}

int dw_hip_graph_run_unbatched(dw_hip_graph_runtime* rth) {
  API_BEGIN
  dw::Runtime& rt = R(rth);
  std::lock_guard<std::mutex> lock(rt.be->mu);
  const bool trace = getenv("DW_TRACE") != nullptr;
  hipStream_t st = rt.be->stream;
  for (size_t i = 0; i < rt.launches.size(); ++i) {
    dw::Launch& L = rt.launches[i];
    if (trace) fprintf(stderr, "[launch %3zu] %s (%s)\n", i, L.kernel.c_str(), L.op.c_str());
    try {
      L.fn(st);
      if (trace) DW_HIP(hipStreamSynchronize(st));
    } catch (const dw::Error& e) {
      dw::fail(e.code, "launch[" + std::to_string(i) + "] " + L.kernel + " (" + L.op + ") failed: " + e.msg);
    }
  }
  API_END
}

int dw_hip_graph_activation_bytes(dw_hip_graph_runtime* rth, size_t* arena, size_t* unshared) {
  API_BEGIN
  if (!rth) dw::fail(DW_ERR_INVALID, "null graph runtime");
  if (arena) *arena = rth->rt.act_bytes;
  if (unshared) *unshared = rth->rt.act_bytes_unshared;
  API_END
}

int dw_hip_graph_num_io(dw_hip_graph_runtime* rth, int which) {
  if (!rth) return -1;
  return (int)(which ? rth->rt.g.outputs.size() : rth->rt.g.inputs.size());
}

const char* dw_hip_graph_io_name(dw_hip_graph_runtime* rth, int which, int index) {
  if (!rth) return "";
  const auto& v = which ? rth->rt.g.outputs : rth->rt.g.inputs;
  if (index < 0 || index >= (int)v.size()) return "";
  return v[index].c_str();
}

int dw_hip_graph_tensor_shape(dw_hip_graph_runtime* rth, const char* name, int64_t* dims4, int* rank) {
  API_BEGIN
  dw::Runtime& rt = R(rth);
  std::lock_guard<std::mutex> lock(rt.be->mu);
  if (!name || !dims4 || !rank) dw::fail(DW_ERR_INVALID, "null argument");
  auto it = rt.g.t.find(name);
  if (it == rt.g.t.end()) dw::fail(DW_ERR_RUNTIME, std::string("runtime: unknown tensor '") + name + "'");
  const auto& d = it->second.dims;
  if (d.size() > 4) dw::fail(DW_ERR_UNSUPPORTED, "tensor rank above 4");
  *rank = (int)d.size();
  for (size_t i = 0; i < d.size(); ++i) dims4[i] = d[i];
  API_END
}

static void download_tensor(dw::Runtime& rt, const std::string& name, std::vector<uint8_t>& out) {
  dw::RtTensor& t = rt.T(name);
  if (!t.base) dw::fail(DW_ERR_RUNTIME, "tensor " + name + " is not materialized");
  DW_HIP(hipStreamSynchronize(rt.be->stream));
  const size_t es = dw::dtype_size(t.dtype);
  out.resize(t.bytes());
  DW_HIP(hipMemcpy2D(out.data(), t.c * es, (const uint8_t*)t.base + (size_t)t.abs_off * es,
                     (size_t)t.pix_stride * es, t.c * es, (size_t)t.pixels(), hipMemcpyDeviceToHost));
}

int dw_hip_graph_get_output_bytes(dw_hip_graph_runtime* rth, const char* name, void* data, size_t len) {
  API_BEGIN
  dw::Runtime& rt = R(rth);
  std::lock_guard<std::mutex> lock(rt.be->mu);
  if (!name) dw::fail(DW_ERR_INVALID, "null name");
  std::vector<uint8_t> buf;
  download_tensor(rt, name, buf);
  if (len != buf.size())
    dw::fail(DW_ERR_RUNTIME, "output size mismatch: expected " + std::to_string(buf.size()) + ", got " +
                                 std::to_string(len));
  memcpy(data, buf.data(), len);
  API_END
}

int dw_hip_graph_get_output_f32(dw_hip_graph_runtime* rth, const char* name, float* data, size_t count) {
  API_BEGIN
  dw::Runtime& rt = R(rth);
  std::lock_guard<std::mutex> lock(rt.be->mu);
  if (!name) dw::fail(DW_ERR_INVALID, "null name");
  dw::RtTensor& t = rt.T(name);
  std::vector<uint8_t> buf;
  download_tensor(rt, name, buf);
  const size_t n = (size_t)(t.pixels() * t.c);
  if (count != n) dw::fail(DW_ERR_RUNTIME, "output size mismatch");
  if (t.dtype == dw::F32) {
    memcpy(data, buf.data(), n * 4);
  } else if (t.dtype == dw::F16) {
    const uint16_t* h = (const uint16_t*)buf.data();
    for (size_t i = 0; i < n; ++i) data[i] = f16_to_f32_ref(h[i]);
  } else if (t.dtype == dw::U8) {
    for (size_t i = 0; i < n; ++i) data[i] = (float)((int)buf[i] - t.zp) * t.scale;
  } else {
    dw::fail(DW_ERR_RUNTIME, "unsupported dtype for get_output_f32");
  }
  API_END
}

int dw_hip_graph_tensor_bytes(dw_hip_graph_runtime* rth, const char* name, size_t* len) {
  API_BEGIN
  dw::Runtime& rt = R(rth);
  std::lock_guard<std::mutex> lock(rt.be->mu);
  if (!name || !len) dw::fail(DW_ERR_INVALID, "null argument");
  *len = rt.T(name).bytes();
  API_END
}

int dw_hip_graph_enable_capture(dw_hip_graph_runtime* rth, int enable) {
  API_BEGIN
  dw::Runtime& rt = R(rth);
  std::lock_guard<std::mutex> lock(rt.be->mu);
  rt.capture = enable != 0;
  API_END
}

int dw_hip_graph_num_launches(dw_hip_graph_runtime* rth) {
  if (!rth) return -1;
  return (int)rth->rt.launches.size();
}

const char* dw_hip_graph_launch_info(dw_hip_graph_runtime* rth, int index) {
  if (!rth || index < 0 || index >= (int)rth->rt.launches.size()) return "";
  dw::Runtime& rt = rth->rt;
  if (rt.info.size() != rt.launches.size()) {
    rt.info.clear();
    for (auto& L : rt.launches) {
      char b[64];
      snprintf(b, sizeof b, " %.17g %.17g", L.work, L.bytes);
      rt.info.push_back(L.kernel + " " + L.op + b);
    }
  }
  return rt.info[index].c_str();
}

int dw_hip_graph_run_profiled(dw_hip_graph_runtime* rth, float* launch_ms) {
  API_BEGIN
  dw::Runtime& rt = R(rth);
  std::lock_guard<std::mutex> lock(rt.be->mu);
  if (!launch_ms) dw::fail(DW_ERR_INVALID, "null output");
  const size_t n = rt.launches.size();
  std::vector<hipEvent_t> ev(n + 1);
  for (auto& e : ev) DW_HIP(hipEventCreate(&e));
  hipStream_t st = rt.be->stream;
  DW_HIP(hipEventRecord(ev[0], st));
  for (size_t i = 0; i < n; ++i) {
    rt.launches[i].fn(st);
    DW_HIP(hipEventRecord(ev[i + 1], st));
  }
  DW_HIP(hipEventSynchronize(ev[n]));
  for (size_t i = 0; i < n; ++i) DW_HIP(hipEventElapsedTime(&launch_ms[i], ev[i], ev[i + 1]));
  for (auto& e : ev) (void)hipEventDestroy(e);
  API_END
}

int dw_hip_graph_time_launches(dw_hip_graph_runtime* rth, int repeat, float* launch_ms) {
  API_BEGIN
  dw::Runtime& rt = R(rth);
  std::lock_guard<std::mutex> lock(rt.be->mu);
  if (!launch_ms || repeat < 1) dw::fail(DW_ERR_INVALID, "time_launches: null output or repeat < 1");
  const size_t n = rt.launches.size();
  hipEvent_t e0, e1;
  DW_HIP(hipEventCreate(&e0));
  DW_HIP(hipEventCreate(&e1));
  hipStream_t st = rt.be->stream;
  for (size_t i = 0; i < n; ++i) {
    DW_HIP(hipEventRecord(e0, st));
    for (int r = 0; r < repeat; ++r) rt.launches[i].fn(st);
    DW_HIP(hipEventRecord(e1, st));
    DW_HIP(hipEventSynchronize(e1));
    float ms = 0;
    DW_HIP(hipEventElapsedTime(&ms, e0, e1));
    launch_ms[i] = ms / repeat;
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  API_END
}

int dw_hip_graph_time_launches_rotated(dw_hip_graph_runtime* const* rths, int n_rt, int repeat, float* launch_ms) {
  API_BEGIN
  if (!rths || n_rt < 1 || !launch_ms || repeat < 1)
    dw::fail(DW_ERR_INVALID, "time_launches_rotated: null argument, no runtime or repeat < 1");
  const dw::Runtime& r0 = R(rths[0]);
  std::lock_guard<std::mutex> lock(r0.be->mu);
  for (int k = 1; k < n_rt; ++k) {
    const dw::Runtime& rk = R(rths[k]);
    if (rk.launches.size() != r0.launches.size() || rk.be != r0.be)
      dw::fail(DW_ERR_INVALID, "time_launches_rotated: runtimes differ in launches or backend");
  }
  const size_t n = r0.launches.size();
  hipEvent_t e0, e1;
  DW_HIP(hipEventCreate(&e0));
  DW_HIP(hipEventCreate(&e1));
  hipStream_t st = r0.be->stream;
  for (size_t i = 0; i < n; ++i) {
    DW_HIP(hipEventRecord(e0, st));
    for (int r = 0; r < repeat; ++r) R(rths[r % n_rt]).launches[i].fn(st);
    DW_HIP(hipEventRecord(e1, st));
    DW_HIP(hipEventSynchronize(e1));
    float ms = 0;
    DW_HIP(hipEventElapsedTime(&ms, e0, e1));
    launch_ms[i] = ms / repeat;
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  API_END
}

// Calibrator (crates/dragonwing-onnx/src/calibration.rs:90-260): runs the F32
// graph on the GPU over `num_images` inputs (in batches of the graph's N),
// records per-tensor min/max (calibration.rs:56-69) and stores the ranges in
// the graph for dw_graph_quantize_qdq.
int dw_hip_calibrate(dw_hip_backend* be, dw_graph* gh, const char* input_name, const float* images,
                     size_t floats_per_image, int num_images) {
  API_BEGIN
  dw::Backend* b = Bk(be);
  std::lock_guard<std::mutex> lock(b->mu);
  if (!gh || !images || !input_name) dw::fail(DW_ERR_INVALID, "null argument");
  if (gh->g.dtype != DW_GRAPH_F32) dw::fail(DW_ERR_RUNTIME, "calibration needs the F32 graph");
  gh->g.json.clear();
  dw::Runtime rt;
  rt.build(b, gh->g, true);
  dw::RtTensor& in = rt.T(input_name);
  const int batch = (int)in.n;
  if (floats_per_image * batch != (size_t)(in.pixels() * in.c))
    dw::fail(DW_ERR_INVALID, "calibration: image size does not match the graph input");
  if (num_images <= 0 || num_images % batch != 0)
    dw::fail(DW_ERR_INVALID, "calibration: image count must be a multiple of the graph batch");
  std::map<std::string, std::pair<float, float>> acc;
  std::vector<float> mm(rt.stats_names.size() * 2);
  for (int i0 = 0; i0 < num_images; i0 += batch) {
    DW_HIP(hipMemcpy(in.base, images + (size_t)i0 * floats_per_image, floats_per_image * batch * 4,
                     hipMemcpyHostToDevice));
    rt.run();
    DW_HIP(hipStreamSynchronize(b->stream));
    DW_HIP(hipMemcpy(mm.data(), rt.stats_dev, mm.size() * 4, hipMemcpyDeviceToHost));
    for (size_t k = 0; k < rt.stats_names.size(); ++k) {
      auto it = acc.find(rt.stats_names[k]);
      if (it == acc.end())
        acc[rt.stats_names[k]] = {mm[2 * k], mm[2 * k + 1]};
      else
        it->second = {std::min(it->second.first, mm[2 * k]), std::max(it->second.second, mm[2 * k + 1])};
    }
  }
  for (auto& kv : acc) {
    if (!(kv.second.first <= kv.second.second)) continue;  // never written
    dw::TensorInfo& ti = gh->g.tensor(kv.first);
    ti.has_range = true;
    ti.rmin = kv.second.first;
    ti.rmax = kv.second.second;
  }
  API_END
}

}  // extern "C"
