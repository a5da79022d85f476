// Graph IR and the compiler passes of dragonwing-onnx, restated in C++:
//   fold_batchnorm          crates/dragonwing-onnx/src/graph.rs:521-690
//   convert_nchw_to_nhwc    crates/dragonwing-onnx/src/graph.rs:248-290
//   apply_fusion_passes     crates/dragonwing-onnx/src/fusion.rs:126-190 (SiLU)
//   convert_to_f16          crates/dragonwing-onnx/src/runtime.rs:800-811
//   quantize_qdq            QDQ-folded u8 graph (QLinearConv etc.); the
//                           reference's quantizer (quantize.rs:73-368) emits
//                           symmetric s8 with one averaged requant scale,
//                           this pass emits the ONNX per-channel form.
// Host-only code: no device work happens here.
#include "graph.h"

#include <math.h>
#include <string.h>

#include <algorithm>
#include <exception>
#include <functional>
#include <numeric>
#include <set>
#include <sstream>

#include "backend.h"

namespace dw {

TensorInfo& GraphIR::tensor(const std::string& name) {
  auto it = t.find(name);
  if (it == t.end()) fail(DW_ERR_RUNTIME, "unknown tensor '" + name + "'");
  return it->second;
}
const TensorInfo& GraphIR::tensor(const std::string& name) const {
  auto it = t.find(name);
  if (it == t.end()) fail(DW_ERR_RUNTIME, "unknown tensor '" + name + "'");
  return it->second;
}
std::vector<int> GraphIR::consumers(const std::string& name) const {
  std::vector<int> r;
  for (size_t i = 0; i < ops.size(); ++i)
    for (auto& in : ops[i].in)
      if (in == name) {
        r.push_back((int)i);
        break;
      }
  return r;
}
int GraphIR::producer(const std::string& name) const {
  for (size_t i = 0; i < ops.size(); ++i)
    for (auto& o : ops[i].out)
      if (o == name) return (int)i;
  return -1;
}
bool GraphIR::is_output(const std::string& name) const {
  return std::find(outputs.begin(), outputs.end(), name) != outputs.end();
}

void build_silu_lut(uint8_t lut[256], float sx, int zx, float sy, int zy) {
  for (int q = 0; q < 256; ++q) {
    const float v = (float)(q - zx) * sx;
    const float s = 1.0f / (1.0f + expf(-v));
    const float a = v * s;
    float r = nearbyintf(a / sy) + (float)zy;
    r = r < 0.0f ? 0.0f : (r > 255.0f ? 255.0f : r);
    lut[q] = (uint8_t)r;
  }
}

namespace {

std::vector<float> as_f32(const TensorInfo& ti) {
  if (ti.dtype != DW_DTYPE_F32) fail(DW_ERR_UNSUPPORTED, "expected an f32 initializer");
  std::vector<float> v(ti.data.size() / 4);
  memcpy(v.data(), ti.data.data(), v.size() * 4);
  return v;
}
void set_f32(TensorInfo& ti, const std::vector<float>& v) {
  ti.data.resize(v.size() * 4);
  memcpy(ti.data.data(), v.data(), ti.data.size());
  ti.dtype = DW_DTYPE_F32;
  ti.is_init = true;
}

uint16_t f16_from_f32(float v) { return f16_bits_from_f32(v); }

}  // namespace

// F16::from_f32 (dtype.rs:164-222): IEEE round to nearest even.
uint16_t f16_bits_from_f32(float v) {
  uint32_t bits;
  memcpy(&bits, &v, 4);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const int32_t e = (int32_t)((bits >> 23) & 0xFF);
  const uint32_t m = bits & 0x7FFFFFu;
  if (e == 255) return (uint16_t)(sign | (m ? 0x7E00u | std::min<uint32_t>(m >> 13, 0x1FF) : 0x7C00u));
  const int32_t ne = e - 112;
  if (ne >= 31) return (uint16_t)(sign | 0x7C00u);
  if (ne <= 0) {
    if (ne < -10) return (uint16_t)sign;
    const int32_t sh = 1 - ne;
    const uint32_t mh = m | 0x800000u;
    const uint32_t q = mh >> (13 + sh);
    const uint32_t rb = (mh >> (12 + sh)) & 1u;
    const uint32_t st = (mh & ((1u << (12 + sh)) - 1u)) != 0;
    return (uint16_t)(sign | (q + (rb & (st | (q & 1u)))));
  }
  const uint32_t q = m >> 13;
  const uint32_t rb = (m >> 12) & 1u;
  const uint32_t st = (m & 0xFFFu) != 0;
  const uint32_t r = q + (rb & (st | (q & 1u)));
  if (r >= 0x400u) {
    if (ne + 1 >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((uint32_t)(ne + 1) << 10));
  }
  return (uint16_t)(sign | ((uint32_t)ne << 10) | r);
}

namespace {

std::string jesc(const std::string& s) {
  std::string o;
  for (char c : s) {
    if (c == '"' || c == '\\') o += '\\';
    o += c;
  }
  return o;
}

std::string fstr(float f) {
  // infinities as out-of-range literals that JSON readers take as +-inf
  if (isinf(f)) return f > 0 ? "1e999" : "-1e999";
  if (isnan(f)) return "NaN";
  char b[64];
  snprintf(b, sizeof b, "%.9g", (double)f);
  return b;
}

// --------------------------------------------------------------------------
// fold_batchnorm (graph.rs:521-690): Conv -> BatchNormalization(scale, B,
// mean, var) with the conv output used only by the BN.  In f64:
//   w' = (f32)(w * g / sqrt(var + eps)),  b' = (f32)((b - mean) * sf + beta)
// The conv takes the BN's output name; a bias "<W>_bias_folded" is added
// when the conv had none (graph.rs:630-664).
// --------------------------------------------------------------------------
int fold_batchnorm(GraphIR& g) {
  int folded = 0;
  for (size_t i = 0; i < g.ops.size(); ++i) {
    OpNode& bn = g.ops[i];
    if (bn.type != "BatchNormalization") continue;
    const int pi = g.producer(bn.in[0]);
    if (pi < 0) continue;
    OpNode& conv = g.ops[pi];
    if (conv.type != "Conv" || g.consumers(bn.in[0]).size() != 1) continue;
    TensorInfo& W = g.tensor(conv.in[1]);
    if (!W.is_init || W.dims.size() != 4) continue;
    const auto gam = as_f32(g.tensor(bn.in[1]));
    const auto beta = as_f32(g.tensor(bn.in[2]));
    const auto mean = as_f32(g.tensor(bn.in[3]));
    const auto var = as_f32(g.tensor(bn.in[4]));
    const float eps = bn.p.epsilon;
    auto w = as_f32(W);
    const size_t co = (size_t)W.dims[0];
    const size_t per = w.size() / co;
    std::vector<float> oldb;
    const bool has_b = conv.in.size() > 2 && !conv.in[2].empty();
    if (has_b) oldb = as_f32(g.tensor(conv.in[2]));
    std::vector<float> nb(co);
    for (size_t c = 0; c < co; ++c) {
      const double std_inv = 1.0 / sqrt((double)var[c] + (double)eps);
      const double sf = (double)gam[c] * std_inv;
      for (size_t k = 0; k < per; ++k) w[c * per + k] = (float)((double)w[c * per + k] * sf);
      const double ob = has_b ? (double)oldb[c] : 0.0;
      nb[c] = (float)((ob - (double)mean[c]) * sf + (double)beta[c]);
    }
    set_f32(W, w);
    std::string bname = has_b ? conv.in[2] : conv.in[1] + "_bias_folded";
    TensorInfo& B = g.t[bname];
    B.dims = {(int64_t)co};
    set_f32(B, nb);
    if (has_b)
      conv.in[2] = bname;
    else
      conv.in.resize(3), conv.in[2] = bname;
    g.t.erase(conv.out[0]);
    conv.out[0] = bn.out[0];
    g.ops.erase(g.ops.begin() + i);
    --i;
    ++folded;
  }
  return folded;
}

// --------------------------------------------------------------------------
// convert_nchw_to_nhwc (graph.rs:248-290): conv weights [Co,Ci,kh,kw] ->
// [kh,kw,Ci,Co] (perm [2,3,1,0]); every other 4-D shape [N,C,H,W] ->
// [N,H,W,C] (4-D initializers that are not conv weights have their data
// permuted with them).  Ops whose meaning depends on the memory order are
// rewritten so the graph still computes what the NCHW model means; the
// reference changes the shapes only, so its NHWC graphs of such models
// compute something else:
//  * Concat / Split / Softmax / Slice axes and Transpose perms of 4-D
//    tensors are renumbered to the NHWC axes (logical axis 1 -> 3, 2 -> 1,
//    3 -> 2);
//  * a Reshape / Flatten that reads a 4-D tensor reads it through a
//    Transpose to NCHW order, and one that writes a 4-D tensor writes NCHW
//    order followed by a Transpose to NHWC (skipped when the permutation
//    only moves dimensions of size 1, where the bytes are the same);
//  * a constant operand of lower rank broadcast against a 4-D tensor in an
//    Add / Mul / Sub / Div becomes a 4-D NHWC initializer.
// --------------------------------------------------------------------------
namespace {
constexpr int kPhysOfLogical[4] = {0, 3, 1, 2};  // NCHW axis -> NHWC position
constexpr int kLogicalOfPhys[4] = {0, 2, 3, 1};  // NHWC position -> NCHW axis

// permute the bytes of a row-major tensor of dims d (esize es) by perm:
// output axis k is input axis perm[k]
std::vector<uint8_t> permute_bytes(const std::vector<uint8_t>& src, const std::vector<int64_t>& d,
                                   const std::vector<int>& perm, int es) {
  const size_t r = d.size();
  std::vector<int64_t> od(r), is(r, 1), os(r, 1);
  for (size_t k = 0; k < r; ++k) od[k] = d[perm[k]];
  for (int64_t k = (int64_t)r - 2; k >= 0; --k) {
    is[k] = is[k + 1] * d[k + 1];
    os[k] = os[k + 1] * od[k + 1];
  }
  int64_t total = 1;
  for (auto v : d) total *= v;
  std::vector<uint8_t> out(src.size());
  for (int64_t o = 0; o < total; ++o) {
    int64_t rem = o, si = 0;
    for (size_t k = 0; k < r; ++k) {
      const int64_t c = rem / os[k];
      rem -= c * os[k];
      si += c * is[perm[k]];
    }
    memcpy(&out[o * es], &src[si * es], es);
  }
  return out;
}

// true when permuting dims d by perm keeps every dimension above 1 in its
// order, i.e. the row-major bytes do not move
bool permutation_is_trivial(const std::vector<int64_t>& d, const std::vector<int>& perm) {
  int last = -1;
  for (int a : perm) {
    if (d[a] == 1) continue;
    if (a < last) return false;
    last = a;
  }
  return true;
}
}  // namespace

void convert_nchw_to_nhwc(GraphIR& g) {
  std::set<std::string> weights;
  for (auto& op : g.ops)
    if (op.type == "Conv" && op.in.size() >= 2 && g.has(op.in[1]) && g.tensor(op.in[1]).is_init)
      weights.insert(op.in[1]);
  for (auto& wn : weights) {
    TensorInfo& W = g.tensor(wn);
    if (W.dims.size() != 4) continue;
    const int64_t co = W.dims[0], ci = W.dims[1], kh = W.dims[2], kw = W.dims[3];
    const int es = dtype_size(W.dtype);
    std::vector<uint8_t> out(W.data.size());
    for (int64_t o = 0; o < co; ++o)
      for (int64_t i = 0; i < ci; ++i)
        for (int64_t y = 0; y < kh; ++y)
          for (int64_t x = 0; x < kw; ++x) {
            const int64_t src = ((o * ci + i) * kh + y) * kw + x;
            const int64_t dst = ((y * kw + x) * ci + i) * co + o;
            memcpy(&out[dst * es], &W.data[src * es], es);
          }
    W.data.swap(out);
    W.dims = {kh, kw, ci, co};
  }
  // the NCHW dims of every tensor before conversion
  std::map<std::string, std::vector<int64_t>> nchw;
  for (auto& kv : g.t) nchw[kv.first] = kv.second.dims;
  for (auto& kv : g.t) {
    if (weights.count(kv.first) || kv.second.dims.size() != 4) continue;
    auto& d = kv.second.dims;
    if (kv.second.is_init && !kv.second.data.empty())
      kv.second.data = permute_bytes(kv.second.data, d, {0, 2, 3, 1}, dtype_size(kv.second.dtype));
    d = {d[0], d[2], d[3], d[1]};
  }
  auto rank_of = [&](const std::string& n) { return nchw.count(n) ? nchw[n].size() : g.tensor(n).dims.size(); };
  std::vector<OpNode> out;
  out.reserve(g.ops.size());
  auto transpose_op = [&](const std::string& name, const std::string& x, const std::string& y,
                          const std::vector<int>& perm) {
    OpNode t;
    t.name = name;
    t.type = "LayoutTranspose";  // a pure byte permutation (no f16 value round trip)
    t.in = {x};
    t.out = {y};
    t.p.kind = DW_OP_TRANSPOSE;
    for (int k = 0; k < 4; ++k) t.p.perm[k] = perm[k];
    out.push_back(t);
  };
  for (OpNode op : g.ops) {
    const bool in4 = !op.in.empty() && rank_of(op.in[0]) == 4;
    if ((op.type == "Concat" || op.type == "Split" || op.type == "Softmax") && in4 && op.p.axis >= 0 &&
        op.p.axis < 4) {
      op.p.axis = kPhysOfLogical[op.p.axis];
    } else if (op.type == "Slice" && in4) {
      for (int k = 0; k < op.p.num_slice_axes; ++k) op.p.slice_axes[k] = kPhysOfLogical[op.p.slice_axes[k]];
    } else if (op.type == "Transpose" && in4) {
      // physical output axis j is logical output axis L[j], which is logical
      // input axis perm[L[j]], found at NHWC position P[perm[L[j]]]
      int q[4];
      for (int j = 0; j < 4; ++j) q[j] = kPhysOfLogical[op.p.perm[kLogicalOfPhys[j]]];
      for (int j = 0; j < 4; ++j) op.p.perm[j] = q[j];
    } else if ((op.type == "Reshape" || op.type == "Flatten") && !op.in.empty() && !op.out.empty()) {
      const std::string x = op.in[0], y = op.out[0];
      if (rank_of(x) == 4 && !permutation_is_trivial(g.tensor(x).dims, {0, 3, 1, 2})) {
        const std::string xr = x + "__nchw";
        if (!g.has(xr)) {
          TensorInfo ti = g.tensor(x);
          ti.is_init = false;
          ti.data.clear();
          ti.dims = nchw[x];
          g.t[xr] = ti;
          transpose_op(op.name + "__to_nchw", x, xr, {0, 3, 1, 2});
        }
        op.in[0] = xr;
      }
      if (rank_of(y) == 4 && !permutation_is_trivial(nchw[y], {0, 2, 3, 1})) {
        const std::string yr = y + "__nchw";
        TensorInfo ti = g.tensor(y);
        ti.dims = nchw[y];
        g.t[yr] = ti;
        op.out[0] = yr;
        out.push_back(op);
        transpose_op(op.name + "__to_nhwc", yr, y, {0, 2, 3, 1});
        continue;
      }
    } else if ((op.type == "Add" || op.type == "Mul" || op.type == "Sub" || op.type == "Div") &&
               op.out.size() == 1 && rank_of(op.out[0]) == 4) {
      for (auto& in : op.in) {
        if (rank_of(in) == 4) continue;
        TensorInfo& ti = g.tensor(in);
        if (ti.numel() == 1) continue;  // a scalar broadcasts the same either way
        if (!ti.is_init) fail(DW_ERR_UNSUPPORTED, "nhwc: " + op.name + " broadcasts a lower-rank activation");
        // ONNX aligns trailing dims: pad to 4-D NCHW, then permute to NHWC
        std::vector<int64_t> d4 = ti.dims;
        while (d4.size() < 4) d4.insert(d4.begin(), 1);
        const std::string n4 = in + "__nhwc";
        if (!g.has(n4)) {
          TensorInfo t4 = ti;
          t4.data = permute_bytes(ti.data, d4, {0, 2, 3, 1}, dtype_size(ti.dtype));
          t4.dims = {d4[0], d4[2], d4[3], d4[1]};
          g.t[n4] = t4;
        }
        in = n4;
      }
    }
    out.push_back(op);
  }
  g.ops.swap(out);
}

// --------------------------------------------------------------------------
// apply_fusion_passes (fusion.rs:42-348).  As in the reference, all three
// passes look at one snapshot of the op list (producer = last op writing a
// tensor, consumers = ops reading it), record replacements and removals, and
// apply them at the end:
//  1. Relu whose input is written by a Conv read by nothing else: the Conv
//     becomes "<conv>_fused_relu" writing the Relu's output (fusion.rs:65-123).
//     The reference keeps plain Conv2d params there and so loses the ReLU;
//     here has_relu = 1 carries it (the runtimes apply it after the bias).
//  2. Mul(x, Sigmoid(x)) with the Sigmoid read only by that Mul becomes
//     SiLU "<mul>_silu" (fusion.rs:125-190).  The reference inspects the
//     first operand's producer and gives up when it is not the Sigmoid, so
//     Mul(x, s) with x written by an op is never fused there; both operand
//     orders are matched here.
//  3. Requantize writing tensor t, with the closest earlier group-1,
//     bias-free Conv also writing t, becomes Conv2dRequantReluI8
//     "<conv>_fused_qrelu" (+ the Relu when it is t's only other reader)
//     (fusion.rs:192-334).
// Tensors no op reads or writes afterwards (and that are not graph inputs or
// outputs) are dropped from the IR.
// --------------------------------------------------------------------------
namespace {
void drop_unreferenced(GraphIR& g) {
  std::set<std::string> used(g.inputs.begin(), g.inputs.end());
  used.insert(g.outputs.begin(), g.outputs.end());
  for (auto& op : g.ops) {
    used.insert(op.in.begin(), op.in.end());
    used.insert(op.out.begin(), op.out.end());
  }
  for (auto it = g.t.begin(); it != g.t.end();) {
    if (!it->second.is_init && !used.count(it->first))
      it = g.t.erase(it);
    else
      ++it;
  }
}
}  // namespace

int apply_fusion_passes(GraphIR& g, bool conv_relu, bool silu, bool conv_requant) {
  const size_t n = g.ops.size();
  std::map<std::string, size_t> producer;
  std::map<std::string, std::vector<size_t>> consumers;
  for (size_t i = 0; i < n; ++i)
    for (auto& o : g.ops[i].out) producer[o] = i;
  for (size_t i = 0; i < n; ++i)
    for (auto& in : g.ops[i].in) consumers[in].push_back(i);
  auto n_consumers = [&](const std::string& t) {
    auto it = consumers.find(t);
    return it == consumers.end() ? (size_t)0 : it->second.size();
  };
  std::set<size_t> remove;
  std::vector<std::pair<size_t, OpNode>> fused;

  // pass 1: Conv + Relu
  for (size_t i = 0; conv_relu && i < n; ++i) {
    const OpNode& op = g.ops[i];
    if (remove.count(i) || op.type != "Relu" || op.in.empty()) continue;
    auto pr = producer.find(op.in[0]);
    if (pr == producer.end()) continue;
    const OpNode& conv = g.ops[pr->second];
    if (conv.type != "Conv" || n_consumers(op.in[0]) != 1) continue;
    remove.insert(i);
    OpNode f = conv;
    f.name = conv.name + "_fused_relu";
    f.out = op.out;
    f.p.has_relu = 1;
    fused.push_back({pr->second, f});
  }
  // pass 2: Mul(x, Sigmoid(x)) -> SiLU
  for (size_t i = 0; silu && i < n; ++i) {
    const OpNode& op = g.ops[i];
    if (remove.count(i) || op.type != "Mul" || op.in.size() != 2) continue;
    int sig = -1;
    std::string x;
    for (int k = 0; k < 2 && sig < 0; ++k) {
      auto pr = producer.find(op.in[k]);
      if (pr == producer.end()) continue;
      const OpNode& s = g.ops[pr->second];
      if (s.type == "Sigmoid" && !s.in.empty() && s.in[0] == op.in[1 - k]) {
        sig = (int)pr->second;
        x = op.in[1 - k];
      }
    }
    if (sig < 0 || remove.count((size_t)sig)) continue;
    const std::string& sout = g.ops[sig].out[0];
    if (n_consumers(sout) != 1 || g.is_output(sout)) continue;
    remove.insert((size_t)sig);
    OpNode f;
    f.name = op.name + "_silu";
    f.type = "SiLU";
    f.in = {x};
    f.out = op.out;
    f.p.kind = DW_OP_NONE;
    fused.push_back({i, f});
  }
  // pass 3: INT8 Conv + Requantize (+ Relu)
  for (size_t i = 0; conv_requant && i < n; ++i) {
    const OpNode& op = g.ops[i];
    if (remove.count(i) || op.type != "Requantize" || op.out.empty()) continue;
    const std::string fin = op.out[0];
    int ci = -1;
    for (int k = (int)i - 1; k >= 0; --k) {
      const OpNode& prev = g.ops[k];
      if (prev.type == "Conv" && !prev.out.empty() && prev.out[0] == fin && prev.p.kind == DW_OP_CONV2D) {
        ci = k;
        break;
      }
    }
    if (ci < 0 || remove.count((size_t)ci)) continue;
    const OpNode& conv = g.ops[ci];
    if (conv.in.size() < 2 || conv.p.group != 1 || op.p.kind != DW_OP_REQUANTIZE) continue;
    int relu = -1;
    auto cs = consumers.find(fin);
    if (cs != consumers.end()) {
      std::vector<size_t> live;
      for (size_t c : cs->second)
        if (c != i && !remove.count(c)) live.push_back(c);
      if (live.size() == 1 && g.ops[live[0]].type == "Relu") relu = (int)live[0];
    }
    if (conv.in.size() > 2 && !conv.in[2].empty()) continue;  // biased INT8 convs are not fused
    OpNode f;
    f.name = conv.name + "_fused_qrelu";
    f.type = "Conv2dRequantReluI8";
    f.in = conv.in;
    f.out = {relu >= 0 ? (g.ops[relu].out.empty() ? fin : g.ops[relu].out[0]) : fin};
    f.p = conv.p;
    f.p.kind = DW_OP_CONV2D_REQUANT_RELU_I8;
    f.p.scale = op.p.scale;
    f.p.has_relu = relu >= 0 ? 1 : 0;
    remove.insert(i);
    if (relu >= 0) remove.insert((size_t)relu);
    fused.push_back({(size_t)ci, f});
  }
  for (auto& kv : fused) g.ops[kv.first] = kv.second;
  std::vector<size_t> rm(remove.begin(), remove.end());
  for (auto it = rm.rbegin(); it != rm.rend(); ++it) g.ops.erase(g.ops.begin() + *it);
  drop_unreferenced(g);
  return (int)fused.size();
}

int fuse_silu(GraphIR& g) { return apply_fusion_passes(g, false, true, false); }

void convert_to_f16(GraphIR& g) {
  if (g.dtype != DW_GRAPH_F32) fail(DW_ERR_RUNTIME, "convert_to_f16 needs an F32 graph");
  for (auto& kv : g.t) {
    TensorInfo& ti = kv.second;
    if (ti.dtype != DW_DTYPE_F32) continue;
    if (ti.is_init) {
      std::vector<uint8_t> out(ti.data.size() / 2);
      for (size_t i = 0; i < ti.data.size() / 4; ++i) {
        float f;
        memcpy(&f, &ti.data[i * 4], 4);
        const uint16_t h = f16_from_f32(f);
        memcpy(&out[i * 2], &h, 2);
      }
      ti.data.swap(out);
    }
    ti.dtype = DW_DTYPE_F16;
  }
  g.dtype = DW_GRAPH_F16;
}

// --------------------------------------------------------------------------
// QDQ quantizer.  Input: an F32 NHWC graph with calibrated ranges on its
// activations.  Output (DW_GRAPH_QU8):
//  * activations u8 with zero point 128 and the reference's symmetric
//    calibration scale absmax / 127 (QuantScale::from_range,
//    crates/dragonwing-core/src/quantization.rs:85-89);
//  * tensors joined by Concat / Split / MaxPool / Resize share one scale
//    (these ops then move bytes only);
//  * Conv -> QLinearConv with s8 weights quantized per output channel
//    (PerChannelScale::from_weights + quantize_weights_per_channel,
//    quantize.rs:344-368: q = clamp(round(w * (1/s)))), int32 bias
//    rint(b / (x_scale * w_scale[c])), and M[c] = x_scale*w_scale[c]/y_scale;
//  * SiLU after a conv -> QLinearLUT on the conv's u8 pre-activation;
//  * Add -> QLinearAdd;
//  * convs named in keep_f16 stay fp16 (f16 weights): a u8 input gets a
//    DequantizeLinear, an f16 result consumed by u8 ops gets a
//    QuantizeLinear (then the SiLU table).
// --------------------------------------------------------------------------
struct UF {
  std::map<std::string, std::string> parent;
  std::string find(const std::string& a) {
    auto it = parent.find(a);
    if (it == parent.end() || it->second == a) return a;
    std::string r = find(it->second);
    parent[a] = r;
    return r;
  }
  void join(const std::string& a, const std::string& b) {
    std::string ra = find(a), rb = find(b);
    if (ra != rb) parent[ra] = rb;
  }
};

float sym_scale(float mn, float mx) {
  const float a = fmaxf(fabsf(mn), fabsf(mx));
  return a > 0.0f ? a / 127.0f : 1.0f;
}

void quantize_qdq(GraphIR& g, const std::set<std::string>& keep_f16) {
  if (g.dtype != DW_GRAPH_F32) fail(DW_ERR_RUNTIME, "quantize_qdq needs an F32 graph");
  fuse_silu(g);
  // --- shared-scale groups
  UF uf;
  auto moves_bytes = [](const std::string& ty) {
    return ty == "Concat" || ty == "Split" || ty == "MaxPool" || ty == "Resize" || ty == "Flatten" ||
           ty == "Reshape" || ty == "Transpose" || ty == "LayoutTranspose" || ty == "Slice";
  };
  for (auto& op : g.ops) {
    if (moves_bytes(op.type)) {
      for (auto& i : op.in)
        if (!g.tensor(i).is_init)
          for (auto& o : op.out) uf.join(i, o);
    }
  }
  bool qdq_model = false;  // quantization fixed by an imported QDQ model
  for (auto& kv : g.t) qdq_model = qdq_model || kv.second.q_fixed || kv.second.prequant;
  // Tensors that stay f16: graph inputs, outputs of kept convs (and of f16
  // concats of those).
  std::set<std::string> f16t(g.inputs.begin(), g.inputs.end());
  for (auto& in : g.inputs) g.tensor(in).dtype = DW_DTYPE_F16;
  // The float tail after the kept fp16 layers (a detect head's layout ops,
  // DFL softmax, box arithmetic, sigmoid): ops of these types that read
  // only f16 tensors and constants stay f16.
  static const std::set<std::string> tail_types = {"Concat", "Split", "Reshape", "Flatten", "Transpose",
                                                   "LayoutTranspose", "Slice", "Softmax", "Sigmoid", "Mul",
                                                   "Add", "Sub", "Div", "Clip", "Relu", "AveragePool",
                                                   "YoloDetect"};
  auto reads_f16_only = [&](const OpNode& op) {
    bool any = false;
    for (auto& i : op.in) {
      if (i.empty() || g.tensor(i).is_init) continue;
      if (!f16t.count(i)) return false;
      any = true;
    }
    return any;
  };
  for (auto& op : g.ops) {
    if (op.type == "Conv" && (keep_f16.count(op.name) ||
                              (qdq_model && op.in.size() > 1 && !g.tensor(op.in[1]).prequant)))
      f16t.insert(op.out[0]);
    else if (tail_types.count(op.type) && reads_f16_only(op))
      for (auto& o : op.out) f16t.insert(o);
  }
  // group ranges
  std::map<std::string, std::pair<float, float>> grange;
  for (auto& kv : g.t) {
    const TensorInfo& ti = kv.second;
    if (ti.is_init || !ti.has_range) continue;
    const std::string r = uf.find(kv.first);
    auto it = grange.find(r);
    if (it == grange.end())
      grange[r] = {ti.rmin, ti.rmax};
    else
      it->second = {std::min(it->second.first, ti.rmin), std::max(it->second.second, ti.rmax)};
  }
  // quantization fixed by the model (QDQ import), per shared-scale group
  std::map<std::string, std::pair<float, int>> gfixed;
  for (auto& kv : g.t) {
    const TensorInfo& ti = kv.second;
    if (ti.is_init || !ti.q_fixed) continue;
    const std::string r = uf.find(kv.first);
    auto it = gfixed.find(r);
    if (it == gfixed.end())
      gfixed[r] = {ti.scale, ti.zp};
    else if (it->second.first != ti.scale || it->second.second != ti.zp)
      fail(DW_ERR_UNSUPPORTED, "quantize_qdq: '" + kv.first + "' must share its quantization with the tensors "
                               "it is concatenated, split, pooled or resized with");
  }
  auto qscale = [&](const std::string& name) -> float {
    auto f = gfixed.find(uf.find(name));
    if (f != gfixed.end()) return f->second.first;
    auto it = grange.find(uf.find(name));
    if (it == grange.end()) fail(DW_ERR_RUNTIME, "no calibration range for '" + name + "'");
    return sym_scale(it->second.first, it->second.second);
  };
  auto qzp = [&](const std::string& name) -> int {
    auto f = gfixed.find(uf.find(name));
    return f != gfixed.end() ? f->second.second : 128;
  };
  auto make_u8 = [&](const std::string& name) {
    TensorInfo& ti = g.tensor(name);
    const float sc = qscale(name);
    const int zp = qzp(name);
    ti.dtype = DW_DTYPE_U8;
    ti.has_q = true;
    ti.scale = sc;
    ti.zp = zp;
  };

  std::vector<OpNode> out;
  std::map<std::string, std::string> as_u8, as_f16;  // converted twins
  auto add_tensor_like = [&](const std::string& src, const std::string& name, int dtype) {
    TensorInfo ti;
    ti.dims = g.tensor(src).dims;
    ti.dtype = dtype;
    g.t[name] = ti;
  };
  // u8 view of tensor x (x is f16): QuantizeLinear with x's own range.
  auto need_u8 = [&](const std::string& x) -> std::string {
    if (!f16t.count(x)) return x;
    auto it = as_u8.find(x);
    if (it != as_u8.end()) return it->second;
    const std::string q = x + "_q";
    add_tensor_like(x, q, DW_DTYPE_U8);
    TensorInfo& tq = g.tensor(q);
    tq.has_q = true;
    tq.scale = qscale(x);
    tq.zp = qzp(x);
    OpNode op;
    op.name = x + "_quantize";
    op.type = "QuantizeLinear";
    op.in = {x};
    op.out = {q};
    op.p.kind = DW_OP_QUANTIZE_LINEAR;
    out.push_back(op);
    as_u8[x] = q;
    return q;
  };
  auto need_f16 = [&](const std::string& x) -> std::string {
    if (f16t.count(x)) return x;
    auto it = as_f16.find(x);
    if (it != as_f16.end()) return it->second;
    const std::string d = x + "_dq";
    add_tensor_like(x, d, DW_DTYPE_F16);
    OpNode op;
    op.name = x + "_dequantize";
    op.type = "DequantizeLinear";
    op.in = {x};
    op.out = {d};
    op.p.kind = DW_OP_DEQUANTIZE_LINEAR;
    out.push_back(op);
    as_f16[x] = d;
    return d;
  };

  for (size_t oi = 0; oi < g.ops.size(); ++oi) {
    OpNode op = g.ops[oi];
    if (tail_types.count(op.type) && !op.out.empty() && f16t.count(op.out[0])) {
      // f16 op of the float tail: its float constants become f16
      for (auto& i : op.in) {
        if (i.empty()) continue;
        TensorInfo& ti = g.tensor(i);
        if (!ti.is_init || ti.dtype != DW_DTYPE_F32) continue;
        std::vector<uint8_t> h(ti.data.size() / 2);
        for (size_t e = 0; e < ti.data.size() / 4; ++e) {
          float f;
          memcpy(&f, &ti.data[e * 4], 4);
          const uint16_t b = f16_from_f32(f);
          memcpy(&h[e * 2], &b, 2);
        }
        ti.data.swap(h);
        ti.dtype = DW_DTYPE_F16;
      }
      for (auto& o : op.out) g.tensor(o).dtype = DW_DTYPE_F16;
      out.push_back(op);
      continue;
    }
    if (op.type == "Conv") {
      TensorInfo& W = g.tensor(op.in[1]);
      if (W.dims.size() != 4) fail(DW_ERR_UNSUPPORTED, "quantize: conv weight must be 4-D (HWIO)");
      // a QDQ model leaves the convs it keeps in float with float weights
      const bool keep = keep_f16.count(op.name) != 0 || (qdq_model && !W.prequant);
      if (keep) {
        op.in[0] = need_f16(op.in[0]);
        // weights / bias -> f16
        for (size_t k = 1; k < op.in.size(); ++k) {
          if (op.in[k].empty()) continue;
          TensorInfo& ti = g.tensor(op.in[k]);
          if (ti.dtype == DW_DTYPE_F32) {
            std::vector<uint8_t> h(ti.data.size() / 2);
            for (size_t e = 0; e < ti.data.size() / 4; ++e) {
              float f;
              memcpy(&f, &ti.data[e * 4], 4);
              const uint16_t b = f16_from_f32(f);
              memcpy(&h[e * 2], &b, 2);
            }
            ti.data.swap(h);
            ti.dtype = DW_DTYPE_F16;
          }
        }
        g.tensor(op.out[0]).dtype = DW_DTYPE_F16;
        out.push_back(op);
        continue;
      }
      const std::string x = need_u8(op.in[0]);
      const TensorInfo& X = g.tensor(x);
      const int64_t kh = W.dims[0], kw = W.dims[1], ci = W.dims[2], co = W.dims[3];
      auto w = as_f32(W);
      std::vector<float> ws(co);
      std::vector<int8_t> wq(w.size());
      if (W.prequant) {
        // the model's own int8 weights and per-output-channel scales
        if (!(W.q_axis == 0 || (W.q_axis < 0 && W.ch_scales.size() == 1)))
          fail(DW_ERR_UNSUPPORTED, "quantize_qdq: weight scales of " + op.name + " are not per output channel");
        for (int64_t c = 0; c < co; ++c) ws[c] = W.ch_scales.size() == 1 ? W.ch_scales[0] : W.ch_scales[c];
        for (size_t e = 0; e < w.size(); ++e) wq[e] = (int8_t)w[e];
      } else {
        for (int64_t c = 0; c < co; ++c) {
          float am = 0.0f;
          for (int64_t k = 0; k < kh * kw * ci; ++k) am = fmaxf(am, fabsf(w[k * co + c]));
          ws[c] = am > 0.0f ? am / 127.0f : 1.0f;
          const float inv = 1.0f / ws[c];
          for (int64_t k = 0; k < kh * kw * ci; ++k) {
            float r = roundf(w[k * co + c] * inv);
            r = r < -128.0f ? -128.0f : (r > 127.0f ? 127.0f : r);
            wq[k * co + c] = (int8_t)r;
          }
        }
      }
      W.data.assign((const uint8_t*)wq.data(), (const uint8_t*)wq.data() + wq.size());
      W.dtype = DW_DTYPE_I8;
      W.ch_scales = ws;
      if (op.in.size() > 2 && !op.in[2].empty()) {
        TensorInfo& Bt = g.tensor(op.in[2]);
        auto b = as_f32(Bt);
        std::vector<int32_t> bq(co);
        for (int64_t c = 0; c < co; ++c) {
          const double s = (double)(X.scale * ws[c]);
          // a QDQ model's int32 bias is q * its scale (input scale x weight
          // scale, so q itself comes back)
          const double bv = Bt.prequant ? (double)b[c] * (double)(Bt.ch_scales.size() == 1 ? Bt.ch_scales[0]
                                                                                          : Bt.ch_scales[c])
                                        : (double)b[c];
          double r = nearbyint(bv / s);
          r = std::min(std::max(r, -2147483648.0), 2147483647.0);
          bq[c] = (int32_t)r;
        }
        Bt.data.assign((const uint8_t*)bq.data(), (const uint8_t*)bq.data() + bq.size() * 4);
        Bt.dtype = DW_DTYPE_I32;
      }
      op.type = "QLinearConv";
      op.p.kind = DW_OP_QLINEAR_CONV;
      op.in[0] = x;
      make_u8(op.out[0]);
      out.push_back(op);
      continue;
    }
    if (op.type == "SiLU") {
      const std::string x = need_u8(op.in[0]);
      make_u8(op.out[0]);
      op.type = "QLinearLUT";
      op.p.kind = DW_OP_QLINEAR_LUT;
      op.p.act = DW_ACT_SILU;
      op.in = {x};
      out.push_back(op);
      continue;
    }
    if (op.type == "Add") {
      op.in = {need_u8(op.in[0]), need_u8(op.in[1])};
      make_u8(op.out[0]);
      op.type = "QLinearAdd";
      op.p.kind = DW_OP_QLINEAR_ADD;
      out.push_back(op);
      continue;
    }

    if (moves_bytes(op.type)) {
      for (auto& i : op.in)
        if (!g.tensor(i).is_init) i = need_u8(i);
      for (auto& o : op.out) make_u8(o);
      out.push_back(op);
      continue;
    }
    if (op.type == "GlobalAveragePool") {
      op.in[0] = need_u8(op.in[0]);
      make_u8(op.out[0]);
      op.type = "QLinearGlobalAveragePool";
      out.push_back(op);
      continue;
    }
    if (op.type == "Gemm") {
      // QGemm: B quantized per output column (symmetric s8, as the convs'
      // output channels), stored [1][1][k][n] so it runs as a 1x1
      // QLinearConv over the rows of A; bias rint(b / (xs * ws[j]))
      if (op.p.trans_a) fail(DW_ERR_UNSUPPORTED, "quantize_qdq: Gemm transA");
      TensorInfo& W = g.tensor(op.in[1]);
      if (!W.is_init || W.dims.size() != 2 || W.dtype != DW_DTYPE_F32)
        fail(DW_ERR_UNSUPPORTED, "quantize_qdq: Gemm B must be a 2-D f32 initializer");
      const bool tb = op.p.trans_b != 0;
      const int64_t k = tb ? W.dims[1] : W.dims[0], n = tb ? W.dims[0] : W.dims[1];
      auto w = as_f32(W);
      std::vector<float> wk((size_t)(k * n));
      for (int64_t p = 0; p < k; ++p)
        for (int64_t j = 0; j < n; ++j) wk[p * n + j] = tb ? w[j * k + p] : w[p * n + j];
      const std::string x = need_u8(op.in[0]);
      const TensorInfo& X = g.tensor(x);
      std::vector<float> ws(n);
      std::vector<int8_t> wq(wk.size());
      if (W.prequant) {
        // scales per output column: along B's n dimension (axis 1, or 0 with transB)
        const int n_axis = tb ? 0 : 1;
        if (!(W.q_axis == n_axis || (W.q_axis < 0 && W.ch_scales.size() == 1)))
          fail(DW_ERR_UNSUPPORTED, "quantize_qdq: weight scales of " + op.name + " are not per output column");
        for (int64_t j = 0; j < n; ++j) ws[j] = W.ch_scales.size() == 1 ? W.ch_scales[0] : W.ch_scales[j];
        for (size_t e = 0; e < wk.size(); ++e) wq[e] = (int8_t)wk[e];
      } else {
        for (int64_t j = 0; j < n; ++j) {
          float am = 0.0f;
          for (int64_t p = 0; p < k; ++p) am = fmaxf(am, fabsf(wk[p * n + j]));
          ws[j] = am > 0.0f ? am / 127.0f : 1.0f;
          const float inv = 1.0f / ws[j];
          for (int64_t p = 0; p < k; ++p) {
            float r = roundf(wk[p * n + j] * inv);
            r = r < -128.0f ? -128.0f : (r > 127.0f ? 127.0f : r);
            wq[p * n + j] = (int8_t)r;
          }
        }
      }
      W.data.assign((const uint8_t*)wq.data(), (const uint8_t*)wq.data() + wq.size());
      W.dtype = DW_DTYPE_I8;
      W.dims = {1, 1, k, n};
      W.ch_scales = ws;
      if (op.in.size() > 2 && !op.in[2].empty()) {
        TensorInfo& Bt = g.tensor(op.in[2]);
        auto b = as_f32(Bt);
        if ((int64_t)b.size() != n) fail(DW_ERR_UNSUPPORTED, "quantize_qdq: Gemm bias must have n values");
        std::vector<int32_t> bq(n);
        for (int64_t j = 0; j < n; ++j) {
          const double sc = (double)(X.scale * ws[j]);
          const double bv = Bt.prequant ? (double)b[j] * (double)(Bt.ch_scales.size() == 1 ? Bt.ch_scales[0]
                                                                                           : Bt.ch_scales[j])
                                        : (double)b[j];
          double r = nearbyint(bv / sc);
          r = std::min(std::max(r, -2147483648.0), 2147483647.0);
          bq[j] = (int32_t)r;
        }
        Bt.data.assign((const uint8_t*)bq.data(), (const uint8_t*)bq.data() + bq.size() * 4);
        Bt.dtype = DW_DTYPE_I32;
      }
      op.type = "QGemm";
      op.p.kind = DW_OP_QLINEAR_CONV;
      op.p.kernel_shape[0] = op.p.kernel_shape[1] = 1;
      op.p.strides[0] = op.p.strides[1] = 1;
      for (int& pd : op.p.pads) pd = 0;
      op.p.trans_b = 0;
      op.in[0] = x;
      make_u8(op.out[0]);
      out.push_back(op);
      continue;
    }
    fail(DW_ERR_UNSUPPORTED, "quantize_qdq: op type '" + op.type + "' is not supported");
  }
  g.ops.swap(out);
  // graph outputs that ended up u8 stay u8 (the caller dequantizes);
  g.dtype = DW_GRAPH_QU8;
}

std::string to_json(const GraphIR& g) {
  std::ostringstream o;
  o << "{\"dtype\":" << g.dtype << ",\"inputs\":[";
  for (size_t i = 0; i < g.inputs.size(); ++i) o << (i ? "," : "") << '"' << jesc(g.inputs[i]) << '"';
  o << "],\"outputs\":[";
  for (size_t i = 0; i < g.outputs.size(); ++i) o << (i ? "," : "") << '"' << jesc(g.outputs[i]) << '"';
  o << "],\"tensors\":{";
  bool first = true;
  for (auto& kv : g.t) {
    const TensorInfo& ti = kv.second;
    o << (first ? "" : ",") << '"' << jesc(kv.first) << "\":{\"dims\":[";
    first = false;
    for (size_t i = 0; i < ti.dims.size(); ++i) o << (i ? "," : "") << ti.dims[i];
    o << "],\"dtype\":" << ti.dtype << ",\"init\":" << (ti.is_init ? "true" : "false");
    if (ti.has_q) o << ",\"scale\":" << fstr(ti.scale) << ",\"zp\":" << ti.zp;
    if (!ti.ch_scales.empty()) {
      o << ",\"ch_scales\":[";
      for (size_t i = 0; i < ti.ch_scales.size(); ++i) o << (i ? "," : "") << fstr(ti.ch_scales[i]);
      o << "]";
    }
    if (ti.has_range) o << ",\"range\":[" << fstr(ti.rmin) << "," << fstr(ti.rmax) << "]";
    o << "}";
  }
  o << "},\"ops\":[";
  for (size_t i = 0; i < g.ops.size(); ++i) {
    const OpNode& op = g.ops[i];
    const dw_op_params& p = op.p;
    o << (i ? "," : "") << "{\"name\":\"" << jesc(op.name) << "\",\"type\":\"" << jesc(op.type)
      << "\",\"inputs\":[";
    for (size_t k = 0; k < op.in.size(); ++k) o << (k ? "," : "") << '"' << jesc(op.in[k]) << '"';
    o << "],\"outputs\":[";
    for (size_t k = 0; k < op.out.size(); ++k) o << (k ? "," : "") << '"' << jesc(op.out[k]) << '"';
    o << "],\"kind\":" << p.kind << ",\"kernel_shape\":[" << p.kernel_shape[0] << ","
      << p.kernel_shape[1] << "],\"strides\":[" << p.strides[0] << "," << p.strides[1]
      << "],\"pads\":[" << p.pads[0] << "," << p.pads[1] << "," << p.pads[2] << "," << p.pads[3]
      << "],\"dilations\":[" << p.dilations[0] << "," << p.dilations[1] << "],\"group\":" << p.group
      << ",\"axis\":" << p.axis << ",\"split_sizes\":[";
    for (int k = 0; k < p.num_splits && k < 8; ++k) o << (k ? "," : "") << p.split_sizes[k];
    o << "],\"out_h\":" << p.out_h << ",\"out_w\":" << p.out_w << ",\"mode_nearest\":" << p.mode_nearest
      << ",\"scale\":" << fstr(p.scale) << ",\"scale_a_over_out\":" << fstr(p.scale_a_over_out)
      << ",\"scale_b_over_out\":" << fstr(p.scale_b_over_out) << ",\"has_relu\":" << p.has_relu
      << ",\"epsilon\":" << fstr(p.epsilon) << ",\"act\":" << p.act << ",\"trans_a\":" << p.trans_a
      << ",\"trans_b\":" << p.trans_b << ",\"clip_min\":" << fstr(p.clip_min)
      << ",\"clip_max\":" << fstr(p.clip_max) << ",\"reg_max\":" << p.reg_max << ",\"level_strides\":["
      << fstr(p.level_strides[0]) << "," << fstr(p.level_strides[1]) << "," << fstr(p.level_strides[2]) << ","
      << fstr(p.level_strides[3]) << "],\"perm\":[" << p.perm[0] << "," << p.perm[1] << "," << p.perm[2] << ","
      << p.perm[3] << "],\"slices\":[";
    for (int k = 0; k < p.num_slice_axes && k < 4; ++k)
      o << (k ? "," : "") << "[" << p.slice_axes[k] << "," << p.slice_starts[k] << "," << p.slice_ends[k] << ","
        << p.slice_steps[k] << "]";
    o << "]}";
  }
  o << "]}";
  return o.str();
}

}  // namespace
}  // namespace dw

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

static dw::GraphIR& G(dw_graph* g) {
  if (!g) dw::fail(DW_ERR_INVALID, "null graph");
  g->g.json.clear();
  return g->g;
}

extern "C" {

int dw_graph_create(int dtype, dw_graph** out) {
  API_BEGIN
  if (!out) dw::fail(DW_ERR_INVALID, "null out");
  if (dtype != DW_GRAPH_F32 && dtype != DW_GRAPH_F16 && dtype != DW_GRAPH_I8 && dtype != DW_GRAPH_QU8)
    dw::fail(DW_ERR_UNSUPPORTED, "graph dtype");
  dw_graph* g = new dw_graph();
  g->g.dtype = dtype;
  *out = g;
  API_END
}

void dw_graph_destroy(dw_graph* g) { delete g; }

int dw_graph_add_tensor(dw_graph* gh, const char* name, const int64_t* dims, int rank, int dtype) {
  API_BEGIN
  dw::GraphIR& g = G(gh);
  if (!name || !*name) dw::fail(DW_ERR_INVALID, "tensor needs a name");
  if (rank < 0 || rank > 4) dw::fail(DW_ERR_UNSUPPORTED, "rank > 4");
  if (dtype < 0 || dtype > DW_DTYPE_I32) dw::fail(DW_ERR_INVALID, "tensor dtype");
  dw::TensorInfo ti;
  for (int i = 0; i < rank; ++i) {
    if (dims[i] <= 0) dw::fail(DW_ERR_INVALID, std::string("non-positive dim in ") + name);
    ti.dims.push_back(dims[i]);
  }
  ti.dtype = dtype;
  g.t[name] = ti;
  API_END
}

int dw_graph_set_initializer(dw_graph* gh, const char* name, const void* data, size_t len) {
  API_BEGIN
  dw::GraphIR& g = G(gh);
  dw::TensorInfo& ti = g.tensor(name);
  const size_t want = (size_t)ti.numel() * dw::dtype_size(ti.dtype);
  if (len != want)
    dw::fail(DW_ERR_INVALID, std::string("initializer size mismatch for ") + name + ": expected " +
                                 std::to_string(want) + ", got " + std::to_string(len));
  ti.data.assign((const uint8_t*)data, (const uint8_t*)data + len);
  ti.is_init = true;
  API_END
}

int dw_graph_set_quant(dw_graph* gh, const char* name, float scale, int zero_point) {
  API_BEGIN
  dw::TensorInfo& ti = G(gh).tensor(name);
  if (!(scale > 0.0f)) dw::fail(DW_ERR_INVALID, "scale must be > 0");
  if (zero_point < 0 || zero_point > 255) dw::fail(DW_ERR_INVALID, "zero point must be in [0, 255]");
  ti.has_q = true;
  ti.scale = scale;
  ti.zp = zero_point;
  API_END
}

int dw_graph_set_channel_scales(dw_graph* gh, const char* name, const float* scales, size_t count) {
  API_BEGIN
  dw::TensorInfo& ti = G(gh).tensor(name);
  if (ti.dims.empty() || (int64_t)count != ti.dims.back())
    dw::fail(DW_ERR_INVALID, "channel scales must match the last (output-channel) dimension");
  for (size_t i = 0; i < count; ++i)
    if (!(scales[i] > 0.0f)) dw::fail(DW_ERR_INVALID, "channel scales must be > 0");
  ti.ch_scales.assign(scales, scales + count);
  API_END
}

int dw_graph_add_op(dw_graph* gh, const char* name, const char* op_type, const char* const* inputs,
                    int num_inputs, const char* const* outputs, int num_outputs,
                    const dw_op_params* params) {
  API_BEGIN
  dw::GraphIR& g = G(gh);
  if (!op_type) dw::fail(DW_ERR_INVALID, "null op_type");
  dw::OpNode op;
  op.name = name ? name : "";
  op.type = op_type;
  for (int i = 0; i < num_inputs; ++i) {
    std::string s = inputs[i] ? inputs[i] : "";
    if (!s.empty() && !g.has(s)) dw::fail(DW_ERR_RUNTIME, "op " + op.name + ": unknown input " + s);
    op.in.push_back(s);
  }
  for (int i = 0; i < num_outputs; ++i) {
    std::string s = outputs[i] ? outputs[i] : "";
    if (!g.has(s)) dw::fail(DW_ERR_RUNTIME, "op " + op.name + ": undeclared output " + s);
    op.out.push_back(s);
  }
  if (params) op.p = *params;
  g.ops.push_back(op);
  API_END
}

int dw_graph_set_io(dw_graph* gh, const char* const* inputs, int num_inputs, const char* const* outputs,
                    int num_outputs) {
  API_BEGIN
  dw::GraphIR& g = G(gh);
  g.inputs.clear();
  g.outputs.clear();
  for (int i = 0; i < num_inputs; ++i) {
    g.tensor(inputs[i]);
    g.inputs.push_back(inputs[i]);
  }
  for (int i = 0; i < num_outputs; ++i) {
    g.tensor(outputs[i]);
    g.outputs.push_back(outputs[i]);
  }
  API_END
}

int dw_graph_fold_batchnorm(dw_graph* gh) {
  API_BEGIN
  dw::fold_batchnorm(G(gh));
  API_END
}

int dw_graph_convert_nchw_to_nhwc(dw_graph* gh) {
  API_BEGIN
  dw::convert_nchw_to_nhwc(G(gh));
  API_END
}

int dw_graph_apply_fusion_passes(dw_graph* gh, int* num_fused) {
  API_BEGIN
  int n = dw::apply_fusion_passes(G(gh), true, true, true);
  if (num_fused) *num_fused = n;
  API_END
}

size_t dw_op_params_size(void) { return sizeof(dw_op_params); }

int dw_graph_convert_to_f16(dw_graph* gh) {
  API_BEGIN
  dw::convert_to_f16(G(gh));
  API_END
}

int dw_graph_set_activation_range(dw_graph* gh, const char* name, float min_v, float max_v) {
  API_BEGIN
  dw::TensorInfo& ti = G(gh).tensor(name);
  if (!(min_v <= max_v)) dw::fail(DW_ERR_INVALID, "range: min > max");
  ti.has_range = true;
  ti.rmin = min_v;
  ti.rmax = max_v;
  API_END
}

int dw_graph_quantize_qdq(dw_graph* gh, const char* const* keep_f16_ops, int num_keep) {
  API_BEGIN
  std::set<std::string> keep;
  for (int i = 0; i < num_keep; ++i) keep.insert(keep_f16_ops[i]);
  dw::quantize_qdq(G(gh), keep);
  API_END
}

const char* dw_graph_to_json(dw_graph* gh) {
  if (!gh) return "";
  if (gh->g.json.empty()) gh->g.json = dw::to_json(gh->g);
  return gh->g.json.c_str();
}

int dw_graph_get_initializer(dw_graph* gh, const char* name, const void** data, size_t* len) {
  API_BEGIN
  if (!gh) dw::fail(DW_ERR_INVALID, "null graph");
  const dw::TensorInfo& ti = gh->g.tensor(name);
  if (data) *data = ti.is_init ? ti.data.data() : nullptr;
  if (len) *len = ti.is_init ? ti.data.size() : 0;
  API_END
}

}  // extern "C"
