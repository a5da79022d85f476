// ONNX model loading: the protobuf wire format, the ModelProto / GraphProto /
// NodeProto / TensorProto / ValueInfoProto subset the reference reads
// (crates/dragonwing-onnx/src/proto.rs:129-271, model.rs:324-707), and the
// build of a graph IR from it (the reference's OpBuilder registry,
// builder.rs:386-420, for the op types this backend runs), plus the QDQ
// folding the reference lists as future work (docs/quantization.md:282).
//
// The result is an F32 graph in ONNX's NCHW layout, the form
// dragonwing_onnx hands to its passes: fold_batchnorm, convert_nchw_to_nhwc,
// then convert_to_f16 or calibration + quantize_qdq.  A QDQ model
// (QuantizeLinear / DequantizeLinear around the float ops) loads as the same
// float graph with its quantization fixed: every activation that passes
// through a QuantizeLinear -> DequantizeLinear pair carries that pair's
// scale and zero point, and every DequantizeLinear of an int8 weight or an
// int32 bias becomes an initializer holding the integers (as exact f32
// values) with their scales.  quantize_qdq then uses these instead of
// calibration ranges and re-quantizing, so the u8 graph computes with the
// model's own integers.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <deque>
#include <functional>
#include <map>
#include <set>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/dw_hip.h"
#include "backend.h"
#include "graph.h"

namespace dw {
namespace onnx {

// ---------------------------------------------------------------------------
// wire format
// ---------------------------------------------------------------------------
enum Wire { WT_VARINT = 0, WT_FIXED64 = 1, WT_LEN = 2, WT_FIXED32 = 5 };

struct Field {
  uint32_t num = 0;
  int wt = 0;
  uint64_t v = 0;              // varint / fixed values
  const uint8_t* p = nullptr;  // length-delimited payload
  size_t n = 0;
};

struct Reader {
  const uint8_t* p;
  const uint8_t* end;
  Reader(const uint8_t* b, size_t n) : p(b), end(b + n) {}
  bool more() const { return p < end; }
  uint64_t varint() {
    uint64_t r = 0;
    for (int shift = 0; shift < 64; shift += 7) {
      if (p >= end) fail(DW_ERR_INVALID, "onnx: unexpected end of input");
      const uint8_t b = *p++;
      r |= (uint64_t)(b & 0x7F) << shift;
      if (!(b & 0x80)) return r;
    }
    fail(DW_ERR_INVALID, "onnx: varint too long");
  }
  uint64_t fixed(int bytes) {
    if (end - p < bytes) fail(DW_ERR_INVALID, "onnx: unexpected end of input for a fixed field");
    uint64_t r = 0;
    for (int i = 0; i < bytes; ++i) r |= (uint64_t)p[i] << (8 * i);
    p += bytes;
    return r;
  }
  bool next(Field& f) {
    if (!more()) return false;
    const uint64_t tag = varint();
    f.num = (uint32_t)(tag >> 3);
    f.wt = (int)(tag & 7);
    f.p = nullptr;
    f.n = 0;
    f.v = 0;
    switch (f.wt) {
      case WT_VARINT: f.v = varint(); break;
      case WT_FIXED64: f.v = fixed(8); break;
      case WT_FIXED32: f.v = fixed(4); break;
      case WT_LEN: {
        const uint64_t n = varint();
        if (n > (uint64_t)(end - p))
          fail(DW_ERR_INVALID, "onnx: length-delimited field extends past the end");
        f.p = p;
        f.n = (size_t)n;
        p += n;
        break;
      }
      default: fail(DW_ERR_INVALID, "onnx: unknown wire type " + std::to_string(f.wt));
    }
    return true;
  }
};

std::string str(const Field& f) {
  if (f.wt != WT_LEN) fail(DW_ERR_INVALID, "onnx: expected a string");
  return std::string((const char*)f.p, f.n);
}
int64_t i64(const Field& f) {
  if (f.wt != WT_VARINT) fail(DW_ERR_INVALID, "onnx: expected a varint");
  return (int64_t)f.v;
}
// repeated int64: packed (length-delimited run of varints) or one varint
void ints(const Field& f, std::vector<int64_t>& out) {
  if (f.wt == WT_VARINT) {
    out.push_back((int64_t)f.v);
  } else if (f.wt == WT_LEN) {
    Reader r(f.p, f.n);
    while (r.more()) out.push_back((int64_t)r.varint());
  } else {
    fail(DW_ERR_INVALID, "onnx: unexpected wire type for ints");
  }
}
void floats(const Field& f, std::vector<float>& out) {
  if (f.wt == WT_FIXED32) {
    const uint32_t b = (uint32_t)f.v;
    float x;
    memcpy(&x, &b, 4);
    out.push_back(x);
  } else if (f.wt == WT_LEN) {
    if (f.n % 4) fail(DW_ERR_INVALID, "onnx: packed floats length not a multiple of 4");
    for (size_t i = 0; i < f.n; i += 4) {
      float x;
      memcpy(&x, f.p + i, 4);
      out.push_back(x);
    }
  } else {
    fail(DW_ERR_INVALID, "onnx: unexpected wire type for floats");
  }
}

// ---------------------------------------------------------------------------
// model
// ---------------------------------------------------------------------------
enum DataType { DT_FLOAT = 1, DT_UINT8 = 2, DT_INT8 = 3, DT_INT32 = 6, DT_INT64 = 7, DT_FLOAT16 = 10, DT_DOUBLE = 11 };

// bytes per element of a TensorProto data type (0: not one this reader holds)
inline int64_t dtype_bytes(int dt) {
  switch (dt) {
    case DT_UINT8: case DT_INT8: return 1;
    case DT_FLOAT16: return 2;
    case DT_FLOAT: case DT_INT32: return 4;
    case DT_INT64: case DT_DOUBLE: return 8;
    default: return 0;
  }
}

// Largest element count a tensor may declare: its dims are checked against
// this when parsed, so numel() never overflows.
constexpr int64_t kMaxElements = int64_t(1) << 40;

struct Tensor {
  std::string name;
  std::vector<int64_t> dims;
  int dtype = DT_FLOAT;
  std::vector<uint8_t> data;
  int64_t numel() const {
    int64_t n = 1;
    for (auto d : dims) n *= d;
    return n;
  }
  // The payload must hold exactly the elements the dims declare, at the
  // element size of `dt` (the type the caller is about to read it as).
  void require_payload(int dt) const {
    const int64_t es = dtype_bytes(dt);
    if (es == 0 || (int64_t)data.size() != numel() * es)
      fail(DW_ERR_INVALID, "onnx: tensor '" + name + "' holds " + std::to_string(data.size()) +
                               " bytes, its dims and type declare " + std::to_string(numel() * es));
  }
};

struct Attr {
  std::string name;
  enum Kind { NONE, INT, FLOAT, STRING, TENSOR, INTS, FLOATS } kind = NONE;
  int64_t i = 0;
  float f = 0;
  std::string s;
  Tensor t;
  std::vector<int64_t> is;
  std::vector<float> fs;
};

struct Node {
  std::string name, op;
  std::vector<std::string> in, out;
  std::vector<Attr> attrs;
  const Attr* attr(const std::string& n) const {
    for (auto& a : attrs)
      if (a.name == n) return &a;
    return nullptr;
  }
  int64_t get_int(const std::string& n, int64_t d) const {
    const Attr* a = attr(n);
    return a && a->kind == Attr::INT ? a->i : d;
  }
  float get_float(const std::string& n, float d) const {
    const Attr* a = attr(n);
    return a && a->kind == Attr::FLOAT ? a->f : d;
  }
  std::vector<int64_t> get_ints(const std::string& n) const {
    const Attr* a = attr(n);
    return a && a->kind == Attr::INTS ? a->is : std::vector<int64_t>{};
  }
  std::string get_string(const std::string& n, const std::string& d) const {
    const Attr* a = attr(n);
    return a && a->kind == Attr::STRING ? a->s : d;
  }
};

struct ValueInfo {
  std::string name;
  std::vector<int64_t> shape;  // -1: dynamic
  int dtype = DT_FLOAT;
};

struct Model {
  int64_t ir_version = 0, opset = 0;
  std::string producer;
  std::vector<Node> nodes;
  std::vector<Tensor> inits;
  std::vector<ValueInfo> inputs, outputs;
};

Tensor parse_tensor(Reader r) {
  Tensor t;
  std::vector<float> fd;
  std::vector<int64_t> i64d, i32d;
  bool raw = false;
  Field f;
  while (r.next(f)) {
    switch (f.num) {
      case 1: ints(f, t.dims); break;
      case 2: t.dtype = (int)i64(f); break;
      case 4: floats(f, fd); break;
      case 5: ints(f, i32d); break;  // int32_data (also carries u8/i8/f16 values)
      case 7: ints(f, i64d); break;
      case 8: t.name = str(f); break;
      case 9:
        if (f.wt != WT_LEN) fail(DW_ERR_INVALID, "onnx: raw_data must be bytes");
        t.data.assign(f.p, f.p + f.n);
        raw = true;
        break;
      default: break;
    }
  }
  int64_t n = 1;
  for (auto d : t.dims) {
    if (d < 0 || d > kMaxElements || (d > 0 && n > kMaxElements / d))
      fail(DW_ERR_INVALID, "onnx: tensor '" + t.name + "' has a negative or oversized dimension");
    n *= d;
  }
  if (raw) return t;
  if (!fd.empty()) {
    t.data.resize(fd.size() * 4);
    memcpy(t.data.data(), fd.data(), t.data.size());
  } else if (!i64d.empty()) {
    t.data.resize(i64d.size() * 8);
    memcpy(t.data.data(), i64d.data(), t.data.size());
  } else if (!i32d.empty()) {
    // int32_data holds int32 values, or the bytes of narrower integer types
    // and the bits of float16 values, one per entry
    const int es = t.dtype == DT_UINT8 || t.dtype == DT_INT8 ? 1 : (t.dtype == DT_FLOAT16 ? 2 : 4);
    t.data.resize(i32d.size() * es);
    for (size_t k = 0; k < i32d.size(); ++k) {
      const int32_t v = (int32_t)i32d[k];
      memcpy(&t.data[k * es], &v, es);
    }
  }
  return t;
}

std::vector<int64_t> parse_shape(Reader r) {
  std::vector<int64_t> dims;
  Field f;
  while (r.next(f)) {
    if (f.num != 1 || f.wt != WT_LEN) continue;
    Reader d(f.p, f.n);
    int64_t v = -1;  // dim_param (symbolic): dynamic
    Field g;
    while (d.next(g))
      if (g.num == 1) v = i64(g);
    dims.push_back(v);
  }
  return dims;
}

ValueInfo parse_value_info(Reader r) {
  ValueInfo vi;
  Field f;
  while (r.next(f)) {
    if (f.num == 1) {
      vi.name = str(f);
    } else if (f.num == 2 && f.wt == WT_LEN) {
      Reader tp(f.p, f.n);  // TypeProto
      Field g;
      while (tp.next(g)) {
        if (g.num != 1 || g.wt != WT_LEN) continue;
        Reader tt(g.p, g.n);  // TypeProto.Tensor
        Field h;
        while (tt.next(h)) {
          if (h.num == 1) vi.dtype = (int)i64(h);
          if (h.num == 2 && h.wt == WT_LEN) vi.shape = parse_shape(Reader(h.p, h.n));
        }
      }
    }
  }
  return vi;
}

Attr parse_attr(Reader r) {
  Attr a;
  Field f;
  bool any = false;
  while (r.next(f)) {
    switch (f.num) {
      case 1: a.name = str(f); break;
      case 2: {
        if (f.wt != WT_FIXED32) fail(DW_ERR_INVALID, "onnx: float attribute must be fixed32");
        const uint32_t b = (uint32_t)f.v;
        memcpy(&a.f, &b, 4);
        a.kind = Attr::FLOAT;
        any = true;
        break;
      }
      case 3: a.i = i64(f); a.kind = Attr::INT; any = true; break;
      case 4: a.s = str(f); a.kind = Attr::STRING; any = true; break;
      case 5:
        if (f.wt != WT_LEN) fail(DW_ERR_INVALID, "onnx: tensor attribute");
        a.t = parse_tensor(Reader(f.p, f.n));
        a.kind = Attr::TENSOR;
        any = true;
        break;
      case 7: floats(f, a.fs); break;
      case 8: ints(f, a.is); break;
      default: break;
    }
  }
  if (!a.is.empty()) a.kind = Attr::INTS;
  else if (!a.fs.empty()) a.kind = Attr::FLOATS;
  else if (!any) a.kind = Attr::INTS;  // an empty repeated field
  return a;
}

Node parse_node(Reader r) {
  Node n;
  Field f;
  while (r.next(f)) {
    switch (f.num) {
      case 1: n.in.push_back(str(f)); break;
      case 2: n.out.push_back(str(f)); break;
      case 3: n.name = str(f); break;
      case 4: n.op = str(f); break;
      case 5:
        if (f.wt != WT_LEN) fail(DW_ERR_INVALID, "onnx: attribute");
        n.attrs.push_back(parse_attr(Reader(f.p, f.n)));
        break;
      default: break;
    }
  }
  if (n.name.empty()) n.name = n.op + "_" + (n.out.empty() ? std::string("unnamed") : n.out[0]);
  return n;
}

Model parse_model(const uint8_t* bytes, size_t len) {
  Model m;
  Reader r(bytes, len);
  Field f;
  bool graph = false;
  while (r.next(f)) {
    switch (f.num) {
      case 1: m.ir_version = i64(f); break;
      case 2: m.producer = str(f); break;
      case 7: {
        if (f.wt != WT_LEN) fail(DW_ERR_INVALID, "onnx: graph");
        graph = true;
        Reader g(f.p, f.n);
        Field h;
        while (g.next(h)) {
          if (h.wt != WT_LEN) continue;
          Reader s(h.p, h.n);
          if (h.num == 1) m.nodes.push_back(parse_node(s));
          else if (h.num == 5) m.inits.push_back(parse_tensor(s));
          else if (h.num == 11) m.inputs.push_back(parse_value_info(s));
          else if (h.num == 12) m.outputs.push_back(parse_value_info(s));
        }
        break;
      }
      case 8: {
        if (f.wt != WT_LEN) fail(DW_ERR_INVALID, "onnx: opset_import");
        Reader o(f.p, f.n);
        Field h;
        std::string domain;
        int64_t v = 0;
        while (o.next(h)) {
          if (h.num == 1) domain = str(h);
          if (h.num == 2) v = i64(h);
        }
        if ((domain.empty() || domain == "ai.onnx") && v > m.opset) m.opset = v;
        break;
      }
      default: break;
    }
  }
  if (!graph) fail(DW_ERR_INVALID, "onnx: no graph in the model");
  // model.rs:356-365: opsets 12 to 20
  if (m.opset < 12 || m.opset > 20)
    fail(DW_ERR_UNSUPPORTED, "onnx: unsupported opset " + std::to_string(m.opset) + " (12 to 20)");
  return m;
}

// ---------------------------------------------------------------------------
// inspection (a JSON summary of the parsed model)
// ---------------------------------------------------------------------------
std::string jq(const std::string& s) {
  std::string o = "\"";
  for (char c : s) {
    if (c == '"' || c == '\\') o += '\\';
    if ((unsigned char)c < 0x20) {
      char b[8];
      snprintf(b, sizeof b, "\\u%04x", (unsigned)(unsigned char)c);
      o += b;
      continue;
    }
    o += c;
  }
  return o + "\"";
}
std::string jints(const std::vector<int64_t>& v) {
  std::string o = "[";
  for (size_t i = 0; i < v.size(); ++i) o += (i ? "," : "") + std::to_string(v[i]);
  return o + "]";
}
std::string jfloat(float f) {
  if (isnan(f)) return "null";
  if (isinf(f)) return f > 0 ? "1e999" : "-1e999";
  char b[32];
  snprintf(b, sizeof b, "%.9g", f);
  return b;
}

std::string inspect(const Model& m) {
  std::ostringstream o;
  o << "{\"ir_version\":" << m.ir_version << ",\"opset\":" << m.opset << ",\"producer\":" << jq(m.producer)
    << ",\"nodes\":[";
  for (size_t i = 0; i < m.nodes.size(); ++i) {
    const Node& n = m.nodes[i];
    o << (i ? "," : "") << "{\"name\":" << jq(n.name) << ",\"op\":" << jq(n.op) << ",\"inputs\":[";
    for (size_t k = 0; k < n.in.size(); ++k) o << (k ? "," : "") << jq(n.in[k]);
    o << "],\"outputs\":[";
    for (size_t k = 0; k < n.out.size(); ++k) o << (k ? "," : "") << jq(n.out[k]);
    o << "],\"attrs\":{";
    for (size_t k = 0; k < n.attrs.size(); ++k) {
      const Attr& a = n.attrs[k];
      o << (k ? "," : "") << jq(a.name) << ":";
      switch (a.kind) {
        case Attr::INT: o << a.i; break;
        case Attr::FLOAT: o << jfloat(a.f); break;
        case Attr::STRING: o << jq(a.s); break;
        case Attr::TENSOR: o << "{\"dims\":" << jints(a.t.dims) << ",\"dtype\":" << a.t.dtype << ",\"bytes\":" << a.t.data.size() << "}"; break;
        case Attr::INTS: o << jints(a.is); break;
        case Attr::FLOATS: {
          o << "[";
          for (size_t j = 0; j < a.fs.size(); ++j) o << (j ? "," : "") << jfloat(a.fs[j]);
          o << "]";
          break;
        }
        default: o << "null";
      }
    }
    o << "}}";
  }
  o << "],\"initializers\":[";
  for (size_t i = 0; i < m.inits.size(); ++i) {
    const Tensor& t = m.inits[i];
    o << (i ? "," : "") << "{\"name\":" << jq(t.name) << ",\"dims\":" << jints(t.dims) << ",\"dtype\":" << t.dtype
      << ",\"bytes\":" << t.data.size() << "}";
  }
  auto vis = [&](const std::vector<ValueInfo>& v) {
    o << "[";
    for (size_t i = 0; i < v.size(); ++i)
      o << (i ? "," : "") << "{\"name\":" << jq(v[i].name) << ",\"shape\":" << jints(v[i].shape)
        << ",\"dtype\":" << v[i].dtype << "}";
    o << "]";
  };
  o << "],\"inputs\":";
  vis(m.inputs);
  o << ",\"outputs\":";
  vis(m.outputs);
  o << "}";
  return o.str();
}

// ---------------------------------------------------------------------------
// build
// ---------------------------------------------------------------------------
struct Builder {
  const Model& m;
  GraphIR& g;
  std::map<std::string, const Tensor*> init;   // ONNX initializers and Constant values
  std::deque<Tensor> consts;                   // storage of Constant node values and folded constants
  // Pad nodes folded into the Conv that reads them: padded tensor ->
  // (unpadded source, [top, left, bottom, right])
  std::map<std::string, std::pair<std::string, std::vector<int64_t>>> pads_of;
  std::map<std::string, std::string> alias;    // tensor name -> the name it stands for
  std::map<std::string, std::pair<float, int>> qparams;  // activation -> (scale, zero point)
  std::set<std::string> used_init;
  int counter = 0;

  Builder(const Model& model, GraphIR& graph) : m(model), g(graph) {}

  std::string A(const std::string& n) const {
    auto it = alias.find(n);
    return it == alias.end() ? n : A(it->second);
  }
  const Tensor* const_of(const std::string& n) const {
    auto it = init.find(A(n));
    return it == init.end() ? nullptr : it->second;
  }
  std::vector<int64_t> const_ints(const std::string& n) const {
    const Tensor* t = const_of(n);
    if (!t) fail(DW_ERR_UNSUPPORTED, "onnx: '" + n + "' must be a constant");
    if (t->dtype != DT_INT64 && t->dtype != DT_INT32)
      fail(DW_ERR_UNSUPPORTED, "onnx: '" + n + "' must be an integer constant");
    t->require_payload(t->dtype);
    std::vector<int64_t> v(t->numel());
    if (t->dtype == DT_INT64) {
      if (!v.empty()) memcpy(v.data(), t->data.data(), v.size() * 8);
    } else {
      for (size_t i = 0; i < v.size(); ++i) {
        int32_t e;
        memcpy(&e, &t->data[i * 4], 4);
        v[i] = e;
      }
    }
    return v;
  }
  std::vector<float> const_floats(const std::string& n) const {
    const Tensor* t = const_of(n);
    if (!t) fail(DW_ERR_UNSUPPORTED, "onnx: '" + n + "' must be a constant");
    if (t->dtype != DT_FLOAT) fail(DW_ERR_UNSUPPORTED, "onnx: '" + n + "' must be a float constant");
    t->require_payload(DT_FLOAT);
    std::vector<float> v(t->numel());
    if (!v.empty()) memcpy(v.data(), t->data.data(), v.size() * 4);
    return v;
  }
  int const_zp(const std::string& n) const {
    if (n.empty()) return 0;
    const Tensor* t = const_of(n);
    if (!t || t->numel() != 1) fail(DW_ERR_UNSUPPORTED, "onnx: zero point '" + n + "' must be a scalar constant");
    if (t->dtype != DT_UINT8 && t->dtype != DT_INT8 && t->dtype != DT_INT32)
      fail(DW_ERR_UNSUPPORTED, "onnx: zero point type");
    t->require_payload(t->dtype);
    if (t->dtype == DT_UINT8) return t->data[0];
    if (t->dtype == DT_INT8) return (int8_t)t->data[0];
    int32_t v;
    memcpy(&v, t->data.data(), 4);
    return v;
  }

  TensorInfo& T(const std::string& n) { return g.tensor(A(n)); }
  const std::vector<int64_t>& dims(const std::string& n) { return T(n).dims; }

  void declare(const std::string& n, const std::vector<int64_t>& d) {
    for (auto v : d)
      if (v <= 0) fail(DW_ERR_UNSUPPORTED, "onnx: '" + n + "' has a dynamic or empty dimension");
    if (d.size() > 4) fail(DW_ERR_UNSUPPORTED, "onnx: '" + n + "' has rank above 4");
    TensorInfo ti;
    ti.dims = d;
    ti.dtype = DW_DTYPE_F32;
    g.t[n] = ti;
  }
  // an ONNX f32 initializer (or constant) as a graph initializer
  void use_init(const std::string& name) {
    const std::string n = A(name);
    if (g.has(n)) return;
    const Tensor* t = const_of(n);
    if (!t) fail(DW_ERR_RUNTIME, "onnx: unknown tensor '" + name + "'");
    if (t->dtype != DT_FLOAT) fail(DW_ERR_UNSUPPORTED, "onnx: initializer '" + n + "' is not f32");
    if (t->dims.size() > 4) fail(DW_ERR_UNSUPPORTED, "onnx: initializer '" + n + "' rank");
    TensorInfo ti;
    ti.dims = t->dims.empty() ? std::vector<int64_t>{1} : t->dims;
    ti.dtype = DW_DTYPE_F32;
    ti.is_init = true;
    t->require_payload(DT_FLOAT);
    ti.data = t->data;
    g.t[n] = ti;
  }
  std::string in_name(const std::string& n) {
    const std::string a = A(n);
    if (pads_of.count(a)) fail(DW_ERR_UNSUPPORTED, "onnx: Pad output '" + a + "' must feed a Conv");
    if (!g.has(a)) use_init(a);
    return a;
  }

  // ---- constants --------------------------------------------------------
  const Tensor& add_const(const std::string& name, std::vector<int64_t> dims, int dtype,
                          std::vector<uint8_t> data) {
    Tensor t;
    t.name = name;
    t.dims = std::move(dims);
    t.dtype = dtype;
    t.data = std::move(data);
    t.require_payload(dtype);
    consts.push_back(std::move(t));
    init[name] = &consts.back();
    return consts.back();
  }
  static std::vector<uint8_t> bytes_of(const std::vector<int64_t>& v) {
    std::vector<uint8_t> b(v.size() * 8);
    if (!v.empty()) memcpy(b.data(), v.data(), b.size());
    return b;
  }
  static std::vector<uint8_t> bytes_of(const std::vector<float>& v) {
    std::vector<uint8_t> b(v.size() * 4);
    if (!v.empty()) memcpy(b.data(), v.data(), b.size());
    return b;
  }
  // a constant's values as f64 (integer or float types)
  std::vector<double> const_values(const Tensor& t) const {
    t.require_payload(t.dtype);
    std::vector<double> v((size_t)t.numel());
    for (size_t i = 0; i < v.size(); ++i) {
      switch (t.dtype) {
        case DT_INT64: { int64_t e; memcpy(&e, &t.data[i * 8], 8); v[i] = (double)e; break; }
        case DT_INT32: { int32_t e; memcpy(&e, &t.data[i * 4], 4); v[i] = e; break; }
        case DT_FLOAT: { float e; memcpy(&e, &t.data[i * 4], 4); v[i] = e; break; }
        case DT_DOUBLE: { double e; memcpy(&e, &t.data[i * 8], 8); v[i] = e; break; }
        case DT_UINT8: v[i] = t.data[i]; break;
        case DT_INT8: v[i] = (int8_t)t.data[i]; break;
        default: fail(DW_ERR_UNSUPPORTED, "onnx: constant '" + t.name + "' of type " + std::to_string(t.dtype));
      }
    }
    return v;
  }
  // a constant of type dt holding values v (integers exactly)
  const Tensor& const_from_values(const std::string& name, std::vector<int64_t> dims, int dt,
                                  const std::vector<double>& v) {
    if (dt == DT_INT64 || dt == DT_INT32) {
      std::vector<int64_t> iv(v.size());
      for (size_t i = 0; i < v.size(); ++i) iv[i] = (int64_t)v[i];
      return add_const(name, std::move(dims), DT_INT64, bytes_of(iv));
    }
    std::vector<float> fv(v.begin(), v.end());
    return add_const(name, std::move(dims), DT_FLOAT, bytes_of(fv));
  }
  // dims of an activation or a constant
  std::vector<int64_t> dims_any(const std::string& n) {
    const std::string a = A(n);
    if (g.has(a)) return g.tensor(a).dims;
    const Tensor* t = const_of(a);
    if (!t) fail(DW_ERR_RUNTIME, "onnx: unknown tensor '" + n + "'");
    return t->dims;
  }
  bool is_const(const std::string& n) const { return !n.empty() && const_of(n) && !g.has(A(n)); }
  // the axes list of Squeeze / Unsqueeze / ReduceX: an input (opset 13+) or an attribute
  std::vector<int64_t> axes_of(const Node& n) {
    if (n.in.size() > 1 && !n.in[1].empty()) return const_ints(n.in[1]);
    return n.get_ints("axes");
  }

  // ONNX multidirectional broadcast of two shapes
  static std::vector<int64_t> broadcast(const std::vector<int64_t>& a, const std::vector<int64_t>& b,
                                        const std::string& who) {
    const size_t r = std::max(a.size(), b.size());
    std::vector<int64_t> o(r);
    for (size_t k = 0; k < r; ++k) {
      const int64_t da = k + a.size() >= r ? a[k + a.size() - r] : 1;
      const int64_t db = k + b.size() >= r ? b[k + b.size() - r] : 1;
      if (da != db && da != 1 && db != 1) fail(DW_ERR_RUNTIME, "onnx: " + who + ": shapes do not broadcast");
      o[k] = std::max(da, db);
    }
    return o;
  }

  void add(const std::string& name, const std::string& type, std::vector<std::string> in,
           std::vector<std::string> out, const dw_op_params& p) {
    OpNode op;
    op.name = name;
    op.type = type;
    op.in = std::move(in);
    op.out = std::move(out);
    op.p = p;
    g.ops.push_back(op);
  }

  static dw_op_params params(int kind) {
    dw_op_params p{};
    p.kind = kind;
    p.group = 1;
    p.dilations[0] = p.dilations[1] = 1;
    p.strides[0] = p.strides[1] = 1;
    p.epsilon = 1e-5f;
    p.alpha = p.beta = 1.0f;
    p.clip_min = -INFINITY;
    p.clip_max = INFINITY;
    p.mode_nearest = 1;
    return p;
  }

  // -------------------------------------------------------------------------
  // QDQ analysis: Constant nodes, dequantized initializers, Q -> DQ pairs
  void prepare() {
    for (const Tensor& t : m.inits) init[t.name] = &t;
    for (const Node& n : m.nodes)
      if (n.op == "Constant") {
        const Attr* a = n.attr("value");
        if (!a || a->kind != Attr::TENSOR || n.out.empty())
          fail(DW_ERR_UNSUPPORTED, "onnx: Constant " + n.name + " without a tensor value");
        consts.push_back(a->t);
      }
    size_t ci = 0;
    for (const Node& n : m.nodes)
      if (n.op == "Constant") {
        consts[ci].name = n.out[0];
        ++ci;
      }
    for (const Tensor& t : consts) init[t.name] = &t;
  }

  // DequantizeLinear of an int8 / int32 initializer: a prequantized f32
  // initializer (the integers as f32 values) with its scales
  bool dq_initializer(const Node& n) {
    const Tensor* q = const_of(n.in[0]);
    if (!q) return false;
    if (q->dtype != DT_INT8 && q->dtype != DT_INT32 && q->dtype != DT_UINT8)
      fail(DW_ERR_UNSUPPORTED, "onnx: DequantizeLinear of a constant of type " + std::to_string(q->dtype));
    const std::vector<float> sc = const_floats(n.in[1]);
    const std::string zpn = n.in.size() > 2 ? n.in[2] : "";
    if (!zpn.empty()) {
      const Tensor* z = const_of(zpn);
      if (!z) fail(DW_ERR_UNSUPPORTED, "onnx: weight zero point must be constant");
      z->require_payload(z->dtype);
      for (uint8_t b : z->data)
        if (b != 0) fail(DW_ERR_UNSUPPORTED, "onnx: weights need zero point 0 (symmetric)");
    }
    if (q->dtype == DT_UINT8) fail(DW_ERR_UNSUPPORTED, "onnx: u8 weights (s8 symmetric only)");
    q->require_payload(q->dtype);
    const int64_t cnt = q->numel();
    TensorInfo ti;
    ti.dims = q->dims.empty() ? std::vector<int64_t>{1} : q->dims;
    ti.dtype = DW_DTYPE_F32;
    ti.is_init = true;
    ti.prequant = true;
    std::vector<float> v(cnt);
    for (int64_t i = 0; i < cnt; ++i) {
      if (q->dtype == DT_INT8) {
        v[i] = (float)(int8_t)q->data[i];
      } else {
        int32_t e;
        memcpy(&e, &q->data[i * 4], 4);
        v[i] = (float)e;
      }
    }
    ti.data.resize(cnt * 4);
    memcpy(ti.data.data(), v.data(), ti.data.size());
    // per-channel scales along `axis` (opset 13 default 1), or one scale
    int64_t axis = n.get_int("axis", 1);
    if (axis < 0) axis += (int64_t)ti.dims.size();
    if (ti.dims.size() == 1) axis = 0;
    if (sc.size() == 1) {
      ti.ch_scales = sc;
      ti.q_axis = -1;
    } else {
      if (axis < 0 || axis >= (int64_t)ti.dims.size() || ti.dims[axis] != (int64_t)sc.size())
        fail(DW_ERR_UNSUPPORTED, "onnx: per-channel scales of " + n.name + " do not match axis " + std::to_string(axis));
      ti.ch_scales = sc;
      ti.q_axis = (int)axis;
    }
    if (q->dtype == DT_INT32) ti.prequant_i32 = true;
    g.t[n.out[0]] = ti;
    return true;
  }

  // -------------------------------------------------------------------------
  void build() {
    prepare();
    // graph inputs (those that are not initializers)
    for (const ValueInfo& vi : m.inputs) {
      if (init.count(vi.name)) continue;
      if (vi.dtype != DT_FLOAT) fail(DW_ERR_UNSUPPORTED, "onnx: graph input '" + vi.name + "' is not f32");
      declare(vi.name, vi.shape);
      g.inputs.push_back(vi.name);
    }
    for (const Node& n : m.nodes) node(n);
    for (const ValueInfo& vi : m.outputs) {
      const std::string o = A(vi.name);
      if (!g.has(o)) fail(DW_ERR_RUNTIME, "onnx: output '" + vi.name + "' is never computed");
      g.outputs.push_back(o);
    }
    // activation quantization parameters of QDQ models
    for (auto& kv : qparams) {
      TensorInfo& ti = T(kv.first);
      if (ti.has_q && (ti.scale != kv.second.first || ti.zp != kv.second.second))
        fail(DW_ERR_UNSUPPORTED, "onnx: '" + kv.first + "' is quantized with two different parameters");
      ti.has_q = true;
      ti.scale = kv.second.first;
      ti.zp = kv.second.second;
      ti.q_fixed = true;
    }
  }

  void out_like(const Node& n, const std::string& x) {
    declare(n.out[0], dims(x));
  }

  void node(const Node& n) {
    const std::string& op = n.op;
    if (op == "Constant") return;
    if (op == "Identity" || op == "Dropout") {
      alias[n.out[0]] = A(n.in[0]);
      return;
    }
    if (op == "QuantizeLinear") {
      // activation quantization: the u8 tensor stands for the f32 one, with
      // its scale and zero point
      const std::string x = A(n.in[0]);
      const std::vector<float> s = const_floats(n.in[1]);
      if (s.size() != 1) fail(DW_ERR_UNSUPPORTED, "onnx: per-channel activation quantization");
      const int zp = n.in.size() > 2 ? const_zp(n.in[2]) : 0;
      if (n.in.size() > 2) {
        const Tensor* z = const_of(n.in[2]);
        if (z->dtype != DT_UINT8) fail(DW_ERR_UNSUPPORTED, "onnx: activations must quantize to u8");
      } else {
        fail(DW_ERR_UNSUPPORTED, "onnx: QuantizeLinear without a u8 zero point");
      }
      auto it = qparams.find(x);
      if (it != qparams.end() && (it->second.first != s[0] || it->second.second != zp))
        fail(DW_ERR_UNSUPPORTED, "onnx: '" + x + "' is quantized with two different parameters");
      qparams[x] = {s[0], zp};
      alias[n.out[0]] = x;
      return;
    }
    if (op == "DequantizeLinear") {
      if (dq_initializer(n)) return;
      // an activation: must undo a QuantizeLinear with the same parameters
      const std::string x = A(n.in[0]);
      const std::vector<float> s = const_floats(n.in[1]);
      const int zp = n.in.size() > 2 ? const_zp(n.in[2]) : 0;
      auto it = qparams.find(x);
      if (it == qparams.end() || s.size() != 1 || it->second.first != s[0] || it->second.second != zp)
        fail(DW_ERR_UNSUPPORTED, "onnx: DequantizeLinear " + n.name + " does not undo a QuantizeLinear");
      alias[n.out[0]] = x;
      return;
    }
    if (op == "Conv") {
      std::vector<int64_t> pre_pad(4, 0);
      std::string xin = A(n.in[0]);
      auto pf = pads_of.find(xin);
      if (pf != pads_of.end()) {
        pre_pad = pf->second.second;
        xin = pf->second.first;
      }
      const std::string x = in_name(xin), w = in_name(n.in[1]);
      const auto& xd = dims(x);
      const auto& wd = dims(w);
      if (xd.size() != 4 || wd.size() != 4) fail(DW_ERR_UNSUPPORTED, "onnx: Conv " + n.name + " is not 2-D");
      dw_op_params p = params(DW_OP_CONV2D);
      std::vector<int64_t> ks = n.get_ints("kernel_shape");
      if (ks.empty()) ks = {wd[2], wd[3]};
      std::vector<int64_t> st = n.get_ints("strides"), dl = n.get_ints("dilations"), pd = n.get_ints("pads");
      if (st.empty()) st = {1, 1};
      if (dl.empty()) dl = {1, 1};
      const std::string ap = n.get_string("auto_pad", "NOTSET");
      if (ap == "SAME_UPPER" || ap == "SAME_LOWER") {
        pd.assign(4, 0);
        for (int k = 0; k < 2; ++k) {
          const int64_t in = xd[2 + k], o = (in + st[k] - 1) / st[k];
          const int64_t tot = std::max<int64_t>(0, (o - 1) * st[k] + (ks[k] - 1) * dl[k] + 1 - in);
          const int64_t lo = ap == "SAME_UPPER" ? tot / 2 : tot - tot / 2;
          pd[k] = lo;
          pd[2 + k] = tot - lo;
        }
      } else if (ap == "VALID") {
        pd.assign(4, 0);
      }
      if (pd.empty()) pd.assign(4, 0);
      for (int k = 0; k < 4; ++k) pd[k] += pre_pad[k];
      const int64_t group = n.get_int("group", 1);
      p.kernel_shape[0] = (int)ks[0]; p.kernel_shape[1] = (int)ks[1];
      p.strides[0] = (int)st[0]; p.strides[1] = (int)st[1];
      p.dilations[0] = (int)dl[0]; p.dilations[1] = (int)dl[1];
      // ONNX pads [top, left, bottom, right] = [x1_begin, x2_begin, x1_end, x2_end]
      for (int k = 0; k < 4; ++k) p.pads[k] = (int)pd[k];
      p.group = (int)group;
      const int64_t ho = (xd[2] + pd[0] + pd[2] - dl[0] * (ks[0] - 1) - 1) / st[0] + 1;
      const int64_t wo = (xd[3] + pd[1] + pd[3] - dl[1] * (ks[1] - 1) - 1) / st[1] + 1;
      declare(n.out[0], {xd[0], wd[0], ho, wo});
      std::vector<std::string> ins{x, w};
      if (n.in.size() > 2 && !n.in[2].empty()) ins.push_back(in_name(n.in[2]));
      add(n.name, "Conv", ins, {n.out[0]}, p);
      return;
    }
    if (op == "QLinearConv") {
      fail(DW_ERR_UNSUPPORTED, "onnx: QLinearConv nodes (export the QDQ form instead)");
    }
    if (op == "Relu" || op == "Sigmoid") {
      const std::string x = in_name(n.in[0]);
      out_like(n, x);
      add(n.name, op, {x}, {n.out[0]}, params(op == "Sigmoid" ? DW_OP_SIGMOID : DW_OP_NONE));
      return;
    }
    if (op == "Clip") {
      const std::string x = in_name(n.in[0]);
      dw_op_params p = params(DW_OP_CLIP);
      // opset 11+: min and max as optional inputs; older: attributes
      p.clip_min = n.get_float("min", -INFINITY);
      p.clip_max = n.get_float("max", INFINITY);
      if (n.in.size() > 1 && !n.in[1].empty()) p.clip_min = const_floats(n.in[1]).at(0);
      if (n.in.size() > 2 && !n.in[2].empty()) p.clip_max = const_floats(n.in[2]).at(0);
      out_like(n, x);
      add(n.name, "Clip", {x}, {n.out[0]}, p);
      return;
    }
    if (op == "Add" || op == "Mul" || op == "Sub" || op == "Div") {
      const auto da = dims_any(n.in[0]), db = dims_any(n.in[1]);
      const auto dy = broadcast(da, db, op + " " + n.name);
      if (is_const(n.in[0]) && is_const(n.in[1])) {
        // shape arithmetic on constants: folded (scalar or equal-size operands)
        const Tensor& ta = *const_of(n.in[0]);
        const Tensor& tb = *const_of(n.in[1]);
        const auto va = const_values(ta), vb = const_values(tb);
        if (!(va.size() == vb.size() || va.size() == 1 || vb.size() == 1))
          fail(DW_ERR_UNSUPPORTED, "onnx: constant " + op + " " + n.name + " with general broadcasting");
        const bool ints = (ta.dtype == DT_INT64 || ta.dtype == DT_INT32) && (tb.dtype == DT_INT64 || tb.dtype == DT_INT32);
        std::vector<double> r(std::max(va.size(), vb.size()));
        for (size_t i = 0; i < r.size(); ++i) {
          const double x = va[va.size() == 1 ? 0 : i], y = vb[vb.size() == 1 ? 0 : i];
          if (op == "Add") r[i] = x + y;
          else if (op == "Sub") r[i] = x - y;
          else if (op == "Mul") r[i] = x * y;
          else if (ints) {
            if (y == 0) fail(DW_ERR_INVALID, "onnx: integer division by zero in " + n.name);
            r[i] = (double)((int64_t)x / (int64_t)y);  // ONNX integer Div truncates
          } else {
            r[i] = (float)x / (float)y;
          }
          if (!ints) r[i] = (float)r[i];
        }
        const_from_values(n.out[0], dy, ints ? DT_INT64 : DT_FLOAT, r);
        return;
      }
      const std::string a = in_name(n.in[0]), b = in_name(n.in[1]);
      if (dy.size() > 4) fail(DW_ERR_UNSUPPORTED, "onnx: " + op + " " + n.name + " above rank 4");
      declare(n.out[0], dy);
      const int kind = op == "Add" ? DW_OP_ADD : op == "Mul" ? DW_OP_MUL : op == "Sub" ? DW_OP_SUB : DW_OP_DIV;
      add(n.name, op, {a, b}, {n.out[0]}, params(kind));
      return;
    }
    if (op == "Shape") {
      const auto d = dims_any(n.in[0]);
      const int64_t r = (int64_t)d.size();
      int64_t st = n.get_int("start", 0), en = n.get_int("end", r);
      if (st < 0) st += r;
      if (en < 0) en += r;
      st = std::min(std::max<int64_t>(st, 0), r);
      en = std::min(std::max<int64_t>(en, st), r);
      std::vector<int64_t> v(d.begin() + st, d.begin() + en);
      add_const(n.out[0], {(int64_t)v.size()}, DT_INT64, bytes_of(v));
      return;
    }
    if (op == "Gather") {
      if (!is_const(n.in[0]) || !is_const(n.in[1]))
        fail(DW_ERR_UNSUPPORTED, "onnx: Gather " + n.name + " of an activation");
      const Tensor& td = *const_of(n.in[0]);
      const Tensor& ti = *const_of(n.in[1]);
      if (td.dims.size() != 1 || n.get_int("axis", 0) != 0)
        fail(DW_ERR_UNSUPPORTED, "onnx: Gather " + n.name + ": only 1-D constants along axis 0");
      const auto vd = const_values(td);
      const auto vi = const_ints(n.in[1]);
      std::vector<double> r;
      for (int64_t k : vi) {
        const int64_t i = k < 0 ? k + (int64_t)vd.size() : k;
        if (i < 0 || i >= (int64_t)vd.size()) fail(DW_ERR_INVALID, "onnx: Gather " + n.name + " index out of range");
        r.push_back(vd[(size_t)i]);
      }
      const_from_values(n.out[0], ti.dims, td.dtype, r);
      return;
    }
    if (op == "Unsqueeze" || op == "Squeeze") {
      auto d = dims_any(n.in[0]);
      auto ax = axes_of(n);
      std::vector<int64_t> out;
      if (op == "Unsqueeze") {
        const int64_t r = (int64_t)(d.size() + ax.size());
        for (auto& a : ax) a = a < 0 ? a + r : a;
        std::sort(ax.begin(), ax.end());
        out = d;
        for (int64_t a : ax) {
          if (a < 0 || a > (int64_t)out.size()) fail(DW_ERR_INVALID, "onnx: Unsqueeze " + n.name + " axis");
          out.insert(out.begin() + a, 1);
        }
      } else {
        const int64_t r = (int64_t)d.size();
        for (auto& a : ax) a = a < 0 ? a + r : a;
        for (int64_t k = 0; k < r; ++k) {
          const bool drop = ax.empty() ? d[k] == 1 : std::find(ax.begin(), ax.end(), k) != ax.end();
          if (drop && d[k] != 1) fail(DW_ERR_INVALID, "onnx: Squeeze " + n.name + " of a dimension above 1");
          if (!drop) out.push_back(d[k]);
        }
      }
      if (is_const(n.in[0])) {
        const Tensor& t = *const_of(n.in[0]);
        add_const(n.out[0], out, t.dtype, t.data);
        return;
      }
      const std::string x = in_name(n.in[0]);
      declare(n.out[0], out);
      add(n.name, "Reshape", {x}, {n.out[0]}, params(DW_OP_RESHAPE));
      return;
    }
    if (op == "Cast") {
      if (!is_const(n.in[0])) {
        // a float activation cast to float: the identity
        if (n.get_int("to", DT_FLOAT) != DT_FLOAT) fail(DW_ERR_UNSUPPORTED, "onnx: Cast " + n.name + " of an activation");
        alias[n.out[0]] = A(n.in[0]);
        return;
      }
      const Tensor& t = *const_of(n.in[0]);
      const int to = (int)n.get_int("to", DT_FLOAT);
      if (to != DT_FLOAT && to != DT_INT64 && to != DT_INT32)
        fail(DW_ERR_UNSUPPORTED, "onnx: Cast " + n.name + " to type " + std::to_string(to));
      auto v = const_values(t);
      if (to != DT_FLOAT)
        for (auto& e : v) e = std::trunc(e);
      const_from_values(n.out[0], t.dims, to, v);
      return;
    }
    if (op == "Transpose") {
      const std::string x = in_name(n.in[0]);
      const auto xd = dims(x);
      std::vector<int64_t> perm = n.get_ints("perm");
      if (perm.empty())
        for (int64_t k = (int64_t)xd.size() - 1; k >= 0; --k) perm.push_back(k);
      if (perm.size() != xd.size() || xd.size() > 4) fail(DW_ERR_UNSUPPORTED, "onnx: Transpose " + n.name + " rank");
      std::vector<int64_t> od;
      std::vector<int> seen(xd.size(), 0);
      for (int64_t a : perm) {
        if (a < 0 || a >= (int64_t)xd.size() || seen[a]++) fail(DW_ERR_INVALID, "onnx: Transpose " + n.name + " perm");
        od.push_back(xd[a]);
      }
      dw_op_params p = params(DW_OP_TRANSPOSE);
      for (size_t k = 0; k < 4; ++k) p.perm[k] = k < perm.size() ? (int)perm[k] : (int)k;
      declare(n.out[0], od);
      add(n.name, "Transpose", {x}, {n.out[0]}, p);
      return;
    }
    if (op == "Slice") {
      const std::string x = in_name(n.in[0]);
      const auto xd = dims(x);
      const auto st = const_ints(n.in[1]), en = const_ints(n.in[2]);
      std::vector<int64_t> ax, sp;
      if (n.in.size() > 3 && !n.in[3].empty()) ax = const_ints(n.in[3]);
      else for (size_t k = 0; k < st.size(); ++k) ax.push_back((int64_t)k);
      if (n.in.size() > 4 && !n.in[4].empty()) sp = const_ints(n.in[4]);
      else sp.assign(st.size(), 1);
      if (en.size() != st.size() || ax.size() != st.size() || sp.size() != st.size() || st.size() > 4)
        fail(DW_ERR_INVALID, "onnx: Slice " + n.name + " arguments");
      dw_op_params p = params(DW_OP_SLICE);
      auto od = xd;
      const int64_t r = (int64_t)xd.size();
      for (size_t k = 0; k < st.size(); ++k) {
        int64_t a = ax[k] < 0 ? ax[k] + r : ax[k];
        if (a < 0 || a >= r) fail(DW_ERR_INVALID, "onnx: Slice " + n.name + " axis");
        if (sp[k] < 1) fail(DW_ERR_UNSUPPORTED, "onnx: Slice " + n.name + " with a step below 1");
        const int64_t dim = xd[a];
        // ONNX: negative indices count from the end; both clamped to [0, dim]
        int64_t s0 = st[k] < 0 ? st[k] + dim : st[k];
        int64_t e0 = en[k] < 0 ? en[k] + dim : en[k];
        s0 = std::min(std::max<int64_t>(s0, 0), dim);
        e0 = std::min(std::max<int64_t>(e0, s0), dim);
        p.slice_axes[k] = (int)a;
        p.slice_starts[k] = (int)s0;
        p.slice_ends[k] = (int)e0;
        p.slice_steps[k] = (int)sp[k];
        od[a] = (e0 - s0 + sp[k] - 1) / sp[k];
      }
      p.num_slice_axes = (int)st.size();
      declare(n.out[0], od);
      add(n.name, "Slice", {x}, {n.out[0]}, p);
      return;
    }
    if (op == "AveragePool") {
      const std::string x = in_name(n.in[0]);
      const auto& xd = dims(x);
      if (xd.size() != 4) fail(DW_ERR_UNSUPPORTED, "onnx: AveragePool " + n.name + " is not 2-D");
      if (n.get_int("ceil_mode", 0)) fail(DW_ERR_UNSUPPORTED, "onnx: AveragePool ceil_mode");
      const auto ks = n.get_ints("kernel_shape");
      auto st = n.get_ints("strides");
      auto pd = n.get_ints("pads");
      if (ks.size() != 2) fail(DW_ERR_UNSUPPORTED, "onnx: AveragePool kernel_shape");
      if (st.empty()) st = {1, 1};
      for (auto v : pd)
        if (v != 0) fail(DW_ERR_UNSUPPORTED, "onnx: padded AveragePool " + n.name);
      const std::string ap = n.get_string("auto_pad", "NOTSET");
      if (ap != "NOTSET" && ap != "VALID") fail(DW_ERR_UNSUPPORTED, "onnx: AveragePool auto_pad " + ap);
      dw_op_params p = params(DW_OP_AVGPOOL);
      p.kernel_shape[0] = (int)ks[0]; p.kernel_shape[1] = (int)ks[1];
      p.strides[0] = (int)st[0]; p.strides[1] = (int)st[1];
      declare(n.out[0], {xd[0], xd[1], (xd[2] - ks[0]) / st[0] + 1, (xd[3] - ks[1]) / st[1] + 1});
      add(n.name, "AveragePool", {x}, {n.out[0]}, p);
      return;
    }
    if (op == "Pad") {
      // a constant zero spatial pad is folded into the Conv that reads it
      if (n.get_string("mode", "constant") != "constant") fail(DW_ERR_UNSUPPORTED, "onnx: Pad mode");
      const std::string x = A(n.in[0]);
      const auto xd = dims_any(x);
      std::vector<int64_t> pd = n.in.size() > 1 && !n.in[1].empty() ? const_ints(n.in[1]) : n.get_ints("pads");
      if (n.in.size() > 2 && !n.in[2].empty()) {
        const auto v = const_values(*const_of(n.in[2]));
        if (!v.empty() && v[0] != 0.0) fail(DW_ERR_UNSUPPORTED, "onnx: Pad " + n.name + " with a nonzero value");
      }
      if (n.in.size() > 3 && !n.in[3].empty()) fail(DW_ERR_UNSUPPORTED, "onnx: Pad axes");
      if (xd.size() != 4 || pd.size() != 8 || pd[0] || pd[1] || pd[4] || pd[5])
        fail(DW_ERR_UNSUPPORTED, "onnx: Pad " + n.name + " other than spatial on a 4-D tensor");
      for (auto v : pd)
        if (v < 0) fail(DW_ERR_UNSUPPORTED, "onnx: negative Pad");
      if (pads_of.count(x)) fail(DW_ERR_UNSUPPORTED, "onnx: Pad of a Pad");
      pads_of[n.out[0]] = {x, {pd[2], pd[3], pd[6], pd[7]}};
      return;
    }
    if (op == "MaxPool") {
      const std::string x = in_name(n.in[0]);
      const auto& xd = dims(x);
      if (n.out.size() > 1) fail(DW_ERR_UNSUPPORTED, "onnx: MaxPool indices output");
      if (n.get_int("ceil_mode", 0)) fail(DW_ERR_UNSUPPORTED, "onnx: MaxPool ceil_mode");
      dw_op_params p = params(DW_OP_MAXPOOL);
      const auto ks = n.get_ints("kernel_shape");
      auto st = n.get_ints("strides");
      auto pd = n.get_ints("pads");
      if (ks.size() != 2) fail(DW_ERR_UNSUPPORTED, "onnx: MaxPool kernel_shape");
      if (st.empty()) st = {1, 1};
      if (pd.empty()) pd.assign(4, 0);
      p.kernel_shape[0] = (int)ks[0]; p.kernel_shape[1] = (int)ks[1];
      p.strides[0] = (int)st[0]; p.strides[1] = (int)st[1];
      for (int k = 0; k < 4; ++k) p.pads[k] = (int)pd[k];
      declare(n.out[0], {xd[0], xd[1], (xd[2] + pd[0] + pd[2] - ks[0]) / st[0] + 1,
                         (xd[3] + pd[1] + pd[3] - ks[1]) / st[1] + 1});
      add(n.name, "MaxPool", {x}, {n.out[0]}, p);
      return;
    }
    if (op == "Concat") {
      bool all_const = true;
      for (auto& i : n.in) all_const = all_const && is_const(i);
      if (all_const) {
        std::vector<double> v;
        int dt = DT_INT64;
        for (auto& i : n.in) {
          const Tensor& t = *const_of(i);
          if (t.dims.size() > 1) fail(DW_ERR_UNSUPPORTED, "onnx: Concat " + n.name + " of constants above rank 1");
          if (t.dtype != DT_INT64 && t.dtype != DT_INT32) dt = DT_FLOAT;
          const auto tv = const_values(t);
          v.insert(v.end(), tv.begin(), tv.end());
        }
        const_from_values(n.out[0], {(int64_t)v.size()}, dt, v);
        return;
      }
      std::vector<std::string> ins;
      for (auto& i : n.in) ins.push_back(in_name(i));
      auto d = dims(ins[0]);
      int64_t axis = n.get_int("axis", 1);
      if (axis < 0) axis += (int64_t)d.size();
      d[axis] = 0;
      for (auto& i : ins) d[axis] += dims(i)[axis];
      dw_op_params p = params(DW_OP_CONCAT);
      p.axis = (int)axis;
      declare(n.out[0], d);
      add(n.name, "Concat", ins, {n.out[0]}, p);
      return;
    }
    if (op == "Split") {
      const std::string x = in_name(n.in[0]);
      const auto xd = dims(x);
      int64_t axis = n.get_int("axis", 0);
      if (axis < 0) axis += (int64_t)xd.size();
      std::vector<int64_t> sizes = n.get_ints("split");
      if (n.in.size() > 1 && !n.in[1].empty()) sizes = const_ints(n.in[1]);
      if (sizes.empty()) sizes.assign(n.out.size(), xd[axis] / (int64_t)n.out.size());
      if (sizes.size() != n.out.size() || sizes.size() > 8) fail(DW_ERR_UNSUPPORTED, "onnx: Split " + n.name);
      dw_op_params p = params(DW_OP_SPLIT);
      p.axis = (int)axis;
      p.num_splits = (int)sizes.size();
      for (size_t k = 0; k < sizes.size(); ++k) {
        p.split_sizes[k] = (int)sizes[k];
        auto d = xd;
        d[axis] = sizes[k];
        declare(n.out[k], d);
      }
      add(n.name, "Split", {x}, n.out, p);
      return;
    }
    if (op == "Resize" || op == "Upsample") {
      const std::string x = in_name(n.in[0]);
      const auto& xd = dims(x);
      if (n.get_string("mode", "nearest") != "nearest") fail(DW_ERR_UNSUPPORTED, "onnx: Resize mode");
      int64_t oh = 0, ow = 0;
      // Resize (opset 11+): X, roi, scales, sizes; Upsample: X, scales
      const std::string scales = op == "Upsample" ? (n.in.size() > 1 ? n.in[1] : "") : (n.in.size() > 2 ? n.in[2] : "");
      const std::string sizes = op == "Resize" && n.in.size() > 3 ? n.in[3] : "";
      if (!sizes.empty() && const_of(sizes) && const_of(sizes)->numel() == 4) {
        const auto s = const_ints(sizes);
        oh = s[2];
        ow = s[3];
      } else if (!scales.empty() && const_of(scales) && const_of(scales)->numel() == 4) {
        const auto s = const_floats(scales);
        oh = (int64_t)floorf((float)xd[2] * s[2]);
        ow = (int64_t)floorf((float)xd[3] * s[3]);
      } else {
        fail(DW_ERR_UNSUPPORTED, "onnx: Resize " + n.name + " needs constant scales or sizes");
      }
      dw_op_params p = params(DW_OP_RESIZE);
      p.out_h = (int)oh;
      p.out_w = (int)ow;
      p.mode_nearest = 1;
      declare(n.out[0], {xd[0], xd[1], oh, ow});
      add(n.name, "Resize", {x}, {n.out[0]}, p);
      return;
    }
    if (op == "BatchNormalization") {
      const std::string x = in_name(n.in[0]);
      dw_op_params p = params(DW_OP_BATCHNORM);
      p.epsilon = n.get_float("epsilon", 1e-5f);
      std::vector<std::string> ins{x};
      for (int k = 1; k < 5; ++k) ins.push_back(in_name(n.in[k]));
      out_like(n, x);
      add(n.name, "BatchNormalization", ins, {n.out[0]}, p);
      return;
    }
    if (op == "GlobalAveragePool") {
      const std::string x = in_name(n.in[0]);
      const auto& xd = dims(x);
      declare(n.out[0], {xd[0], xd[1], 1, 1});
      add(n.name, "GlobalAveragePool", {x}, {n.out[0]}, params(DW_OP_GLOBAL_AVG_POOL));
      return;
    }
    if (op == "Flatten") {
      const std::string x = in_name(n.in[0]);
      const auto& xd = dims(x);
      int64_t axis = n.get_int("axis", 1);
      if (axis < 0) axis += (int64_t)xd.size();
      int64_t a = 1, b = 1;
      for (int64_t k = 0; k < (int64_t)xd.size(); ++k) (k < axis ? a : b) *= xd[k];
      declare(n.out[0], {a, b});
      add(n.name, "Flatten", {x}, {n.out[0]}, params(DW_OP_NONE));
      return;
    }
    if (op == "Reshape") {
      const std::string x = in_name(n.in[0]);
      const auto& xd = dims(x);
      auto shp = const_ints(n.in[1]);
      int64_t total = 1, known = 1, infer = -1;
      for (auto d : xd) total *= d;
      for (size_t k = 0; k < shp.size(); ++k) {
        if (shp[k] == 0 && k < xd.size()) shp[k] = xd[k];
        if (shp[k] == -1) infer = (int64_t)k;
        else known *= shp[k];
      }
      if (infer >= 0) shp[infer] = total / known;
      declare(n.out[0], shp);
      add(n.name, "Reshape", {x}, {n.out[0]}, params(DW_OP_RESHAPE));
      return;
    }
    if (op == "Softmax") {
      const std::string x = in_name(n.in[0]);
      const auto xd = dims(x);
      const int64_t r = (int64_t)xd.size();
      int64_t axis = n.get_int("axis", m.opset >= 13 ? -1 : 1);
      if (axis < 0) axis += r;
      if (axis < 0 || axis >= r) fail(DW_ERR_INVALID, "onnx: Softmax " + n.name + " axis");
      if (m.opset < 13) {
        // opset < 13: softmax over the flattened dimensions from axis on,
        // which is the per-axis softmax when every later dimension is 1
        for (int64_t k = axis + 1; k < r; ++k)
          if (xd[k] != 1) fail(DW_ERR_UNSUPPORTED, "onnx: opset < 13 Softmax " + n.name + " over several axes");
      }
      dw_op_params p = params(DW_OP_SOFTMAX);
      p.axis = (int)axis;
      out_like(n, x);
      add(n.name, "Softmax", {x}, {n.out[0]}, p);
      return;
    }
    if (op == "Gemm" || op == "MatMul") {
      const std::string a = in_name(n.in[0]), b = in_name(n.in[1]);
      const auto& ad = dims(a);
      const auto& bd = dims(b);
      if (ad.size() != 2 || bd.size() != 2) fail(DW_ERR_UNSUPPORTED, "onnx: " + op + " operands must be 2-D");
      dw_op_params p = params(op == "Gemm" ? DW_OP_GEMM : DW_OP_NONE);
      int64_t ta = 0, tb = 0;
      if (op == "Gemm") {
        ta = n.get_int("transA", 0);
        tb = n.get_int("transB", 0);
        p.alpha = n.get_float("alpha", 1.0f);
        p.beta = n.get_float("beta", 1.0f);
        if (p.alpha != 1.0f || p.beta != 1.0f) fail(DW_ERR_UNSUPPORTED, "onnx: Gemm alpha/beta other than 1");
        p.trans_a = (int)ta;
        p.trans_b = (int)tb;
      }
      const int64_t mm = ta ? ad[1] : ad[0];
      const int64_t nn = tb ? bd[0] : bd[1];
      declare(n.out[0], {mm, nn});
      std::vector<std::string> ins{a, b};
      if (op == "Gemm" && n.in.size() > 2 && !n.in[2].empty()) ins.push_back(in_name(n.in[2]));
      add(n.name, op, ins, {n.out[0]}, p);
      return;
    }
    fail(DW_ERR_UNSUPPORTED, "onnx: op type '" + op + "' (" + n.name + ") is not supported");
  }
};

}  // namespace onnx
}  // namespace dw

// ===========================================================================
// C ABI
// ===========================================================================
namespace dw {
void set_last_error(const std::string& m);
}

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

extern "C" {

int dw_onnx_inspect(const void* bytes, size_t len, char* buf, size_t cap, size_t* need) {
  API_BEGIN
  if (!bytes && len) dw::fail(DW_ERR_INVALID, "null bytes");
  const dw::onnx::Model m = dw::onnx::parse_model((const uint8_t*)bytes, len);
  const std::string s = dw::onnx::inspect(m);
  if (need) *need = s.size() + 1;
  if (buf && cap) {
    const size_t k = std::min(cap - 1, s.size());
    memcpy(buf, s.data(), k);
    buf[k] = 0;
    if (k < s.size()) dw::fail(DW_ERR_INVALID, "inspect: buffer too small");
  }
  API_END
}

int dw_graph_from_onnx(const void* bytes, size_t len, dw_graph** out) {
  API_BEGIN
  if (!out || (!bytes && len)) dw::fail(DW_ERR_INVALID, "null argument");
  const dw::onnx::Model m = dw::onnx::parse_model((const uint8_t*)bytes, len);
  dw_graph* g = new dw_graph();
  try {
    g->g.dtype = DW_GRAPH_F32;
    dw::onnx::Builder b(m, g->g);
    b.build();
  } catch (...) {
    delete g;
    throw;
  }
  *out = g;
  API_END
}

}  // extern "C"
