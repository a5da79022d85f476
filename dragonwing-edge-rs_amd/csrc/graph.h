// Graph IR: the C++ form of dragonwing_onnx::Graph / CompiledOp / OpParams
// (crates/dragonwing-onnx/src/graph.rs:18-31, builder.rs:204-361), plus
// per-tensor element types and quantization parameters for the u8 graphs.
#pragma once

#include <stdint.h>

#include <map>
#include <string>
#include <vector>

#include "../../include/dw_hip.h"

namespace dw {

struct TensorInfo {
  std::vector<int64_t> dims;
  int dtype = 0;            // DW_DTYPE_*
  bool is_init = false;
  std::vector<uint8_t> data;
  // u8 activations: real = (q - zp) * scale
  bool has_q = false;
  float scale = 1.0f;
  int zp = 0;
  // s8 weights: per-output-channel scales (zero point 0)
  std::vector<float> ch_scales;
  // calibration range (calibration.rs:56-69)
  bool has_range = false;
  float rmin = 0.0f, rmax = 0.0f;
  // quantization fixed by the model (QDQ import): an f32 activation whose
  // scale / zp (has_q) quantize_qdq takes as given
  bool q_fixed = false;
  // an initializer holding integers as exact f32 values (a dequantized int8
  // weight or int32 bias of a QDQ model) with their scales in ch_scales
  // (one, or one per index of dimension q_axis of the original layout)
  bool prequant = false;
  bool prequant_i32 = false;
  int q_axis = -1;

  int64_t numel() const {
    int64_t n = 1;
    for (auto d : dims) n *= d;
    return n;
  }
};

struct OpNode {
  std::string name;
  std::string type;
  std::vector<std::string> in, out;
  dw_op_params p{};
};

struct GraphIR {
  int dtype = DW_GRAPH_F32;
  std::map<std::string, TensorInfo> t;
  std::vector<OpNode> ops;
  std::vector<std::string> inputs, outputs;
  std::string json;  // cache for dw_graph_to_json

  TensorInfo& tensor(const std::string& name);
  const TensorInfo& tensor(const std::string& name) const;
  bool has(const std::string& name) const { return t.count(name) != 0; }
  // ops consuming `name` (indices into ops)
  std::vector<int> consumers(const std::string& name) const;
  int producer(const std::string& name) const;
  bool is_output(const std::string& name) const;
};

// Quantized SiLU table: lut[q] = clamp(rint(silu((q - zx) * sx) / sy) + zy)
// with silu(v) = v * (1 / (1 + expf(-v))) (Sigmoid then Mul in f32).
void build_silu_lut(uint8_t lut[256], float sx, int zx, float sy, int zy);

// F16::from_f32 (crates/dragonwing-core/src/dtype.rs:164-222): IEEE binary16,
// round to nearest even.
uint16_t f16_bits_from_f32(float v);

}  // namespace dw

// The opaque C handle wraps the IR.
struct dw_graph {
  dw::GraphIR g;
};
