// Native ONNX reader: protobuf wire format (varint, 64-bit, length-delimited,
// 32-bit records) decoded directly into the IR. Field numbers are those of
// the public ONNX schema (onnx/onnx.proto, IR version 3 and later).
#include "cutriton/ir/onnx_import.h"

#include <cstring>
#include <fstream>
#include <iterator>
#include <memory>
#include <optional>
#include <sstream>
#include <unordered_set>
#include <vector>

#include "cutriton/core/buffer.h"

namespace cutriton {
namespace {

// ---- protobuf wire format ------------------------------------------------

enum WireType : uint32_t { kVarint = 0, kFixed64 = 1, kBytes = 2, kFixed32 = 5 };

struct Span {
  const uint8_t* data{nullptr};
  std::size_t size{0};
  std::string str() const { return std::string(reinterpret_cast<const char*>(data), size); }
};

class Reader {
 public:
  explicit Reader(Span span) : p_(span.data), end_(span.data + span.size) {}

  bool done() const { return p_ == end_; }

  // Next field: number and wire type. False on malformed data.
  bool Tag(uint32_t* field, uint32_t* wire) {
    uint64_t key = 0;
    if (!Varint(&key) || (key >> 3) == 0 || (key >> 3) > 0x1fffffffu) return false;
    *field = static_cast<uint32_t>(key >> 3);
    *wire = static_cast<uint32_t>(key & 7);
    return true;
  }

  bool Varint(uint64_t* value) {
    uint64_t v = 0;
    for (int shift = 0; shift < 64; shift += 7) {
      if (p_ == end_) return false;
      const uint8_t byte = *p_++;
      v |= static_cast<uint64_t>(byte & 0x7f) << shift;
      if ((byte & 0x80) == 0) {
        *value = v;
        return true;
      }
    }
    return false;
  }

  bool Fixed32(uint32_t* value) {
    if (end_ - p_ < 4) return false;
    std::memcpy(value, p_, 4);
    p_ += 4;
    return true;
  }

  bool Fixed64(uint64_t* value) {
    if (end_ - p_ < 8) return false;
    std::memcpy(value, p_, 8);
    p_ += 8;
    return true;
  }

  bool Bytes(Span* span) {
    uint64_t length = 0;
    if (!Varint(&length) || length > static_cast<uint64_t>(end_ - p_)) return false;
    *span = Span{p_, static_cast<std::size_t>(length)};
    p_ += length;
    return true;
  }

  bool Skip(uint32_t wire) {
    uint64_t ignored64 = 0;
    uint32_t ignored32 = 0;
    Span ignored;
    switch (wire) {
      case kVarint: return Varint(&ignored64);
      case kFixed64: return Fixed64(&ignored64);
      case kBytes: return Bytes(&ignored);
      case kFixed32: return Fixed32(&ignored32);
      default: return false;  // groups (3, 4) are not used by ONNX
    }
  }

 private:
  const uint8_t* p_;
  const uint8_t* end_;
};

Status Malformed(const std::string& what) { return Status::InvalidArgument("malformed ONNX model: " + what); }

// Appends the values of a repeated integer field, packed or not.
bool ReadInts(Reader& r, uint32_t wire, std::vector<int64_t>* out) {
  uint64_t v = 0;
  if (wire == kVarint) {
    if (!r.Varint(&v)) return false;
    out->push_back(static_cast<int64_t>(v));
    return true;
  }
  if (wire != kBytes) return false;
  Span packed;
  if (!r.Bytes(&packed)) return false;
  Reader inner(packed);
  while (!inner.done()) {
    if (!inner.Varint(&v)) return false;
    out->push_back(static_cast<int64_t>(v));
  }
  return true;
}

// Appends the values of a repeated float field, packed or not.
bool ReadFloats(Reader& r, uint32_t wire, std::vector<float>* out) {
  uint32_t bits = 0;
  auto push = [&] {
    float f;
    std::memcpy(&f, &bits, 4);
    out->push_back(f);
  };
  if (wire == kFixed32) {
    if (!r.Fixed32(&bits)) return false;
    push();
    return true;
  }
  if (wire != kBytes) return false;
  Span packed;
  if (!r.Bytes(&packed) || packed.size % 4 != 0) return false;
  Reader inner(packed);
  while (!inner.done()) {
    if (!inner.Fixed32(&bits)) return false;
    push();
  }
  return true;
}

// Appends the values of a repeated double field, packed or not.
bool ReadDoubles(Reader& r, uint32_t wire, std::vector<double>* out) {
  uint64_t bits = 0;
  auto push = [&] {
    double d;
    std::memcpy(&d, &bits, 8);
    out->push_back(d);
  };
  if (wire == kFixed64) {
    if (!r.Fixed64(&bits)) return false;
    push();
    return true;
  }
  if (wire != kBytes) return false;
  Span packed;
  if (!r.Bytes(&packed) || packed.size % 8 != 0) return false;
  Reader inner(packed);
  while (!inner.done()) {
    if (!inner.Fixed64(&bits)) return false;
    push();
  }
  return true;
}

// ---- ONNX messages --------------------------------------------------------

// TensorProto.DataType values that have an engine dtype.
constexpr int kOnnxFloat = 1, kOnnxInt32 = 6, kOnnxInt64 = 7, kOnnxFloat16 = 10;

std::optional<DataType> EngineType(int onnx_type) {
  switch (onnx_type) {
    case kOnnxFloat: return DataType::kFloat32;
    case kOnnxFloat16: return DataType::kFloat16;
    case kOnnxInt32: return DataType::kInt32;
    case kOnnxInt64: return DataType::kInt64;
    default: return std::nullopt;
  }
}

struct TensorData {
  std::string name;
  std::vector<int64_t> dims;
  int data_type{0};
  Span raw;
  bool has_raw{false};
  std::vector<float> floats;
  std::vector<int64_t> int32s;  // int32_data also carries FLOAT16 bit patterns
  std::vector<int64_t> int64s;
  std::vector<double> doubles;
  bool external{false};
};

Status ParseTensor(Span span, TensorData* t) {
  Reader r(span);
  while (!r.done()) {
    uint32_t field = 0, wire = 0;
    if (!r.Tag(&field, &wire)) return Malformed("TensorProto");
    bool ok = true;
    Span s;
    uint64_t v = 0;
    switch (field) {
      case 1: ok = ReadInts(r, wire, &t->dims); break;
      case 2: ok = wire == kVarint && r.Varint(&v); t->data_type = static_cast<int>(v); break;
      case 4: ok = ReadFloats(r, wire, &t->floats); break;
      case 5: ok = ReadInts(r, wire, &t->int32s); break;
      case 7: ok = ReadInts(r, wire, &t->int64s); break;
      case 8: ok = wire == kBytes && r.Bytes(&s); t->name = s.str(); break;
      case 9: ok = wire == kBytes && r.Bytes(&t->raw); t->has_raw = true; break;
      case 10: ok = ReadDoubles(r, wire, &t->doubles); break;
      case 13: t->external = true; ok = r.Skip(wire); break;  // external_data
      case 14:  // data_location: 1 = EXTERNAL
        ok = wire == kVarint && r.Varint(&v);
        if (v == 1) t->external = true;
        break;
      default: ok = r.Skip(wire);
    }
    if (!ok) return Malformed("TensorProto field " + std::to_string(field));
  }
  return Status::OK();
}

// Host tensor of `t`'s dims and data in the engine dtype.
Status ToHostTensor(const TensorData& t, Tensor* out) {
  if (t.external) return Status::Unsupported("ONNX tensor with external data: " + t.name);
  const std::optional<DataType> dtype = EngineType(t.data_type);
  if (!dtype) {
    return Status::Unsupported("ONNX tensor data type " + std::to_string(t.data_type) + " of " + t.name +
                               " (FLOAT, FLOAT16, INT32 and INT64 are supported)");
  }
  for (const int64_t d : t.dims) {
    if (d < 0) return Malformed("negative dimension in tensor " + t.name);
  }
  TensorDesc desc(t.dims, *dtype, DeviceType::kCPU, 0, "");
  const std::size_t element = ElementSize(*dtype);
  // The data the file supplies bounds the element count before anything is
  // allocated, so dims that claim more than the file holds are rejected.
  const std::size_t supplied = t.has_raw ? t.raw.size / element
                               : *dtype == DataType::kFloat32 ? t.floats.size()
                               : *dtype == DataType::kInt64   ? t.int64s.size()
                                                              : t.int32s.size();
  std::size_t n = 1;
  for (const int64_t d : t.dims) {
    if (d != 0 && n > supplied / static_cast<std::size_t>(d)) n = supplied + 1;  // more than supplied
    else n *= static_cast<std::size_t>(d);
  }
  const std::size_t bytes = n * element;
  auto mismatch = [&] { return Malformed("element count of tensor " + t.name + " does not match its dims"); };
  if (n != supplied || (t.has_raw && t.raw.size != bytes)) return mismatch();
  auto buffer = Buffer::AllocateHost(bytes);
  auto* dst = static_cast<uint8_t*>(buffer->data());
  if (t.has_raw) {
    if (bytes != 0) std::memcpy(dst, t.raw.data, bytes);  // little endian, as the host
  } else if (*dtype == DataType::kFloat32) {
    if (n != 0) std::memcpy(dst, t.floats.data(), bytes);
  } else if (*dtype == DataType::kFloat16 || *dtype == DataType::kInt32) {
    for (std::size_t i = 0; i < n; ++i) {
      if (*dtype == DataType::kFloat16) {
        const uint16_t bits = static_cast<uint16_t>(t.int32s[i]);
        std::memcpy(dst + 2 * i, &bits, 2);
      } else {
        const int32_t value = static_cast<int32_t>(t.int32s[i]);
        std::memcpy(dst + 4 * i, &value, 4);
      }
    }
  } else {
    if (n != 0) std::memcpy(dst, t.int64s.data(), bytes);
  }
  *out = Tensor(desc, std::move(buffer));
  return Status::OK();
}

struct AttributeData {
  std::string name;
  int type{0};  // AttributeProto.AttributeType
  bool has_f{false}, has_i{false}, has_s{false}, has_t{false}, has_g{false};
  float f{0.0f};
  int64_t i{0};
  std::string s;
  TensorData t;
  std::vector<float> floats;
  std::vector<int64_t> ints;
  int strings{0};
};

// AttributeProto.AttributeType values.
constexpr int kAttrFloat = 1, kAttrInt = 2, kAttrString = 3, kAttrTensor = 4, kAttrGraph = 5, kAttrFloats = 6,
              kAttrInts = 7;

Status ParseAttribute(Span span, AttributeData* a) {
  Reader r(span);
  while (!r.done()) {
    uint32_t field = 0, wire = 0;
    if (!r.Tag(&field, &wire)) return Malformed("AttributeProto");
    bool ok = true;
    Span s;
    uint64_t v = 0;
    uint32_t bits = 0;
    switch (field) {
      case 1: ok = wire == kBytes && r.Bytes(&s); a->name = s.str(); break;
      case 2:
        ok = wire == kFixed32 && r.Fixed32(&bits);
        std::memcpy(&a->f, &bits, 4);
        a->has_f = true;
        break;
      case 3: ok = wire == kVarint && r.Varint(&v); a->i = static_cast<int64_t>(v); a->has_i = true; break;
      case 4: ok = wire == kBytes && r.Bytes(&s); a->s = s.str(); a->has_s = true; break;
      case 5:
        ok = wire == kBytes && r.Bytes(&s);
        if (ok) {
          CUTRITON_RETURN_IF_ERROR(ParseTensor(s, &a->t));
        }
        a->has_t = true;
        break;
      case 6: a->has_g = true; ok = r.Skip(wire); break;
      case 7: ok = ReadFloats(r, wire, &a->floats); break;
      case 8: ok = ReadInts(r, wire, &a->ints); break;
      case 9: ++a->strings; ok = r.Skip(wire); break;
      case 20: ok = wire == kVarint && r.Varint(&v); a->type = static_cast<int>(v); break;
      default: ok = r.Skip(wire);
    }
    if (!ok) return Malformed("AttributeProto field " + std::to_string(field) + " of " + a->name);
  }
  if (a->type == 0) {  // IR version 1 files carry no type: infer it from the field that is set
    a->type = a->has_f ? kAttrFloat : a->has_i ? kAttrInt : a->has_s ? kAttrString : a->has_t ? kAttrTensor
              : a->has_g ? kAttrGraph : !a->floats.empty() ? kAttrFloats : !a->ints.empty() ? kAttrInts : 0;
  }
  return Status::OK();
}

struct NodeData {
  std::string name, op_type, domain;
  std::vector<std::string> inputs, outputs;
  std::vector<AttributeData> attributes;
};

Status ParseNode(Span span, NodeData* n) {
  Reader r(span);
  while (!r.done()) {
    uint32_t field = 0, wire = 0;
    if (!r.Tag(&field, &wire)) return Malformed("NodeProto");
    bool ok = true;
    Span s;
    switch (field) {
      case 1: ok = wire == kBytes && r.Bytes(&s); n->inputs.push_back(s.str()); break;
      case 2: ok = wire == kBytes && r.Bytes(&s); n->outputs.push_back(s.str()); break;
      case 3: ok = wire == kBytes && r.Bytes(&s); n->name = s.str(); break;
      case 4: ok = wire == kBytes && r.Bytes(&s); n->op_type = s.str(); break;
      case 5:
        ok = wire == kBytes && r.Bytes(&s);
        if (ok) {
          n->attributes.emplace_back();
          CUTRITON_RETURN_IF_ERROR(ParseAttribute(s, &n->attributes.back()));
        }
        break;
      case 7: ok = wire == kBytes && r.Bytes(&s); n->domain = s.str(); break;
      default: ok = r.Skip(wire);
    }
    if (!ok) return Malformed("NodeProto field " + std::to_string(field));
  }
  return Status::OK();
}

struct Dim {
  std::optional<int64_t> value;
  std::string param;
};

struct ValueInfoData {
  std::string name;
  int elem_type{0};
  bool has_shape{false};
  std::vector<Dim> dims;
};

Status ParseDimension(Span span, Dim* d) {
  Reader r(span);
  while (!r.done()) {
    uint32_t field = 0, wire = 0;
    if (!r.Tag(&field, &wire)) return Malformed("TensorShapeProto.Dimension");
    bool ok = true;
    Span s;
    uint64_t v = 0;
    if (field == 1) {
      ok = wire == kVarint && r.Varint(&v);
      d->value = static_cast<int64_t>(v);
    } else if (field == 2) {
      ok = wire == kBytes && r.Bytes(&s);
      d->param = s.str();
    } else {
      ok = r.Skip(wire);
    }
    if (!ok) return Malformed("TensorShapeProto.Dimension");
  }
  return Status::OK();
}

// Walks ValueInfoProto.type (TypeProto) -> tensor_type -> elem_type, shape.
Status ParseValueInfo(Span span, ValueInfoData* v) {
  Reader r(span);
  while (!r.done()) {
    uint32_t field = 0, wire = 0;
    if (!r.Tag(&field, &wire)) return Malformed("ValueInfoProto");
    Span s;
    if (field == 1) {
      if (wire != kBytes || !r.Bytes(&s)) return Malformed("ValueInfoProto.name");
      v->name = s.str();
      continue;
    }
    if (field != 2) {
      if (!r.Skip(wire)) return Malformed("ValueInfoProto");
      continue;
    }
    if (wire != kBytes || !r.Bytes(&s)) return Malformed("ValueInfoProto.type");
    Reader type(s);
    while (!type.done()) {
      uint32_t tf = 0, tw = 0;
      if (!type.Tag(&tf, &tw)) return Malformed("TypeProto");
      Span ts;
      if (tf != 1) {  // only tensor_type
        if (!type.Skip(tw)) return Malformed("TypeProto");
        continue;
      }
      if (tw != kBytes || !type.Bytes(&ts)) return Malformed("TypeProto.tensor_type");
      Reader tensor(ts);
      while (!tensor.done()) {
        uint32_t ef = 0, ew = 0;
        if (!tensor.Tag(&ef, &ew)) return Malformed("TypeProto.Tensor");
        uint64_t value = 0;
        Span shape;
        if (ef == 1) {
          if (ew != kVarint || !tensor.Varint(&value)) return Malformed("TypeProto.Tensor.elem_type");
          v->elem_type = static_cast<int>(value);
        } else if (ef == 2) {
          if (ew != kBytes || !tensor.Bytes(&shape)) return Malformed("TypeProto.Tensor.shape");
          v->has_shape = true;
          Reader dims(shape);
          while (!dims.done()) {
            uint32_t df = 0, dw = 0;
            if (!dims.Tag(&df, &dw)) return Malformed("TensorShapeProto");
            Span ds;
            if (df != 1) {
              if (!dims.Skip(dw)) return Malformed("TensorShapeProto");
              continue;
            }
            if (dw != kBytes || !dims.Bytes(&ds)) return Malformed("TensorShapeProto.dim");
            v->dims.emplace_back();
            CUTRITON_RETURN_IF_ERROR(ParseDimension(ds, &v->dims.back()));
          }
        } else if (!tensor.Skip(ew)) {
          return Malformed("TypeProto.Tensor");
        }
      }
    }
  }
  return Status::OK();
}

struct GraphData {
  std::vector<NodeData> nodes;
  std::vector<TensorData> initializers;
  std::vector<ValueInfoData> inputs, outputs;
  bool sparse{false};
};

Status ParseGraph(Span span, GraphData* g) {
  Reader r(span);
  while (!r.done()) {
    uint32_t field = 0, wire = 0;
    if (!r.Tag(&field, &wire)) return Malformed("GraphProto");
    Span s;
    bool ok = true;
    switch (field) {
      case 1:
        ok = wire == kBytes && r.Bytes(&s);
        if (ok) {
          g->nodes.emplace_back();
          CUTRITON_RETURN_IF_ERROR(ParseNode(s, &g->nodes.back()));
        }
        break;
      case 5:
        ok = wire == kBytes && r.Bytes(&s);
        if (ok) {
          g->initializers.emplace_back();
          CUTRITON_RETURN_IF_ERROR(ParseTensor(s, &g->initializers.back()));
        }
        break;
      case 11:
      case 12:
        ok = wire == kBytes && r.Bytes(&s);
        if (ok) {
          auto& list = field == 11 ? g->inputs : g->outputs;
          list.emplace_back();
          CUTRITON_RETURN_IF_ERROR(ParseValueInfo(s, &list.back()));
        }
        break;
      case 15: g->sparse = true; ok = r.Skip(wire); break;
      default: ok = r.Skip(wire);
    }
    if (!ok) return Malformed("GraphProto field " + std::to_string(field));
  }
  return Status::OK();
}

// ---- mapping onto the IR ---------------------------------------------------

bool DefaultDomain(const std::string& domain) { return domain.empty() || domain == "ai.onnx"; }

// Refuses attribute values whose meaning the engine's op would drop.
Status CheckSupported(const NodeData& n, const Node& node) {
  const std::string& op = n.op_type;
  auto refuse = [&](const std::string& what) {
    return Status::Unsupported("ONNX node " + node.name() + " (" + op + "): " + what);
  };
  if (op == "Conv" || op == "MaxPool") {
    if (const auto pad = node.GetAttribute<std::string>("auto_pad"); pad && *pad != "NOTSET") {
      return refuse("auto_pad " + *pad + " (explicit pads are supported)");
    }
  }
  if (op == "Conv" && GetIntAttribute(node, "group", 1) != 1) return refuse("grouped convolution");
  if (op == "MaxPool" && GetIntAttribute(node, "ceil_mode", 0) != 0) return refuse("ceil_mode 1");
  if (op == "Gemm") {
    for (const char* key : {"alpha", "beta"}) {
      if (const auto v = node.GetAttribute<double>(key); v && *v != 1.0) {
        return refuse(std::string(key) + " other than 1");
      }
    }
  }
  if (op == "Gelu") {
    if (const auto a = node.GetAttribute<std::string>("approximate"); a && *a != "none") {
      return refuse("approximate " + *a + " (the erf form is supported)");
    }
  }
  return Status::OK();
}

// Conv(x, W, b) as Conv(x, W) followed by BatchNormalization with scale 1,
// mean 0, variance 1 and epsilon 0, i.e. y + b exactly (the factor
// 1 / sqrt(1 + 0) is 1). The engine's Conv takes no bias, and its
// Conv + BatchNormalization fusion then serves the pair with one kernel.
// The bias must be a rank-1 constant of the weight's output channels.
Status AddConvBias(Node conv, Model* model) {
  const std::string weight_name = conv.inputs()[1], bias_name = conv.inputs()[2];
  const auto weight = model->constants().find(weight_name);
  const auto bias = model->constants().find(bias_name);
  if (weight == model->constants().end() || bias == model->constants().end() ||
      weight->second.desc().shape.empty() ||
      bias->second.desc().shape != std::vector<int64_t>{weight->second.desc().shape[0]}) {
    return Status::Unsupported("ONNX Conv " + conv.name() + ": the bias must be a constant of the output channels");
  }
  const TensorDesc& bias_desc = bias->second.desc();
  const int64_t channels = bias_desc.shape[0];
  auto filled = [&](const std::string& suffix, double value) -> Status {
    auto buffer = Buffer::AllocateHost(bias_desc.ByteSize());
    for (int64_t c = 0; c < channels; ++c) {
      if (bias_desc.dtype == DataType::kFloat32) {
        static_cast<float*>(buffer->data())[c] = static_cast<float>(value);
      } else if (bias_desc.dtype == DataType::kFloat16) {
        const uint16_t bits = value == 0.0 ? 0x0000 : 0x3c00;  // 0 or 1 in binary16
        std::memcpy(static_cast<uint8_t*>(buffer->data()) + 2 * c, &bits, 2);
      } else {
        return Status::Unsupported("ONNX Conv " + conv.name() + ": bias of an integer type");
      }
    }
    return model->AddConstant(conv.name() + "::bias_" + suffix, Tensor(bias_desc, std::move(buffer)));
  };
  CUTRITON_RETURN_IF_ERROR(filled("scale", 1.0));
  CUTRITON_RETURN_IF_ERROR(filled("mean", 0.0));
  CUTRITON_RETURN_IF_ERROR(filled("variance", 1.0));
  const std::string output = conv.outputs().at(0);
  const std::string conv_out = conv.name() + "::without_bias";
  Node bn(conv.name() + "::bias", "BatchNormalization",
          {conv_out, conv.name() + "::bias_scale", bias_name, conv.name() + "::bias_mean",
           conv.name() + "::bias_variance"},
          {output});
  bn.SetAttribute("epsilon", 0.0);
  conv.set_inputs({conv.inputs()[0], weight_name});
  conv.set_outputs({conv_out});
  CUTRITON_RETURN_IF_ERROR(model->graph().AddNode(std::move(conv)));
  return model->graph().AddNode(std::move(bn));
}

Status BuildModel(const GraphData& g, int64_t opset, const OnnxDimValues& dim_values, Model* model) {
  if (g.sparse) return Status::Unsupported("ONNX sparse initializers");
  Graph& graph = model->graph();
  std::unordered_set<std::string> constant_names;
  for (const TensorData& t : g.initializers) {
    Tensor tensor;
    CUTRITON_RETURN_IF_ERROR(ToHostTensor(t, &tensor));
    CUTRITON_RETURN_IF_ERROR(model->AddConstant(t.name, std::move(tensor)));
    constant_names.insert(t.name);
  }
  for (const ValueInfoData& v : g.inputs) {
    if (constant_names.count(v.name) != 0) continue;  // IR < 4 lists initializers as inputs too
    const std::optional<DataType> dtype = EngineType(v.elem_type);
    if (!dtype) return Status::Unsupported("ONNX input " + v.name + " has data type " + std::to_string(v.elem_type));
    if (!v.has_shape) return Status::InvalidArgument("ONNX input " + v.name + " has no shape");
    std::vector<int64_t> shape;
    for (const Dim& d : v.dims) {
      if (d.value) {
        shape.push_back(*d.value);
      } else if (const auto it = dim_values.find(d.param); !d.param.empty() && it != dim_values.end()) {
        shape.push_back(it->second);
      } else {
        return Status::InvalidArgument("ONNX input " + v.name + " has a symbolic dimension '" + d.param +
                                       "' without a value");
      }
    }
    const std::string layout = shape.size() == 4 ? "NCHW" : "";
    CUTRITON_RETURN_IF_ERROR(graph.AddInput(v.name, TensorDesc(std::move(shape), *dtype, DeviceType::kCPU, 0, layout)));
  }
  for (std::size_t index = 0; index < g.nodes.size(); ++index) {
    const NodeData& n = g.nodes[index];
    if (!DefaultDomain(n.domain)) {
      return Status::Unsupported("ONNX node " + n.name + " of domain " + n.domain);
    }
    if (n.op_type == "Constant") {
      const AttributeData* value = nullptr;
      for (const auto& a : n.attributes) {
        if (a.name == "value" && a.type == kAttrTensor) value = &a;
      }
      if (value == nullptr || n.outputs.size() != 1) {
        return Status::Unsupported("ONNX Constant node " + n.name + " without a tensor 'value'");
      }
      Tensor tensor;
      CUTRITON_RETURN_IF_ERROR(ToHostTensor(value->t, &tensor));
      CUTRITON_RETURN_IF_ERROR(model->AddConstant(n.outputs[0], std::move(tensor)));
      continue;
    }
    // Optional inputs left empty at the end of the list are dropped; an empty
    // one before a given input cannot be expressed.
    std::vector<std::string> inputs = n.inputs;
    while (!inputs.empty() && inputs.back().empty()) inputs.pop_back();
    for (const auto& in : inputs) {
      if (in.empty()) return Status::Unsupported("ONNX node " + n.name + " skips an optional input");
    }
    std::vector<std::string> outputs = n.outputs;
    while (!outputs.empty() && outputs.back().empty()) outputs.pop_back();
    Node node(n.name.empty() ? n.op_type + "_" + std::to_string(index) : n.name, n.op_type, std::move(inputs),
              std::move(outputs));
    for (const AttributeData& a : n.attributes) {
      switch (a.type) {
        case kAttrFloat: node.SetAttribute(a.name, static_cast<double>(a.f)); break;
        case kAttrInt: node.SetAttribute(a.name, a.i); break;
        case kAttrString: node.SetAttribute(a.name, a.s); break;
        case kAttrFloats: node.SetAttribute(a.name, std::vector<double>(a.floats.begin(), a.floats.end())); break;
        case kAttrInts: node.SetAttribute(a.name, a.ints); break;
        default:
          return Status::Unsupported("ONNX attribute " + a.name + " of node " + node.name() + " has type " +
                                     std::to_string(a.type));
      }
    }
    if (n.op_type == "Softmax" && opset < 13 && !node.GetAttribute<int64_t>("axis")) {
      node.SetAttribute("axis", int64_t{1});
    }
    CUTRITON_RETURN_IF_ERROR(CheckSupported(n, node));
    if (n.op_type == "Identity" && node.inputs().size() == 1 && node.outputs().size() == 1 &&
        model->constants().count(node.inputs()[0]) != 0) {
      // Identity of a constant (exporters route shared initializers through
      // one): the output is the same constant.
      CUTRITON_RETURN_IF_ERROR(model->AddConstant(node.outputs()[0], model->constants().at(node.inputs()[0])));
      continue;
    }
    if (n.op_type == "Conv" && node.inputs().size() == 3) {
      CUTRITON_RETURN_IF_ERROR(AddConvBias(std::move(node), model));
      continue;
    }
    CUTRITON_RETURN_IF_ERROR(graph.AddNode(std::move(node)));
  }
  for (const ValueInfoData& v : g.outputs) CUTRITON_RETURN_IF_ERROR(graph.AddOutput(v.name));
  return Status::OK();
}

}  // namespace

Status ImportOnnxModel(const void* data, std::size_t size, const OnnxDimValues& dim_values, Model* model) {
  if (model == nullptr || (data == nullptr && size != 0)) return Status::InvalidArgument("ONNX import arguments");
  if (!model->graph().nodes().empty() || !model->graph().inputs().empty() || !model->constants().empty()) {
    return Status::InvalidArgument("ONNX import needs an empty model");
  }
  Reader r(Span{static_cast<const uint8_t*>(data), size});
  Span graph;
  bool has_graph = false;
  int64_t opset = 0;
  while (!r.done()) {
    uint32_t field = 0, wire = 0;
    if (!r.Tag(&field, &wire)) return Malformed("ModelProto");
    Span s;
    if (field == 7) {
      if (wire != kBytes || !r.Bytes(&graph)) return Malformed("ModelProto.graph");
      has_graph = true;
    } else if (field == 8) {  // OperatorSetIdProto: domain = 1, version = 2
      if (wire != kBytes || !r.Bytes(&s)) return Malformed("ModelProto.opset_import");
      Reader o(s);
      std::string domain;
      int64_t version = 0;
      while (!o.done()) {
        uint32_t of = 0, ow = 0;
        Span ds;
        uint64_t v = 0;
        if (!o.Tag(&of, &ow)) return Malformed("OperatorSetIdProto");
        if (of == 1 && ow == kBytes && o.Bytes(&ds)) {
          domain = ds.str();
        } else if (of == 2 && ow == kVarint && o.Varint(&v)) {
          version = static_cast<int64_t>(v);
        } else if ((of == 1 || of == 2) || !o.Skip(ow)) {
          return Malformed("OperatorSetIdProto");
        }
      }
      if (DefaultDomain(domain)) opset = version;
    } else if (!r.Skip(wire)) {
      return Malformed("ModelProto field " + std::to_string(field));
    }
  }
  if (!has_graph) return Malformed("no graph");
  GraphData g;
  CUTRITON_RETURN_IF_ERROR(ParseGraph(graph, &g));
  return BuildModel(g, opset, dim_values, model);
}

Status ImportOnnxFile(const std::string& path, const OnnxDimValues& dim_values, Model* model) {
  std::ifstream in(path, std::ios::binary);
  if (!in) return Status::NotFound("cannot open ONNX model " + path);
  const std::string bytes((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
  return ImportOnnxModel(bytes.data(), bytes.size(), dim_values, model);
}

}  // namespace cutriton
