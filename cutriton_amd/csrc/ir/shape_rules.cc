// Output-shape rules of every operator the engine runs, and their schema
// registration (arity + rule per op type).
//
// The rules are the ONNX operators' own shape semantics, restricted as the
// reference restricts them (src/ir/pass.cpp:45-238): NCHW / OIHW convolution
// and pooling with 2-D windows, rank-2 Gemm with optional transA / transB and
// an [N] or [M, N] bias, LayerNormalization over the last axis only,
// elementwise binaries over identical descriptions. Additions of this
// backend: FusedConvBatchNormAddRelu (a residual input shaped like the
// output), Softmax (last axis only), Attention (4-D).
#include <array>
#include <utility>

#include "cutriton/ir/op_schema.h"
#include "cutriton/ir/pass.h"

namespace cutriton {
namespace {

// Access to one node's operand descriptions while its rule runs.
class RuleContext {
 public:
  RuleContext(Graph* graph, const Node& node) : graph_(graph), node_(node) {}

  const Node& node() const { return node_; }
  std::size_t input_count() const { return node_.inputs().size(); }
  // The description of input `i`, or null when the input or its value is missing.
  const TensorDesc* In(std::size_t i) const {
    if (i >= node_.inputs().size()) return nullptr;
    const ValueDesc* value = graph_->FindValue(node_.inputs()[i]);
    return value == nullptr ? nullptr : &value->tensor;
  }
  Status Fail(const std::string& why) const {
    return Status::ShapeError(node_.op_type() + " " + node_.name() + ": " + why);
  }
  // Sets every output to `desc` after validating it.
  Status Emit(const TensorDesc& desc) const {
    CUTRITON_RETURN_IF_ERROR(desc.Validate());
    for (const auto& name : node_.outputs()) CUTRITON_RETURN_IF_ERROR(graph_->SetValueDesc(name, desc));
    return Status::OK();
  }

 private:
  Graph* graph_;
  const Node& node_;
};

// One spatial axis of a sliding window.
struct Window {
  int64_t extent{1};  // kernel size along the axis
  int64_t stride{1};
  int64_t pad_begin{0};
  int64_t pad_end{0};
  int64_t dilation{1};
  // Output length: the number of window positions that fit the padded input.
  int64_t Out(int64_t in) const { return (in + pad_begin + pad_end - dilation * (extent - 1) - 1) / stride + 1; }
};

// The height and width windows of a node with ONNX attributes strides[2],
// pads[4] (begin h, begin w, end h, end w) and dilations[2]; extents come from
// the weight (convolution) or kernel_shape (pooling, whose strides default to
// the kernel).
Status ReadWindows(const RuleContext& rule, std::array<int64_t, 2> extent, bool strides_default_to_extent,
                   std::array<Window, 2>* out) {
  const Node& node = rule.node();
  const std::vector<int64_t> unit{1, 1};
  const auto strides = GetIntListAttribute(node, "strides", strides_default_to_extent
                                                                ? std::vector<int64_t>{extent[0], extent[1]}
                                                                : unit);
  const auto pads = GetIntListAttribute(node, "pads", {0, 0, 0, 0});
  const auto dilations = GetIntListAttribute(node, "dilations", unit);
  if (strides.size() != 2 || pads.size() != 4 || dilations.size() != 2) {
    return rule.Fail("attributes must be strides[2], pads[4] and dilations[2]");
  }
  for (int axis = 0; axis < 2; ++axis) {
    (*out)[axis] = Window{extent[axis], strides[axis], pads[axis], pads[axis + 2], dilations[axis]};
  }
  return Status::OK();
}

TensorDesc Like(const TensorDesc& base, std::vector<int64_t> shape, std::string layout) {
  return TensorDesc(std::move(shape), base.dtype, base.device_type, base.device_id, std::move(layout));
}

Status SameAsFirstInput(const RuleContext& rule) {
  const TensorDesc* x = rule.In(0);
  if (x == nullptr || x->dtype == DataType::kUnknown) return rule.Fail("the first input has no description");
  return rule.Emit(*x);
}

Status IdenticalOperands(const RuleContext& rule) {
  const TensorDesc* a = rule.In(0);
  const TensorDesc* b = rule.In(1);
  if (rule.input_count() != 2 || a == nullptr || b == nullptr) return rule.Fail("expects two described inputs");
  if (a->shape != b->shape || a->dtype != b->dtype || a->layout != b->layout) {
    return rule.Fail("inputs must have identical shape, dtype and layout");
  }
  return rule.Emit(*a);
}

// NCHW input, OIHW weight -> [N, O, OH, OW] in the input's layout.
Status Convolution(const RuleContext& rule) {
  const TensorDesc* x = rule.In(0);
  const TensorDesc* w = rule.In(1);
  if (x == nullptr || w == nullptr || x->shape.size() != 4 || w->shape.size() != 4) {
    return rule.Fail("expects an NCHW input and an OIHW weight");
  }
  std::array<Window, 2> windows;
  CUTRITON_RETURN_IF_ERROR(ReadWindows(rule, {w->shape[2], w->shape[3]}, false, &windows));
  return rule.Emit(Like(*x, {x->shape[0], w->shape[0], windows[0].Out(x->shape[2]), windows[1].Out(x->shape[3])},
                        x->layout));
}

// The convolution whose epilogue adds input 6 before the ReLU.
Status ConvolutionWithResidual(const RuleContext& rule) {
  CUTRITON_RETURN_IF_ERROR(Convolution(rule));
  const TensorDesc* x = rule.In(0);
  const TensorDesc* w = rule.In(1);
  const TensorDesc* residual = rule.In(6);
  std::array<Window, 2> windows;
  CUTRITON_RETURN_IF_ERROR(ReadWindows(rule, {w->shape[2], w->shape[3]}, false, &windows));
  const std::vector<int64_t> out{x->shape[0], w->shape[0], windows[0].Out(x->shape[2]), windows[1].Out(x->shape[3])};
  if (residual == nullptr || residual->shape != out || residual->dtype != x->dtype) {
    return rule.Fail("the residual input must match the convolution output");
  }
  return Status::OK();
}

Status Pooling(const RuleContext& rule) {
  const TensorDesc* x = rule.In(0);
  if (x == nullptr || x->shape.size() != 4) return rule.Fail("expects an NCHW input");
  const auto kernel = GetIntListAttribute(rule.node(), "kernel_shape", {1, 1});
  if (kernel.size() != 2) return rule.Fail("kernel_shape must have two entries");
  std::array<Window, 2> windows;
  CUTRITON_RETURN_IF_ERROR(ReadWindows(rule, {kernel[0], kernel[1]}, true, &windows));
  return rule.Emit(Like(*x, {x->shape[0], x->shape[1], windows[0].Out(x->shape[2]), windows[1].Out(x->shape[3])},
                        x->layout));
}

Status GlobalPooling(const RuleContext& rule) {
  const TensorDesc* x = rule.In(0);
  if (x == nullptr || x->shape.size() != 4) return rule.Fail("expects an NCHW input");
  return rule.Emit(Like(*x, {x->shape[0], x->shape[1], 1, 1}, x->layout));
}

// [d0..dk-1 | dk..dr-1] -> [prod(d0..dk-1), prod(dk..dr-1)], no layout.
Status Flattening(const RuleContext& rule) {
  const TensorDesc* x = rule.In(0);
  if (x == nullptr || x->shape.empty()) return rule.Fail("needs a known input shape");
  const auto rank = static_cast<int64_t>(x->shape.size());
  int64_t axis = GetIntAttribute(rule.node(), "axis", 1);
  if (axis < 0) axis += rank;
  if (axis < 0 || axis > rank) return rule.Fail("axis is outside the input rank");
  int64_t outer = 1;
  int64_t inner = 1;
  for (int64_t i = 0; i < rank; ++i) {
    const int64_t d = x->shape[static_cast<std::size_t>(i)];
    if (d <= 0) return rule.Emit(Like(*x, {0, 0}, ""));  // unresolved: Validate reports it
    (i < axis ? outer : inner) *= d;
  }
  return rule.Emit(Like(*x, {outer, inner}, ""));
}

// A[M,K] (or [K,M] with transA) times B[K,N] (or [N,K] with transB), plus an
// optional bias of [N] or [M,N].
Status MatrixProduct(const RuleContext& rule) {
  const TensorDesc* a = rule.In(0);
  const TensorDesc* b = rule.In(1);
  if (a == nullptr || b == nullptr || a->shape.size() != 2 || b->shape.size() != 2) {
    return rule.Fail("expects two rank-2 inputs");
  }
  if (a->dtype != b->dtype) return rule.Fail("inputs must share a dtype");
  const bool ta = GetIntAttribute(rule.node(), "transA", 0) != 0;
  const bool tb = GetIntAttribute(rule.node(), "transB", 0) != 0;
  const int64_t m = a->shape[ta ? 1 : 0];
  const int64_t n = b->shape[tb ? 0 : 1];
  if (a->shape[ta ? 0 : 1] != b->shape[tb ? 1 : 0]) return rule.Fail("inner dimensions do not match");
  if (const TensorDesc* bias = rule.In(2); rule.input_count() == 3) {
    const bool shaped = bias != nullptr && (bias->shape == std::vector<int64_t>{n} ||
                                            bias->shape == std::vector<int64_t>{m, n});
    if (!shaped || bias->dtype != a->dtype) return rule.Fail("bias must be [N] or [M,N] of the inputs' dtype");
  }
  return rule.Emit(Like(*a, {m, n}, ""));
}

// Normalisation over the last axis of `x` with scale (and bias) of that length.
Status CheckLastAxisAffine(const RuleContext& rule, const TensorDesc& x, const TensorDesc* scale,
                           const TensorDesc* bias, bool has_bias) {
  const std::vector<int64_t> row{x.shape.back()};
  if (scale == nullptr || scale->shape != row || scale->dtype != x.dtype) {
    return rule.Fail("scale must match the last dimension");
  }
  if (has_bias && (bias == nullptr || bias->shape != row || bias->dtype != x.dtype)) {
    return rule.Fail("bias must match the scale");
  }
  const int64_t axis = GetIntAttribute(rule.node(), "axis", -1);
  if (axis != -1 && axis != static_cast<int64_t>(x.shape.size()) - 1) {
    return Status::Unsupported(rule.node().op_type() + " is supported over the last axis only");
  }
  return Status::OK();
}

Status LayerNorm(const RuleContext& rule) {
  const TensorDesc* x = rule.In(0);
  if (x == nullptr || x->shape.empty()) return rule.Fail("needs a described input");
  CUTRITON_RETURN_IF_ERROR(CheckLastAxisAffine(rule, *x, rule.In(1), rule.In(2), rule.input_count() == 3));
  return rule.Emit(*x);
}

// LayerNormalization(input + residual, scale, bias).
Status SkipLayerNorm(const RuleContext& rule) {
  const TensorDesc* x = rule.In(0);
  const TensorDesc* residual = rule.In(1);
  if (x == nullptr || residual == nullptr || x->shape.empty()) return rule.Fail("needs described inputs");
  if (residual->shape != x->shape || residual->dtype != x->dtype || residual->layout != x->layout) {
    return rule.Fail("input and residual must have identical descriptions");
  }
  CUTRITON_RETURN_IF_ERROR(CheckLastAxisAffine(rule, *x, rule.In(2), rule.In(3), true));
  return rule.Emit(*x);
}

// Softmax over the last axis: the reference's kernel ignores `axis`
// (python/cutriton/triton_kernels/transformer.py:180-190) and would give a
// last-axis result for any other axis; here another axis is refused.
Status LastAxisSoftmax(const RuleContext& rule) {
  const TensorDesc* x = rule.In(0);
  if (x == nullptr || x->shape.empty()) return rule.Fail("expects one input of rank >= 1");
  const int64_t axis = GetIntAttribute(rule.node(), "axis", -1);
  if (axis != -1 && axis != static_cast<int64_t>(x->shape.size()) - 1) {
    return Status::Unsupported("only last-axis Softmax is supported");
  }
  return rule.Emit(*x);
}

// Attention (the ONNX operator's 4-D form): Q [B, H, Sq, D], K [B, H, Sk, D],
// V [B, H, Sk, D] -> [B, H, Sq, D], attributes scale and is_causal. The mask
// and past key/value inputs, the 3-D form (q_num_heads / kv_num_heads),
// softcap, the extra outputs and a value head dimension other than the
// query's are refused.
Status ScaledDotProductAttention(const RuleContext& rule) {
  const Node& node = rule.node();
  for (const char* key : {"q_num_heads", "kv_num_heads"}) {
    if (node.attributes().count(key) != 0) return Status::Unsupported("Attention: 3-D inputs (" + std::string(key) + ")");
  }
  if (node.GetAttribute<double>("softcap").value_or(0.0) != 0.0) return Status::Unsupported("Attention: softcap");
  if (GetIntAttribute(node, "qk_matmul_output_mode", 0) != 0) {
    return Status::Unsupported("Attention: qk_matmul_output_mode");
  }
  const TensorDesc* q = rule.In(0);
  const TensorDesc* k = rule.In(1);
  const TensorDesc* v = rule.In(2);
  if (q == nullptr || k == nullptr || v == nullptr || q->shape.size() != 4 || k->shape.size() != 4 ||
      v->shape.size() != 4) {
    return rule.Fail("expects Q, K and V of rank 4 [batch, heads, sequence, head dimension]");
  }
  const bool same_type = q->dtype == k->dtype && q->dtype == v->dtype;
  const bool same_heads = q->shape[0] == k->shape[0] && q->shape[0] == v->shape[0] && q->shape[1] == k->shape[1] &&
                          q->shape[1] == v->shape[1];
  if (!same_type || !same_heads || q->shape[3] != k->shape[3] || k->shape[2] != v->shape[2]) {
    return rule.Fail("Q, K and V disagree in type, batch, heads, keys or head dimension");
  }
  if (v->shape[3] != q->shape[3]) return Status::Unsupported("Attention: a value head dimension other than the query's");
  return rule.Emit(Like(*q, q->shape, ""));
}

using Rule = Status (*)(const RuleContext&);

struct SchemaRow {
  const char* op;
  std::size_t min_inputs;
  std::size_t max_inputs;
  Rule rule;
};

constexpr SchemaRow kSchemas[] = {
    {"Conv", 2, 2, Convolution},
    {"FusedConvBatchNorm", 6, 6, Convolution},
    {"FusedConvBatchNormRelu", 6, 6, Convolution},
    {"FusedConvBatchNormAddRelu", 7, 7, ConvolutionWithResidual},
    {"BatchNormalization", 5, 5, SameAsFirstInput},
    {"Relu", 1, 1, SameAsFirstInput},
    {"Gelu", 1, 1, SameAsFirstInput},
    {"Softmax", 1, 1, LastAxisSoftmax},
    {"Attention", 3, 3, ScaledDotProductAttention},
    {"Add", 2, 2, IdenticalOperands},
    {"AddRelu", 2, 2, IdenticalOperands},
    {"LayerNormalization", 2, 3, LayerNorm},
    {"SkipLayerNormalization", 4, 4, SkipLayerNorm},
    {"Flatten", 1, 1, Flattening},
    {"Gemm", 2, 3, MatrixProduct},
    {"GemmGelu", 2, 3, MatrixProduct},
    {"MatMul", 2, 2, MatrixProduct},
    {"MaxPool", 1, 1, Pooling},
    {"AveragePool", 1, 1, Pooling},
    {"GlobalAveragePool", 1, 1, GlobalPooling},
};

}  // namespace

Status RegisterBuiltinOpSchemas() {
  auto& registry = OpSchemaRegistry::Global();
  auto add = [&](OpSchema schema) {
    const Status status = registry.Register(std::move(schema));
    return status.code() == ErrorCode::kAlreadyExists ? Status::OK() : status;
  };
  for (const SchemaRow& row : kSchemas) {
    const Rule rule = row.rule;
    CUTRITON_RETURN_IF_ERROR(add(OpSchema{row.op, row.min_inputs, row.max_inputs, 1,
                                          [rule](Graph* graph, const Node& node) {
                                            return rule(RuleContext(graph, node));
                                          }}));
  }
  // Constant nodes carry their value as a model constant: nothing to infer.
  return add(OpSchema{"Constant", 0, 0, 1, [](Graph*, const Node&) { return Status::OK(); }});
}

}  // namespace cutriton
