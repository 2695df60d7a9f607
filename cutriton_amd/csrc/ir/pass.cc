// Shape inference, graph passes and the default pipeline.
// Shape rules follow reference src/ir/pass.cpp:45-238; fusion rewrites follow
// src/ir/pass.cpp:319-501; the pipeline order follows src/ir/pass.cpp:666-684.
// FusedConvBatchNormAddRelu (schema, pass) is specific to this backend: it
// moves the residual join of a bottleneck block into the conv epilogue.
#include "cutriton/ir/pass.h"

#include <algorithm>
#include <cmath>
#include <unordered_set>

#include "cutriton/ir/op_schema.h"

namespace cutriton {
namespace {

bool IsGraphOutput(const Graph& graph, const std::string& name) {
  return std::find(graph.outputs().begin(), graph.outputs().end(), name) != graph.outputs().end();
}

int64_t DimProduct(const std::vector<int64_t>& dims, std::size_t begin, std::size_t end) {
  int64_t product = 1;
  for (std::size_t i = begin; i < end; ++i) {
    if (dims[i] <= 0) return 0;
    product *= dims[i];
  }
  return product;
}

Status InferSameAsFirstInput(Graph* graph, const Node& node) {
  const ValueDesc* first = node.inputs().empty() ? nullptr : graph->FindValue(node.inputs()[0]);
  if (first == nullptr || first->tensor.dtype == DataType::kUnknown) {
    return Status::ShapeError("cannot infer the output of " + node.name());
  }
  for (const auto& output : node.outputs()) {
    CUTRITON_RETURN_IF_ERROR(graph->SetValueDesc(output, first->tensor));
  }
  return Status::OK();
}

Status InferElementwiseBinary(Graph* graph, const Node& node) {
  if (node.inputs().size() != 2 || node.outputs().size() != 1) {
    return Status::ShapeError(node.op_type() + " expects two inputs and one output");
  }
  const ValueDesc* a = graph->FindValue(node.inputs()[0]);
  const ValueDesc* b = graph->FindValue(node.inputs()[1]);
  if (a == nullptr || b == nullptr) {
    return Status::ShapeError(node.op_type() + " references an unknown tensor");
  }
  if (a->tensor.shape != b->tensor.shape || a->tensor.dtype != b->tensor.dtype ||
      a->tensor.layout != b->tensor.layout) {
    return Status::ShapeError(node.op_type() + " inputs must have identical descriptions");
  }
  return graph->SetValueDesc(node.outputs()[0], a->tensor);
}

// out = (in + pad_begin + pad_end - dilation*(kernel-1) - 1) / stride + 1
Status InferConvLike(Graph* graph, const Node& node) {
  if (node.inputs().size() < 2 || node.outputs().empty()) {
    return Status::ShapeError("convolution needs an input, a weight and an output");
  }
  const ValueDesc* x = graph->FindValue(node.inputs()[0]);
  const ValueDesc* w = graph->FindValue(node.inputs()[1]);
  if (x == nullptr || w == nullptr) return Status::ShapeError("convolution references an unknown tensor");
  const auto& xs = x->tensor.shape;
  const auto& ws = w->tensor.shape;
  if (xs.size() != 4 || ws.size() != 4) {
    return Status::ShapeError("convolution expects an NCHW input and an OIHW weight");
  }
  const auto strides = GetIntListAttribute(node, "strides", {1, 1});
  const auto pads = GetIntListAttribute(node, "pads", {0, 0, 0, 0});
  const auto dilations = GetIntListAttribute(node, "dilations", {1, 1});
  if (strides.size() != 2 || pads.size() != 4 || dilations.size() != 2) {
    return Status::ShapeError("convolution attributes must be strides[2], pads[4], dilations[2]");
  }
  const int64_t out_h = (xs[2] + pads[0] + pads[2] - dilations[0] * (ws[2] - 1) - 1) / strides[0] + 1;
  const int64_t out_w = (xs[3] + pads[1] + pads[3] - dilations[1] * (ws[3] - 1) - 1) / strides[1] + 1;
  TensorDesc out({xs[0], ws[0], out_h, out_w}, x->tensor.dtype, x->tensor.device_type,
                 x->tensor.device_id, x->tensor.layout);
  CUTRITON_RETURN_IF_ERROR(out.Validate());
  return graph->SetValueDesc(node.outputs()[0], std::move(out));
}

// Convolution whose epilogue adds input 6 (the residual) before the ReLU.
Status InferConvResidual(Graph* graph, const Node& node) {
  CUTRITON_RETURN_IF_ERROR(InferConvLike(graph, node));
  const ValueDesc* residual = graph->FindValue(node.inputs()[6]);
  const ValueDesc* out = graph->FindValue(node.outputs()[0]);
  if (residual == nullptr || out == nullptr || residual->tensor.shape != out->tensor.shape ||
      residual->tensor.dtype != out->tensor.dtype) {
    return Status::ShapeError("residual input must match the convolution output: " + node.name());
  }
  return Status::OK();
}

Status InferPool(Graph* graph, const Node& node) {
  const ValueDesc* x = graph->FindValue(node.inputs().front());
  if (x == nullptr || x->tensor.shape.size() != 4) return Status::ShapeError("pooling expects an NCHW input");
  const auto kernel = GetIntListAttribute(node, "kernel_shape", {1, 1});
  const auto strides = GetIntListAttribute(node, "strides", kernel);
  const auto pads = GetIntListAttribute(node, "pads", {0, 0, 0, 0});
  const auto dilations = GetIntListAttribute(node, "dilations", {1, 1});
  if (kernel.size() != 2 || strides.size() != 2 || pads.size() != 4 || dilations.size() != 2) {
    return Status::ShapeError(
        "pooling attributes must be kernel_shape[2], strides[2], pads[4], dilations[2]");
  }
  const auto& s = x->tensor.shape;
  const int64_t span_h = dilations[0] * (kernel[0] - 1) + 1;
  const int64_t span_w = dilations[1] * (kernel[1] - 1) + 1;
  const int64_t out_h = (s[2] + pads[0] + pads[2] - span_h) / strides[0] + 1;
  const int64_t out_w = (s[3] + pads[1] + pads[3] - span_w) / strides[1] + 1;
  TensorDesc out({s[0], s[1], out_h, out_w}, x->tensor.dtype, x->tensor.device_type,
                 x->tensor.device_id, x->tensor.layout);
  CUTRITON_RETURN_IF_ERROR(out.Validate());
  return graph->SetValueDesc(node.outputs()[0], std::move(out));
}

Status InferFlatten(Graph* graph, const Node& node) {
  const ValueDesc* x = graph->FindValue(node.inputs().front());
  if (x == nullptr || x->tensor.shape.empty()) return Status::ShapeError("Flatten needs a known input shape");
  const auto& s = x->tensor.shape;
  int64_t axis = GetIntAttribute(node, "axis", 1);
  if (axis < 0) axis += static_cast<int64_t>(s.size());
  if (axis < 0 || axis > static_cast<int64_t>(s.size())) {
    return Status::ShapeError("Flatten axis is outside the input rank");
  }
  const auto split = static_cast<std::size_t>(axis);
  TensorDesc out({DimProduct(s, 0, split), DimProduct(s, split, s.size())}, x->tensor.dtype,
                 x->tensor.device_type, x->tensor.device_id, "");
  CUTRITON_RETURN_IF_ERROR(out.Validate());
  return graph->SetValueDesc(node.outputs()[0], std::move(out));
}

Status InferGemm(Graph* graph, const Node& node) {
  if (node.inputs().size() < 2) return Status::ShapeError("Gemm expects two inputs");
  const ValueDesc* a = graph->FindValue(node.inputs()[0]);
  const ValueDesc* b = graph->FindValue(node.inputs()[1]);
  if (a == nullptr || b == nullptr || a->tensor.shape.size() != 2 || b->tensor.shape.size() != 2) {
    return Status::ShapeError("Gemm expects rank-2 inputs");
  }
  if (a->tensor.dtype != b->tensor.dtype) return Status::ShapeError("Gemm inputs must share a dtype");
  const bool trans_a = GetIntAttribute(node, "transA", 0) != 0;
  const bool trans_b = GetIntAttribute(node, "transB", 0) != 0;
  const auto& as = a->tensor.shape;
  const auto& bs = b->tensor.shape;
  const int64_t m = trans_a ? as[1] : as[0];
  const int64_t ka = trans_a ? as[0] : as[1];
  const int64_t kb = trans_b ? bs[1] : bs[0];
  const int64_t n = trans_b ? bs[0] : bs[1];
  if (ka != kb) return Status::ShapeError("Gemm inner dimensions do not match");
  if (node.inputs().size() == 3) {
    const ValueDesc* bias = graph->FindValue(node.inputs()[2]);
    if (bias == nullptr || bias->tensor.dtype != a->tensor.dtype ||
        (bias->tensor.shape != std::vector<int64_t>{n} &&
         bias->tensor.shape != std::vector<int64_t>{m, n})) {
      return Status::ShapeError("Gemm bias must be [N] or [M,N]");
    }
  }
  TensorDesc out({m, n}, a->tensor.dtype, a->tensor.device_type, a->tensor.device_id, "");
  CUTRITON_RETURN_IF_ERROR(out.Validate());
  return graph->SetValueDesc(node.outputs()[0], std::move(out));
}

Status InferLayerNormalization(Graph* graph, const Node& node) {
  if (node.inputs().size() < 2 || node.inputs().size() > 3) {
    return Status::ShapeError("LayerNormalization expects input, scale and an optional bias");
  }
  const ValueDesc* x = graph->FindValue(node.inputs()[0]);
  const ValueDesc* scale = graph->FindValue(node.inputs()[1]);
  if (x == nullptr || scale == nullptr || x->tensor.shape.empty() ||
      scale->tensor.shape != std::vector<int64_t>{x->tensor.shape.back()} ||
      x->tensor.dtype != scale->tensor.dtype) {
    return Status::ShapeError("LayerNormalization scale must match the last dimension");
  }
  if (node.inputs().size() == 3) {
    const ValueDesc* bias = graph->FindValue(node.inputs()[2]);
    if (bias == nullptr || bias->tensor.shape != scale->tensor.shape ||
        bias->tensor.dtype != x->tensor.dtype) {
      return Status::ShapeError("LayerNormalization bias must match scale");
    }
  }
  const int64_t axis = GetIntAttribute(node, "axis", -1);
  if (axis != -1 && axis != static_cast<int64_t>(x->tensor.shape.size()) - 1) {
    return Status::Unsupported("only last-axis LayerNormalization is supported");
  }
  return graph->SetValueDesc(node.outputs()[0], x->tensor);
}

// Attention (the ONNX operator's 4-D form): Q [B, H, Sq, D], K [B, H, Sk, D],
// V [B, H, Sk, D] -> [B, H, Sq, D], attributes `scale` and `is_causal`. The
// attention-mask and past key/value inputs, the 3-D form (q_num_heads /
// kv_num_heads), softcap, the extra outputs and a value head dimension that
// differs from the query's are refused. The reference has no attention.
Status InferAttention(Graph* graph, const Node& node) {
  if (node.inputs().size() != 3 || node.outputs().size() != 1) {
    return Status::Unsupported("Attention takes Q, K and V and gives one output (no mask, past or present)");
  }
  for (const char* key : {"q_num_heads", "kv_num_heads"}) {
    if (node.attributes().count(key) != 0) return Status::Unsupported("Attention: 3-D inputs (" + std::string(key) + ")");
  }
  if (const auto softcap = node.GetAttribute<double>("softcap"); softcap && *softcap != 0.0) {
    return Status::Unsupported("Attention: softcap");
  }
  if (GetIntAttribute(node, "qk_matmul_output_mode", 0) != 0) {
    return Status::Unsupported("Attention: qk_matmul_output_mode");
  }
  const ValueDesc* q = graph->FindValue(node.inputs()[0]);
  const ValueDesc* k = graph->FindValue(node.inputs()[1]);
  const ValueDesc* v = graph->FindValue(node.inputs()[2]);
  if (q == nullptr || k == nullptr || v == nullptr || q->tensor.shape.size() != 4 || k->tensor.shape.size() != 4 ||
      v->tensor.shape.size() != 4) {
    return Status::ShapeError("Attention expects Q, K and V of rank 4 [batch, heads, sequence, head dimension]");
  }
  const auto& qs = q->tensor.shape;
  const auto& ks = k->tensor.shape;
  const auto& vs = v->tensor.shape;
  if (q->tensor.dtype != k->tensor.dtype || q->tensor.dtype != v->tensor.dtype || qs[0] != ks[0] ||
      qs[0] != vs[0] || qs[1] != ks[1] || qs[1] != vs[1] || qs[3] != ks[3] || ks[2] != vs[2]) {
    return Status::ShapeError("Attention: Q, K and V disagree in type, batch, heads, keys or head dimension");
  }
  if (vs[3] != qs[3]) return Status::Unsupported("Attention: a value head dimension other than the query's");
  TensorDesc out = q->tensor;
  out.layout = "";
  return graph->SetValueDesc(node.outputs()[0], out);
}

// Softmax over the last axis only: the reference's kernel ignores `axis`
// (python/cutriton/triton_kernels/transformer.py:180-190) and would give a
// last-axis result for any other axis; here another axis is refused.
Status InferSoftmax(Graph* graph, const Node& node) {
  const ValueDesc* x = node.inputs().size() == 1 ? graph->FindValue(node.inputs()[0]) : nullptr;
  if (x == nullptr || x->tensor.shape.empty() || node.outputs().size() != 1) {
    return Status::ShapeError("Softmax expects one input of rank >= 1 and one output");
  }
  const int64_t axis = GetIntAttribute(node, "axis", -1);
  if (axis != -1 && axis != static_cast<int64_t>(x->tensor.shape.size()) - 1) {
    return Status::Unsupported("only last-axis Softmax is supported");
  }
  return graph->SetValueDesc(node.outputs()[0], x->tensor);
}

Status InferSkipLayerNormalization(Graph* graph, const Node& node) {
  if (node.inputs().size() != 4) {
    return Status::ShapeError("SkipLayerNormalization expects input, residual, scale and bias");
  }
  // Add(input, residual) followed by LayerNormalization(sum, scale, bias).
  const Node add(node.name() + "::shape_add", "Add", {node.inputs()[0], node.inputs()[1]},
                 {node.outputs()[0]});
  CUTRITON_RETURN_IF_ERROR(InferElementwiseBinary(graph, add));
  Node norm(node.name() + "::shape_norm", "LayerNormalization",
            {node.outputs()[0], node.inputs()[2], node.inputs()[3]}, node.outputs());
  norm.SetAttribute("axis", GetIntAttribute(node, "axis", -1));
  return InferLayerNormalization(graph, norm);
}

Status InferGlobalAveragePool(Graph* graph, const Node& node) {
  const ValueDesc* x = graph->FindValue(node.inputs().front());
  if (x == nullptr || x->tensor.shape.size() != 4) {
    return Status::ShapeError("GlobalAveragePool expects an NCHW input");
  }
  TensorDesc out({x->tensor.shape[0], x->tensor.shape[1], 1, 1}, x->tensor.dtype,
                 x->tensor.device_type, x->tensor.device_id, x->tensor.layout);
  return graph->SetValueDesc(node.outputs()[0], std::move(out));
}

class TopologicalSortPass final : public GraphPass {
 public:
  const char* name() const override { return "topological_sort"; }
  Status Run(Graph* graph) const override { return graph->TopologicalSort(); }
};

class ShapeInferencePass final : public GraphPass {
 public:
  const char* name() const override { return "shape_inference"; }
  Status Run(Graph* graph) const override {
    CUTRITON_RETURN_IF_ERROR(RegisterBuiltinOpSchemas());
    for (const auto& node : graph->nodes()) {
      const auto schema = OpSchemaRegistry::Global().Find(node.op_type());
      if (schema == nullptr) return Status::Unsupported("no shape inference for op " + node.op_type());
      if (node.inputs().size() < schema->min_inputs || node.inputs().size() > schema->max_inputs ||
          node.outputs().size() != schema->outputs) {
        return Status::ShapeError("input/output count violates the OpSchema: " + node.name());
      }
      CUTRITON_RETURN_IF_ERROR(schema->infer(graph, node));
    }
    return Status::OK();
  }
};

// Constants carry no folding opportunity in the supported graphs; the pass
// keeps its slot in the pipeline.
class ConstantFoldingPass final : public GraphPass {
 public:
  const char* name() const override { return "constant_folding"; }
  Status Run(Graph*) const override { return Status::OK(); }
};

class DeadNodeEliminationPass final : public GraphPass {
 public:
  const char* name() const override { return "dead_node_elimination"; }
  Status Run(Graph* graph) const override {
    std::unordered_set<std::string> live(graph->outputs().begin(), graph->outputs().end());
    std::unordered_set<int> keep;
    const auto& nodes = graph->nodes();
    for (auto it = nodes.rbegin(); it != nodes.rend(); ++it) {
      const bool needed = std::any_of(it->outputs().begin(), it->outputs().end(),
                                      [&](const std::string& o) { return live.count(o) != 0; });
      if (!needed) continue;
      keep.insert(it->id());
      live.insert(it->inputs().begin(), it->inputs().end());
    }
    std::vector<int> dead;
    for (const auto& node : nodes) {
      if (keep.count(node.id()) == 0) dead.push_back(node.id());
    }
    return graph->RemoveNodes(dead);
  }
};

// Returns the single consumer of `value`, or -1.
int SoleConsumer(const std::unordered_map<std::string, std::vector<int>>& consumers,
                 const std::string& value, std::size_t node_count) {
  const auto it = consumers.find(value);
  if (it == consumers.end() || it->second.size() != 1) return -1;
  const int id = it->second.front();
  return id >= 0 && static_cast<std::size_t>(id) < node_count ? id : -1;
}

// Each fusion pass rewrites one match per sweep and re-scans, so consumer
// maps are always current.
template <typename TryFuse>
Status FuseToFixpoint(Graph* graph, TryFuse try_fuse) {
  for (;;) {
    const auto consumers = graph->BuildConsumerMap();
    bool rewrote = false;
    for (std::size_t i = 0; i < graph->nodes().size() && !rewrote; ++i) {
      std::vector<int> removed;
      if (try_fuse(graph, i, consumers, &removed)) {
        CUTRITON_RETURN_IF_ERROR(graph->RemoveNodes(removed));
        rewrote = true;
      }
    }
    if (!rewrote) return Status::OK();
  }
}

class ConvBatchNormReluFusionPass final : public GraphPass {
 public:
  const char* name() const override { return "conv_batchnorm_relu_fusion"; }
  Status Run(Graph* graph) const override {
    return FuseToFixpoint(graph, [](Graph* g, std::size_t i, const auto& consumers,
                                    std::vector<int>* removed) {
      Node& conv = g->mutable_nodes()[i];
      if (conv.op_type() != "Conv" || conv.outputs().size() != 1) return false;
      const int bn_id = SoleConsumer(consumers, conv.outputs()[0], g->nodes().size());
      if (bn_id < 0) return false;
      const Node bn = g->nodes()[static_cast<std::size_t>(bn_id)];
      if (bn.op_type() != "BatchNormalization" || bn.outputs().size() != 1) return false;
      const int relu_id = SoleConsumer(consumers, bn.outputs()[0], g->nodes().size());
      const bool with_relu = relu_id >= 0 &&
                             g->nodes()[static_cast<std::size_t>(relu_id)].op_type() == "Relu" &&
                             !g->nodes()[static_cast<std::size_t>(relu_id)].outputs().empty();
      std::vector<std::string> inputs = conv.inputs();
      inputs.insert(inputs.end(), bn.inputs().begin() + 1, bn.inputs().end());
      Node& fused = g->mutable_nodes()[i];
      fused.set_name(fused.name() + (with_relu ? "_bn_relu" : "_bn"));
      fused.set_op_type(with_relu ? "FusedConvBatchNormRelu" : "FusedConvBatchNorm");
      fused.set_inputs(std::move(inputs));
      fused.set_outputs(with_relu ? g->nodes()[static_cast<std::size_t>(relu_id)].outputs()
                                  : bn.outputs());
      fused.SetAttribute("fused_batchnorm_relu", with_relu);
      fused.SetAttribute("batchnorm_epsilon", bn.GetAttribute<double>("epsilon").value_or(1e-5));
      removed->push_back(bn_id);
      if (with_relu) removed->push_back(relu_id);
      return true;
    });
  }
};

class AddReluFusionPass final : public GraphPass {
 public:
  const char* name() const override { return "add_relu_fusion"; }
  Status Run(Graph* graph) const override {
    return FuseToFixpoint(graph, [](Graph* g, std::size_t i, const auto& consumers,
                                    std::vector<int>* removed) {
      const Node& add = g->nodes()[i];
      if (add.op_type() != "Add" || add.outputs().size() != 1) return false;
      const int relu_id = SoleConsumer(consumers, add.outputs()[0], g->nodes().size());
      if (relu_id < 0) return false;
      const Node& relu = g->nodes()[static_cast<std::size_t>(relu_id)];
      if (relu.op_type() != "Relu" || relu.outputs().size() != 1) return false;
      Node& fused = g->mutable_nodes()[i];
      fused.set_name(fused.name() + "_relu");
      fused.set_op_type("AddRelu");
      fused.set_outputs(relu.outputs());
      removed->push_back(relu_id);
      return true;
    });
  }
};

class ConvBatchNormAddReluFusionPass final : public GraphPass {
 public:
  const char* name() const override { return "conv_batchnorm_add_relu_fusion"; }
  Status Run(Graph* graph) const override {
    return FuseToFixpoint(graph, [](Graph* g, std::size_t i, const auto& consumers,
                                    std::vector<int>* removed) {
      const Node& join = g->nodes()[i];
      if (join.op_type() != "AddRelu" || join.inputs().size() != 2 || join.outputs().size() != 1) {
        return false;
      }
      const auto producers = g->BuildProducerMap();
      // Prefer the operand produced last, so the other operand (the residual)
      // is already available when the fused convolution runs.
      int best = -1;
      int best_operand = -1;
      for (int operand = 0; operand < 2; ++operand) {
        const std::string& value = join.inputs()[static_cast<std::size_t>(operand)];
        const auto producer = producers.find(value);
        if (producer == producers.end()) continue;
        const Node& conv = g->nodes()[static_cast<std::size_t>(producer->second)];
        if (conv.op_type() != "FusedConvBatchNorm" || conv.outputs().size() != 1 ||
            conv.inputs().size() != 6 || IsGraphOutput(*g, value) ||
            SoleConsumer(consumers, value, g->nodes().size()) != static_cast<int>(i)) {
          continue;
        }
        if (producer->second > best) {
          best = producer->second;
          best_operand = operand;
        }
      }
      if (best < 0) return false;
      const std::string residual = join.inputs()[static_cast<std::size_t>(1 - best_operand)];
      if (residual == join.inputs()[static_cast<std::size_t>(best_operand)]) return false;
      const std::vector<std::string> outputs = join.outputs();
      Node& conv = g->mutable_nodes()[static_cast<std::size_t>(best)];
      std::vector<std::string> inputs = conv.inputs();
      inputs.push_back(residual);
      conv.set_name(conv.name() + "_add_relu");
      conv.set_op_type("FusedConvBatchNormAddRelu");
      conv.set_inputs(std::move(inputs));
      conv.set_outputs(outputs);
      removed->push_back(static_cast<int>(i));
      return true;
    });
  }
};

class GemmGeluFusionPass final : public GraphPass {
 public:
  const char* name() const override { return "gemm_gelu_fusion"; }
  Status Run(Graph* graph) const override {
    return FuseToFixpoint(graph, [](Graph* g, std::size_t i, const auto& consumers,
                                    std::vector<int>* removed) {
      const Node& gemm = g->nodes()[i];
      if (gemm.op_type() != "Gemm" || gemm.outputs().size() != 1 ||
          IsGraphOutput(*g, gemm.outputs()[0])) {
        return false;
      }
      const int gelu_id = SoleConsumer(consumers, gemm.outputs()[0], g->nodes().size());
      if (gelu_id < 0) return false;
      const Node& gelu = g->nodes()[static_cast<std::size_t>(gelu_id)];
      if (gelu.op_type() != "Gelu" || gelu.inputs().size() != 1 || gelu.outputs().size() != 1) {
        return false;
      }
      Node& fused = g->mutable_nodes()[i];
      fused.set_name(fused.name() + "_gelu");
      fused.set_op_type("GemmGelu");
      fused.set_outputs(gelu.outputs());
      removed->push_back(gelu_id);
      return true;
    });
  }
};

class SkipLayerNormalizationFusionPass final : public GraphPass {
 public:
  const char* name() const override { return "skip_layer_norm_fusion"; }
  Status Run(Graph* graph) const override {
    return FuseToFixpoint(graph, [](Graph* g, std::size_t i, const auto& consumers,
                                    std::vector<int>* removed) {
      const Node& add = g->nodes()[i];
      if (add.op_type() != "Add" || add.outputs().size() != 1 ||
          IsGraphOutput(*g, add.outputs()[0])) {
        return false;
      }
      const int norm_id = SoleConsumer(consumers, add.outputs()[0], g->nodes().size());
      if (norm_id < 0) return false;
      const Node norm = g->nodes()[static_cast<std::size_t>(norm_id)];
      if (norm.op_type() != "LayerNormalization" || norm.inputs().size() != 3 ||
          norm.outputs().size() != 1 || norm.inputs()[0] != add.outputs()[0]) {
        return false;
      }
      Node& fused = g->mutable_nodes()[i];
      std::vector<std::string> inputs = fused.inputs();
      inputs.push_back(norm.inputs()[1]);
      inputs.push_back(norm.inputs()[2]);
      fused.set_name(fused.name() + "_layer_norm");
      fused.set_op_type("SkipLayerNormalization");
      fused.set_inputs(std::move(inputs));
      fused.set_outputs(norm.outputs());
      fused.SetAttribute("axis", GetIntAttribute(norm, "axis", -1));
      fused.SetAttribute("epsilon", norm.GetAttribute<double>("epsilon").value_or(1e-5));
      removed->push_back(norm_id);
      return true;
    });
  }
};

class FlattenGemmNormalizationPass final : public GraphPass {
 public:
  const char* name() const override { return "flatten_gemm_normalization"; }
  Status Run(Graph* graph) const override {
    for (auto& node : graph->mutable_nodes()) {
      if (node.op_type() == "MatMul") {
        node.set_op_type("Gemm");
        node.SetAttribute("normalized_from_matmul", true);
      }
      if (node.op_type() == "Flatten" && !node.GetAttribute<int64_t>("axis").has_value()) {
        node.SetAttribute("axis", static_cast<int64_t>(1));
      }
    }
    return Status::OK();
  }
};

// Attention's `scale` as a float attribute: ONNX's default 1 / sqrt(D) from
// Q's head dimension when it is absent, a float when it was given as an
// integer. Kernels then read one value.
class AttentionScalePass final : public GraphPass {
 public:
  const char* name() const override { return "attention_scale"; }
  Status Run(Graph* graph) const override {
    for (auto& node : graph->mutable_nodes()) {
      if (node.op_type() != "Attention") continue;
      if (const auto given = node.GetAttribute<int64_t>("scale")) {
        node.SetAttribute("scale", static_cast<double>(*given));
      } else if (!node.GetAttribute<double>("scale")) {
        const ValueDesc* q = node.inputs().empty() ? nullptr : graph->FindValue(node.inputs()[0]);
        if (q == nullptr || q->tensor.shape.empty() || q->tensor.shape.back() <= 0) {
          return Status::ShapeError("Attention " + node.name() + " needs a known head dimension for its scale");
        }
        node.SetAttribute("scale", 1.0 / std::sqrt(static_cast<double>(q->tensor.shape.back())));
      }
    }
    return Status::OK();
  }
};

class StaticShapeValidationPass final : public GraphPass {
 public:
  const char* name() const override { return "static_shape_validation"; }
  Status Run(Graph* graph) const override {
    for (const auto& entry : graph->values()) {
      const ValueDesc& value = entry.second;
      if (value.tensor.dtype == DataType::kUnknown && !value.is_constant) continue;
      if (!value.tensor.shape.empty()) CUTRITON_RETURN_IF_ERROR(value.tensor.Validate());
    }
    for (const auto& name : graph->outputs()) {
      const ValueDesc* value = graph->FindValue(name);
      if (value == nullptr) return Status::NotFound("graph output is missing: " + name);
      CUTRITON_RETURN_IF_ERROR(value->tensor.Validate());
    }
    return Status::OK();
  }
};

}  // namespace

Status RegisterBuiltinOpSchemas() {
  auto& registry = OpSchemaRegistry::Global();
  auto add = [&](const char* op, std::size_t lo, std::size_t hi, ShapeInferenceFunction fn) {
    const Status status = registry.Register(OpSchema{op, lo, hi, 1, std::move(fn)});
    return status.code() == ErrorCode::kAlreadyExists ? Status::OK() : status;
  };
  CUTRITON_RETURN_IF_ERROR(add("Conv", 2, 2, InferConvLike));
  CUTRITON_RETURN_IF_ERROR(add("FusedConvBatchNorm", 6, 6, InferConvLike));
  CUTRITON_RETURN_IF_ERROR(add("FusedConvBatchNormRelu", 6, 6, InferConvLike));
  CUTRITON_RETURN_IF_ERROR(add("FusedConvBatchNormAddRelu", 7, 7, InferConvResidual));
  CUTRITON_RETURN_IF_ERROR(add("BatchNormalization", 5, 5, InferSameAsFirstInput));
  for (const char* op : {"Relu", "Gelu"}) {
    CUTRITON_RETURN_IF_ERROR(add(op, 1, 1, InferSameAsFirstInput));
  }
  CUTRITON_RETURN_IF_ERROR(add("Softmax", 1, 1, InferSoftmax));
  CUTRITON_RETURN_IF_ERROR(add("Attention", 3, 3, InferAttention));
  CUTRITON_RETURN_IF_ERROR(add("LayerNormalization", 2, 3, InferLayerNormalization));
  CUTRITON_RETURN_IF_ERROR(add("Add", 2, 2, InferElementwiseBinary));
  CUTRITON_RETURN_IF_ERROR(add("AddRelu", 2, 2, InferElementwiseBinary));
  CUTRITON_RETURN_IF_ERROR(add("Flatten", 1, 1, InferFlatten));
  CUTRITON_RETURN_IF_ERROR(add("Gemm", 2, 3, InferGemm));
  CUTRITON_RETURN_IF_ERROR(add("GemmGelu", 2, 3, InferGemm));
  CUTRITON_RETURN_IF_ERROR(add("MatMul", 2, 2, InferGemm));
  CUTRITON_RETURN_IF_ERROR(add("SkipLayerNormalization", 4, 4, InferSkipLayerNormalization));
  CUTRITON_RETURN_IF_ERROR(add("MaxPool", 1, 1, InferPool));
  CUTRITON_RETURN_IF_ERROR(add("AveragePool", 1, 1, InferPool));
  CUTRITON_RETURN_IF_ERROR(add("GlobalAveragePool", 1, 1, InferGlobalAveragePool));
  {
    const Status status = registry.Register(
        OpSchema{"Constant", 0, 0, 1, [](Graph*, const Node&) { return Status::OK(); }});
    if (!status.ok() && status.code() != ErrorCode::kAlreadyExists) return status;
  }
  return Status::OK();
}

void PassManager::Add(std::unique_ptr<GraphPass> pass) { passes_.push_back(std::move(pass)); }

Status PassManager::Run(Graph* graph) const {
  executed_passes_.clear();
  for (const auto& pass : passes_) {
    CUTRITON_RETURN_IF_ERROR(pass->Run(graph));
    executed_passes_.emplace_back(pass->name());
  }
  return Status::OK();
}

std::unique_ptr<GraphPass> CreateTopologicalSortPass() { return std::make_unique<TopologicalSortPass>(); }
std::unique_ptr<GraphPass> CreateShapeInferencePass() { return std::make_unique<ShapeInferencePass>(); }
std::unique_ptr<GraphPass> CreateConstantFoldingPass() { return std::make_unique<ConstantFoldingPass>(); }
std::unique_ptr<GraphPass> CreateDeadNodeEliminationPass() {
  return std::make_unique<DeadNodeEliminationPass>();
}
std::unique_ptr<GraphPass> CreateConvBatchNormReluFusionPass() {
  return std::make_unique<ConvBatchNormReluFusionPass>();
}
std::unique_ptr<GraphPass> CreateAddReluFusionPass() { return std::make_unique<AddReluFusionPass>(); }
std::unique_ptr<GraphPass> CreateConvBatchNormAddReluFusionPass() {
  return std::make_unique<ConvBatchNormAddReluFusionPass>();
}
std::unique_ptr<GraphPass> CreateGemmGeluFusionPass() { return std::make_unique<GemmGeluFusionPass>(); }
std::unique_ptr<GraphPass> CreateSkipLayerNormalizationFusionPass() {
  return std::make_unique<SkipLayerNormalizationFusionPass>();
}
std::unique_ptr<GraphPass> CreateFlattenGemmNormalizationPass() {
  return std::make_unique<FlattenGemmNormalizationPass>();
}
std::unique_ptr<GraphPass> CreateAttentionScalePass() { return std::make_unique<AttentionScalePass>(); }
std::unique_ptr<GraphPass> CreateStaticShapeValidationPass() {
  return std::make_unique<StaticShapeValidationPass>();
}

PassManager CreateDefaultCompilePasses(bool enable_transformer_fusions,
                                       bool enable_residual_epilogue_fusion) {
  PassManager manager;
  manager.Add(CreateTopologicalSortPass());
  manager.Add(CreateShapeInferencePass());
  manager.Add(CreateConstantFoldingPass());
  manager.Add(CreateDeadNodeEliminationPass());
  manager.Add(CreateConvBatchNormReluFusionPass());
  manager.Add(CreateAddReluFusionPass());
  if (enable_residual_epilogue_fusion) manager.Add(CreateConvBatchNormAddReluFusionPass());
  if (enable_transformer_fusions) {
    manager.Add(CreateGemmGeluFusionPass());
    manager.Add(CreateSkipLayerNormalizationFusionPass());
  }
  manager.Add(CreateTopologicalSortPass());
  manager.Add(CreateShapeInferencePass());
  manager.Add(CreateFlattenGemmNormalizationPass());
  manager.Add(CreateAttentionScalePass());
  manager.Add(CreateDeadNodeEliminationPass());
  manager.Add(CreateStaticShapeValidationPass());
  return manager;
}

}  // namespace cutriton
