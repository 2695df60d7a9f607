// Graph passes and the default compile pipeline.
//
// Fusions are chain rewrites: a node whose output has exactly one reader,
// which is a node of an expected op type, merges with that reader (and
// possibly the reader's own sole reader). Each fusion is a matcher that
// proposes a Rewrite for one starting node; the driver collects, per sweep,
// every proposal whose nodes no earlier proposal of the sweep claimed, applies
// them all, and sweeps again until nothing matches. A value that is a graph
// output is never fused away.
//
// The rewrites and the pipeline order are the reference's
// (src/ir/pass.cpp:266-501, 666-684): Conv + BatchNormalization [+ Relu] ->
// FusedConvBatchNorm[Relu] (attributes fused_batchnorm_relu and
// batchnorm_epsilon), Add + Relu -> AddRelu, Gemm + Gelu -> GemmGelu, Add +
// LayerNormalization -> SkipLayerNormalization (axis, epsilon), MatMul ->
// Gemm, Flatten's default axis 1; the fused node keeps the first node's name
// with a suffix. Added here: FusedConvBatchNorm + AddRelu ->
// FusedConvBatchNormAddRelu (the residual join in the convolution epilogue)
// and Attention's default scale.
#include "cutriton/ir/pass.h"

#include <algorithm>
#include <cmath>
#include <deque>
#include <optional>
#include <unordered_set>

#include "cutriton/ir/op_schema.h"

namespace cutriton {
namespace {

// Edits a fusion makes: the `keep` node takes a new identity, `drop` nodes go.
struct Rewrite {
  int keep{-1};
  std::string name;
  std::string op_type;
  std::vector<std::string> inputs;
  std::vector<std::string> outputs;
  std::vector<std::pair<std::string, Attribute>> attributes;
  std::vector<int> drop;
};

class FusionScope {
 public:
  explicit FusionScope(const Graph& graph)
      : graph_(graph), readers_(graph.BuildConsumerMap()), producer_(graph.BuildProducerMap()),
        outputs_(graph.outputs().begin(), graph.outputs().end()) {}

  const Graph& graph() const { return graph_; }
  bool IsGraphOutput(const std::string& value) const { return outputs_.count(value) != 0; }

  // The one node reading `value` when it is private to the graph and read
  // exactly once, if that node has op type `op`.
  const Node* SoleReader(const std::string& value, const char* op) const {
    if (IsGraphOutput(value)) return nullptr;
    const auto found = readers_.find(value);
    if (found == readers_.end() || found->second.size() != 1) return nullptr;
    const Node& reader = graph_.nodes().at(static_cast<std::size_t>(found->second.front()));
    return reader.op_type() == op ? &reader : nullptr;
  }
  const Node* Producer(const std::string& value) const {
    const auto found = producer_.find(value);
    return found == producer_.end() ? nullptr : &graph_.nodes().at(static_cast<std::size_t>(found->second));
  }

 private:
  const Graph& graph_;
  std::unordered_map<std::string, std::vector<int>> readers_;
  std::unordered_map<std::string, int> producer_;
  std::unordered_set<std::string> outputs_;
};

using Matcher = std::optional<Rewrite> (*)(const FusionScope&, const Node&);

bool SingleOutput(const Node& node) { return node.outputs().size() == 1; }

// Conv -> BatchNormalization [-> Relu].
std::optional<Rewrite> MatchConvBatchNorm(const FusionScope& scope, const Node& conv) {
  if (conv.op_type() != "Conv" || !SingleOutput(conv)) return std::nullopt;
  const Node* bn = scope.SoleReader(conv.outputs()[0], "BatchNormalization");
  if (bn == nullptr || !SingleOutput(*bn) || bn->inputs().size() < 1) return std::nullopt;
  const Node* relu = scope.SoleReader(bn->outputs()[0], "Relu");
  if (relu != nullptr && relu->outputs().empty()) relu = nullptr;
  Rewrite r;
  r.keep = conv.id();
  r.name = conv.name() + (relu != nullptr ? "_bn_relu" : "_bn");
  r.op_type = relu != nullptr ? "FusedConvBatchNormRelu" : "FusedConvBatchNorm";
  r.inputs = conv.inputs();
  r.inputs.insert(r.inputs.end(), bn->inputs().begin() + 1, bn->inputs().end());
  r.outputs = relu != nullptr ? relu->outputs() : bn->outputs();
  r.attributes = {{"fused_batchnorm_relu", relu != nullptr},
                  {"batchnorm_epsilon", bn->GetAttribute<double>("epsilon").value_or(1e-5)}};
  r.drop = {bn->id()};
  if (relu != nullptr) r.drop.push_back(relu->id());
  return r;
}

// Add -> Relu.
std::optional<Rewrite> MatchAddRelu(const FusionScope& scope, const Node& add) {
  if (add.op_type() != "Add" || !SingleOutput(add)) return std::nullopt;
  const Node* relu = scope.SoleReader(add.outputs()[0], "Relu");
  if (relu == nullptr || !SingleOutput(*relu)) return std::nullopt;
  Rewrite r;
  r.keep = add.id();
  r.name = add.name() + "_relu";
  r.op_type = "AddRelu";
  r.inputs = add.inputs();
  r.outputs = relu->outputs();
  r.drop = {relu->id()};
  return r;
}

// AddRelu(conv, residual) where conv is a FusedConvBatchNorm read only by the
// join: the join moves into the convolution's epilogue. Of two such operands
// the one produced later is fused, so that the other (the residual) is
// already computed when the fused convolution runs.
std::optional<Rewrite> MatchResidualEpilogue(const FusionScope& scope, const Node& join) {
  if (join.op_type() != "AddRelu" || join.inputs().size() != 2 || !SingleOutput(join)) return std::nullopt;
  if (join.inputs()[0] == join.inputs()[1]) return std::nullopt;
  const Node* conv = nullptr;
  std::size_t conv_operand = 0;
  for (std::size_t operand = 0; operand < 2; ++operand) {
    const std::string& value = join.inputs()[operand];
    const Node* producer = scope.Producer(value);
    const bool eligible = producer != nullptr && producer->op_type() == "FusedConvBatchNorm" &&
                          SingleOutput(*producer) && producer->inputs().size() == 6 &&
                          scope.SoleReader(value, "AddRelu") == &join;
    if (eligible && (conv == nullptr || producer->id() > conv->id())) {
      conv = producer;
      conv_operand = operand;
    }
  }
  if (conv == nullptr) return std::nullopt;
  Rewrite r;
  r.keep = conv->id();
  r.name = conv->name() + "_add_relu";
  r.op_type = "FusedConvBatchNormAddRelu";
  r.inputs = conv->inputs();
  r.inputs.push_back(join.inputs()[1 - conv_operand]);
  r.outputs = join.outputs();
  r.drop = {join.id()};
  return r;
}

// Gemm -> Gelu.
std::optional<Rewrite> MatchGemmGelu(const FusionScope& scope, const Node& gemm) {
  if (gemm.op_type() != "Gemm" || !SingleOutput(gemm)) return std::nullopt;
  const Node* gelu = scope.SoleReader(gemm.outputs()[0], "Gelu");
  if (gelu == nullptr || gelu->inputs().size() != 1 || !SingleOutput(*gelu)) return std::nullopt;
  Rewrite r;
  r.keep = gemm.id();
  r.name = gemm.name() + "_gelu";
  r.op_type = "GemmGelu";
  r.inputs = gemm.inputs();
  r.outputs = gelu->outputs();
  r.drop = {gelu->id()};
  return r;
}

// Add -> LayerNormalization(sum, scale, bias).
std::optional<Rewrite> MatchSkipLayerNorm(const FusionScope& scope, const Node& add) {
  if (add.op_type() != "Add" || !SingleOutput(add)) return std::nullopt;
  const Node* norm = scope.SoleReader(add.outputs()[0], "LayerNormalization");
  if (norm == nullptr || norm->inputs().size() != 3 || !SingleOutput(*norm) || norm->inputs()[0] != add.outputs()[0]) {
    return std::nullopt;
  }
  Rewrite r;
  r.keep = add.id();
  r.name = add.name() + "_layer_norm";
  r.op_type = "SkipLayerNormalization";
  r.inputs = add.inputs();
  r.inputs.insert(r.inputs.end(), norm->inputs().begin() + 1, norm->inputs().end());
  r.outputs = norm->outputs();
  r.attributes = {{"axis", GetIntAttribute(*norm, "axis", -1)},
                  {"epsilon", norm->GetAttribute<double>("epsilon").value_or(1e-5)}};
  r.drop = {norm->id()};
  return r;
}

Status FuseUntilStable(Graph* graph, Matcher matcher) {
  for (;;) {
    std::vector<Rewrite> rewrites;
    {
      const FusionScope scope(*graph);
      std::unordered_set<int> claimed;
      for (const Node& node : graph->nodes()) {
        std::optional<Rewrite> r = matcher(scope, node);
        if (!r) continue;
        std::vector<int> touched = r->drop;
        touched.push_back(r->keep);
        if (std::any_of(touched.begin(), touched.end(), [&](int id) { return claimed.count(id) != 0; })) continue;
        claimed.insert(touched.begin(), touched.end());
        rewrites.push_back(std::move(*r));
      }
    }
    if (rewrites.empty()) return Status::OK();
    std::vector<int> dropped;
    for (Rewrite& r : rewrites) {
      Node& node = graph->mutable_nodes().at(static_cast<std::size_t>(r.keep));
      node.set_name(std::move(r.name));
      node.set_op_type(std::move(r.op_type));
      node.set_inputs(std::move(r.inputs));
      node.set_outputs(std::move(r.outputs));
      for (auto& [key, value] : r.attributes) node.SetAttribute(key, std::move(value));
      dropped.insert(dropped.end(), r.drop.begin(), r.drop.end());
    }
    CUTRITON_RETURN_IF_ERROR(graph->RemoveNodes(dropped));
  }
}

class FusionPass final : public GraphPass {
 public:
  FusionPass(const char* name, Matcher matcher) : name_(name), matcher_(matcher) {}
  const char* name() const override { return name_; }
  Status Run(Graph* graph) const override { return FuseUntilStable(graph, matcher_); }

 private:
  const char* name_;
  Matcher matcher_;
};

// A pass given by a plain function.
class FunctionPass final : public GraphPass {
 public:
  using Body = Status (*)(Graph*);
  FunctionPass(const char* name, Body body) : name_(name), body_(body) {}
  const char* name() const override { return name_; }
  Status Run(Graph* graph) const override { return body_(graph); }

 private:
  const char* name_;
  Body body_;
};

Status SortNodes(Graph* graph) { return graph->TopologicalSort(); }

// Runs every node's schema rule in node order, checking arity first.
Status InferShapes(Graph* graph) {
  CUTRITON_RETURN_IF_ERROR(RegisterBuiltinOpSchemas());
  const auto& registry = OpSchemaRegistry::Global();
  for (const Node& node : graph->nodes()) {
    const auto schema = registry.Find(node.op_type());
    if (schema == nullptr) return Status::Unsupported("no shape inference for op " + node.op_type());
    const std::size_t inputs = node.inputs().size();
    if (inputs < schema->min_inputs || inputs > schema->max_inputs || node.outputs().size() != schema->outputs) {
      return Status::ShapeError("input/output count violates the OpSchema: " + node.name());
    }
    CUTRITON_RETURN_IF_ERROR(schema->infer(graph, node));
  }
  return Status::OK();
}

// Constants carry no folding opportunity in the supported graphs; the pass
// keeps its place in the pipeline.
Status FoldConstants(Graph*) { return Status::OK(); }

// Keeps the nodes a graph output depends on: a walk from the outputs back
// through producers.
Status EliminateDeadNodes(Graph* graph) {
  const auto producer = graph->BuildProducerMap();
  std::vector<bool> live(graph->nodes().size(), false);
  std::unordered_set<std::string> seen(graph->outputs().begin(), graph->outputs().end());
  std::deque<std::string> pending(graph->outputs().begin(), graph->outputs().end());
  while (!pending.empty()) {
    const std::string value = pending.front();
    pending.pop_front();
    const auto found = producer.find(value);
    if (found == producer.end() || live[static_cast<std::size_t>(found->second)]) continue;
    live[static_cast<std::size_t>(found->second)] = true;
    for (const auto& input : graph->nodes()[static_cast<std::size_t>(found->second)].inputs()) {
      if (seen.insert(input).second) pending.push_back(input);
    }
  }
  std::vector<int> dead;
  for (const Node& node : graph->nodes()) {
    if (!live[static_cast<std::size_t>(node.id())]) dead.push_back(node.id());
  }
  return graph->RemoveNodes(dead);
}

Status NormalizeFlattenAndMatMul(Graph* graph) {
  for (Node& node : graph->mutable_nodes()) {
    if (node.op_type() == "MatMul") {
      node.set_op_type("Gemm");
      node.SetAttribute("normalized_from_matmul", true);
    } else if (node.op_type() == "Flatten" && !node.GetAttribute<int64_t>("axis")) {
      node.SetAttribute("axis", static_cast<int64_t>(1));
    }
  }
  return Status::OK();
}

// Attention's `scale` as one float attribute: ONNX's default 1 / sqrt(D) from
// Q's head dimension when absent, a float when given as an integer.
Status SettleAttentionScale(Graph* graph) {
  for (Node& node : graph->mutable_nodes()) {
    if (node.op_type() != "Attention") continue;
    if (const auto integral = node.GetAttribute<int64_t>("scale")) {
      node.SetAttribute("scale", static_cast<double>(*integral));
      continue;
    }
    if (node.GetAttribute<double>("scale")) continue;
    const ValueDesc* q = node.inputs().empty() ? nullptr : graph->FindValue(node.inputs()[0]);
    if (q == nullptr || q->tensor.shape.empty() || q->tensor.shape.back() <= 0) {
      return Status::ShapeError("Attention " + node.name() + " needs a known head dimension for its scale");
    }
    node.SetAttribute("scale", 1.0 / std::sqrt(static_cast<double>(q->tensor.shape.back())));
  }
  return Status::OK();
}

// Every described value and every graph output has a valid static shape.
Status ValidateStaticShapes(Graph* graph) {
  for (const auto& [name, value] : graph->values()) {
    const bool described = value.tensor.dtype != DataType::kUnknown || value.is_constant;
    if (described && !value.tensor.shape.empty()) CUTRITON_RETURN_IF_ERROR(value.tensor.Validate());
  }
  for (const auto& name : graph->outputs()) {
    const ValueDesc* value = graph->FindValue(name);
    if (value == nullptr) return Status::NotFound("graph output is missing: " + name);
    CUTRITON_RETURN_IF_ERROR(value->tensor.Validate());
  }
  return Status::OK();
}

}  // namespace

void PassManager::Add(std::unique_ptr<GraphPass> pass) { passes_.push_back(std::move(pass)); }

Status PassManager::Run(Graph* graph) const {
  executed_passes_.clear();
  for (const auto& pass : passes_) {
    CUTRITON_RETURN_IF_ERROR(pass->Run(graph));
    executed_passes_.emplace_back(pass->name());
  }
  return Status::OK();
}

std::unique_ptr<GraphPass> CreateTopologicalSortPass() {
  return std::make_unique<FunctionPass>("topological_sort", SortNodes);
}
std::unique_ptr<GraphPass> CreateShapeInferencePass() {
  return std::make_unique<FunctionPass>("shape_inference", InferShapes);
}
std::unique_ptr<GraphPass> CreateConstantFoldingPass() {
  return std::make_unique<FunctionPass>("constant_folding", FoldConstants);
}
std::unique_ptr<GraphPass> CreateDeadNodeEliminationPass() {
  return std::make_unique<FunctionPass>("dead_node_elimination", EliminateDeadNodes);
}
std::unique_ptr<GraphPass> CreateConvBatchNormReluFusionPass() {
  return std::make_unique<FusionPass>("conv_batchnorm_relu_fusion", MatchConvBatchNorm);
}
std::unique_ptr<GraphPass> CreateAddReluFusionPass() {
  return std::make_unique<FusionPass>("add_relu_fusion", MatchAddRelu);
}
std::unique_ptr<GraphPass> CreateConvBatchNormAddReluFusionPass() {
  return std::make_unique<FusionPass>("conv_batchnorm_add_relu_fusion", MatchResidualEpilogue);
}
std::unique_ptr<GraphPass> CreateGemmGeluFusionPass() {
  return std::make_unique<FusionPass>("gemm_gelu_fusion", MatchGemmGelu);
}
std::unique_ptr<GraphPass> CreateSkipLayerNormalizationFusionPass() {
  return std::make_unique<FusionPass>("skip_layer_norm_fusion", MatchSkipLayerNorm);
}
std::unique_ptr<GraphPass> CreateFlattenGemmNormalizationPass() {
  return std::make_unique<FunctionPass>("flatten_gemm_normalization", NormalizeFlattenAndMatMul);
}
std::unique_ptr<GraphPass> CreateAttentionScalePass() {
  return std::make_unique<FunctionPass>("attention_scale", SettleAttentionScale);
}
std::unique_ptr<GraphPass> CreateStaticShapeValidationPass() {
  return std::make_unique<FunctionPass>("static_shape_validation", ValidateStaticShapes);
}

PassManager CreateDefaultCompilePasses(bool enable_transformer_fusions, bool enable_residual_epilogue_fusion) {
  PassManager manager;
  // Canonical order and shapes, then the fusions, then the same again over
  // the fused graph.
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
