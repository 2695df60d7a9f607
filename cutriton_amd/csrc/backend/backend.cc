// Backends, lowering and the backend registry.
//
// "hip_gfx950" lowers a node in three layers:
//   * a screen of the node itself: a HIP device, a registered schema whose
//     arity the node meets, FP32/FP16 tensors placed on that device, and at
//     least one pack entry for its op type (Flatten needs none: it is a view
//     and refused only as a graph output, which would need a copy);
//   * KernelFit, which decides whether one pack entry can run the node: the
//     device's architecture, the entry's dtype and layout, constant re-layouts
//     (OHWI / NK / T copies of constant inputs), and the declarative
//     constraints of the entry;
//   * candidates: one per fitting entry, then one per FusionRegistry
//     alternative whose recipe (the unfused op sequence) finds a fitting
//     default entry for every step; recipe intermediates are candidate
//     temporaries shaped like the fused output.
// The reference's lowering (src/backend/backend.cpp) yields the same
// candidate set: fused entries first, the decomposition last, defaults as the
// pack flags them; "cpu_reference" refuses every node.
#include "cutriton/backend/backend.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <map>
#include <mutex>

#include "cutriton/ir/fusion.h"
#include "cutriton/ir/op_schema.h"
#include "cutriton_hip_runtime.h"

namespace cutriton {
namespace {

using ValueLookup = std::function<const ValueDesc*(const std::string&)>;

class CpuReferenceBackend final : public Backend {
 public:
  const char* name() const override { return "cpu_reference"; }
  Status CheckSupport(const Node&, const Graph&, const BackendOptions&) const override {
    return Status::Unsupported("the CPU reference kernels are not implemented");
  }
  Status CreateKernel(const Node&, const Graph&, const BackendOptions&,
                      std::unique_ptr<OpKernel>*) const override {
    return Status::Unsupported("the CPU reference kernels are not implemented");
  }
};

// Flatten: the output shares the input's memory; nothing is launched.
class ViewKernel final : public OpKernel {
 public:
  const char* backend_name() const override { return kHipBackendName; }
  const char* op_type() const override { return "Flatten"; }
  Status Compute(KernelContext* context) override {
    const bool valid = context != nullptr && context->node != nullptr && context->tensors != nullptr;
    return valid ? Status::OK() : Status::InvalidArgument("Flatten KernelContext is invalid");
  }
};

const std::string& ValueName(const Node& node, bool output, int index) {
  static const std::string kNone;
  const auto& names = output ? node.outputs() : node.inputs();
  return index >= 0 && static_cast<std::size_t>(index) < names.size() ? names[static_cast<std::size_t>(index)] : kNone;
}

// Whether a pack entry can run a node on a device of numeric architecture
// `capability` (named `arch`).
class KernelFit {
 public:
  KernelFit(int capability, std::string arch) : capability_(capability), arch_(std::move(arch)) {}

  bool Accepts(const KernelArtifact& entry, const Node& node, const ValueLookup& lookup) const {
    return RunsOnDevice(entry) && TypesMatch(entry, node, lookup) && ConstantLayoutsMatch(entry, node, lookup) &&
           std::all_of(entry.constraints.begin(), entry.constraints.end(),
                       [&](const KernelConstraint& c) { return Holds(c, node, lookup); });
  }

 private:
  bool RunsOnDevice(const KernelArtifact& entry) const {
    return entry.min_compute_capability <= capability_ && (entry.target_arch.empty() || entry.target_arch == arch_);
  }

  // The entry's dtype is the node's (its first output, else first input);
  // its layout, when set, that of the first input and of every output.
  static bool TypesMatch(const KernelArtifact& entry, const Node& node, const ValueLookup& lookup) {
    const ValueDesc* typed = lookup(node.outputs().empty() ? node.inputs().front() : node.outputs().front());
    if (typed == nullptr || entry.dtype != DataTypeName(typed->tensor.dtype)) return false;
    auto in_layout = [&](const std::string& name) {
      const ValueDesc* value = lookup(name);
      return value != nullptr && (entry.layout.empty() || value->tensor.layout == entry.layout);
    };
    if (!node.inputs().empty() && !in_layout(node.inputs().front())) return false;
    return std::all_of(node.outputs().begin(), node.outputs().end(), in_layout);
  }

  // An argument read in another layout must be a constant of a shape that
  // layout is defined for (the engine makes the copy at constant upload).
  static bool ConstantLayoutsMatch(const KernelArtifact& entry, const Node& node, const ValueLookup& lookup) {
    for (const auto& argument : entry.arguments) {
      const std::string& layout = argument.source.layout;
      if (layout.empty()) continue;
      const ValueDesc* value = lookup(ValueName(node, false, argument.source.index));
      if (value == nullptr || !value->is_constant) return false;
      const std::size_t rank = value->tensor.shape.size();
      const bool defined = layout == "OHWI" ? rank == 4 && value->tensor.dtype == DataType::kFloat32
                                            : (layout == "NK" || layout == "T") && rank == 2;
      if (!defined) return false;
    }
    return true;
  }

  static bool Holds(const KernelConstraint& c, const Node& node, const ValueLookup& lookup) {
    switch (c.kind) {
      case KernelConstraintKind::kInputCountEquals:
        return node.inputs().size() == static_cast<std::size_t>(c.expected);
      case KernelConstraintKind::kAttributeInt64Equals:
        return GetIntAttribute(node, c.attribute_name, c.default_value) == c.expected;
      case KernelConstraintKind::kTensorRankEquals:
      case KernelConstraintKind::kTensorDimAtMost: {
        const ValueDesc* value = lookup(ValueName(node, c.tensor_is_output, c.tensor_index));
        if (value == nullptr) return false;
        const auto& shape = value->tensor.shape;
        if (c.kind == KernelConstraintKind::kTensorRankEquals) return shape.size() == static_cast<std::size_t>(c.expected);
        return static_cast<std::size_t>(c.tensor_axis) < shape.size() && shape[static_cast<std::size_t>(c.tensor_axis)] <= c.expected;
      }
      case KernelConstraintKind::kTensorBytesAtMost:
        for (const auto* names : {&node.inputs(), &node.outputs()}) {
          for (const auto& name : *names) {
            const ValueDesc* value = lookup(name);
            if (value == nullptr || static_cast<int64_t>(value->tensor.ByteSize()) > c.expected) return false;
          }
        }
        return true;
    }
    return false;
  }

  int capability_;
  std::string arch_;
};

// Inputs of a kernel step: constants read in another layout are bound under
// the name of their re-laid-out copy.
std::vector<std::string> StepInputs(const KernelArtifact& entry, std::vector<std::string> inputs) {
  for (const auto& argument : entry.arguments) {
    const int index = argument.source.index;
    if (argument.source.layout.empty() || index < 0 || static_cast<std::size_t>(index) >= inputs.size()) continue;
    inputs[static_cast<std::size_t>(index)] = LaidOutConstantName(inputs[static_cast<std::size_t>(index)], argument.source.layout);
  }
  return inputs;
}

// The unfused op sequence of a fused op. Operands name the fused node's
// inputs ("in0".."in6", "in*" for all of them), its output ("out") or a
// temporary ("t0", "t1": workspace slots 0 and 1, shaped like the output).
struct RecipeStep {
  const char* op;
  std::vector<const char*> inputs;
  const char* output;
};

const std::map<std::string, std::vector<RecipeStep>>& Recipes() {
  static const std::map<std::string, std::vector<RecipeStep>> recipes = {
      {"FusedConvBatchNormRelu",
       {{"Conv", {"in0", "in1"}, "t0"},
        {"BatchNormalization", {"t0", "in2", "in3", "in4", "in5"}, "t1"},
        {"Relu", {"t1"}, "out"}}},
      {"FusedConvBatchNorm",
       {{"Conv", {"in0", "in1"}, "t0"}, {"BatchNormalization", {"t0", "in2", "in3", "in4", "in5"}, "out"}}},
      {"FusedConvBatchNormAddRelu",
       {{"FusedConvBatchNorm", {"in0", "in1", "in2", "in3", "in4", "in5"}, "t0"}, {"AddRelu", {"t0", "in6"}, "out"}}},
      {"AddRelu", {{"Add", {"in0", "in1"}, "t0"}, {"Relu", {"t0"}, "out"}}},
      {"GemmGelu", {{"Gemm", {"in*"}, "t0"}, {"Gelu", {"t0"}, "out"}}},
      {"SkipLayerNormalization",
       {{"Add", {"in0", "in1"}, "t0"}, {"LayerNormalization", {"t0", "in2", "in3"}, "out"}}},
  };
  return recipes;
}

class HipLowering {
 public:
  HipLowering(const Node& node, const Graph& graph, const ArtifactRepository& repository, KernelFit fit)
      : node_(node), graph_(graph), repository_(repository), fit_(std::move(fit)) {}

  // One candidate per pack entry that fits the node.
  void AddFusedEntries(const KernelCatalog& catalog, int capability, std::vector<ExecutionCandidate>* out) const {
    const ValueLookup lookup = [&](const std::string& name) { return graph_.FindValue(name); };
    const std::string dtype = DataTypeName(graph_.FindValue(node_.outputs().front())->tensor.dtype);
    const std::string layout = node_.inputs().empty() ? std::string() : graph_.FindValue(node_.inputs().front())->tensor.layout;
    for (const KernelArtifact* entry : catalog.Query(node_.op_type(), dtype, layout, capability)) {
      if (!fit_.Accepts(*entry, node_, lookup)) continue;
      ExecutionCandidate candidate;
      candidate.candidate_id = entry->identity();
      candidate.is_default = entry->is_default;
      candidate.steps.push_back(KernelInvocation{*entry, StepInputs(*entry, node_.inputs()), node_.outputs()});
      out->push_back(std::move(candidate));
    }
  }

  // The decomposition of `alternative`, or false when a step has no default
  // entry that fits it.
  bool BuildDecomposition(const FusionAlternative& alternative, ExecutionCandidate* candidate) const {
    const auto recipe = Recipes().find(node_.op_type());
    if (recipe == Recipes().end()) return false;
    const std::string& output = node_.outputs().front();
    const std::string dtype = DataTypeName(graph_.FindValue(output)->tensor.dtype);
    std::map<std::string, std::string> temporaries;  // operand -> value name
    auto resolve = [&](const std::string& operand, std::vector<std::string>* names) {
      if (operand == "out") {
        names->push_back(output);
      } else if (operand == "in*") {
        names->insert(names->end(), node_.inputs().begin(), node_.inputs().end());
      } else if (operand.rfind("in", 0) == 0) {
        names->push_back(node_.inputs().at(static_cast<std::size_t>(std::stoi(operand.substr(2)))));
      } else {
        auto [slot, fresh] = temporaries.try_emplace(operand, node_.name() + "::" + operand);
        if (fresh) {
          candidate->temporaries.push_back(
              CandidateTemporary{slot->second, output, static_cast<std::size_t>(std::stoi(operand.substr(1)))});
        }
        names->push_back(slot->second);
      }
    };
    // Temporaries are described like the fused output.
    const ValueLookup lookup = [&](const std::string& name) -> const ValueDesc* {
      for (const auto& temporary : candidate->temporaries) {
        if (temporary.name == name) return graph_.FindValue(output);
      }
      return graph_.FindValue(name);
    };
    candidate->candidate_id = alternative.candidate_id;
    for (const RecipeStep& step : recipe->second) {
      std::vector<std::string> inputs;
      std::vector<std::string> outputs;
      for (const char* operand : step.inputs) resolve(operand, &inputs);
      resolve(step.output, &outputs);
      // The step is a node of its own carrying the fused node's attributes.
      Node probe(node_.name(), step.op, inputs, outputs);
      for (const auto& [key, value] : node_.attributes()) probe.SetAttribute(key, value);
      const auto* entries = repository_.Find(step.op);
      const KernelArtifact* chosen = nullptr;
      for (std::size_t i = 0; entries != nullptr && i < entries->size() && chosen == nullptr; ++i) {
        const KernelArtifact& entry = (*entries)[i];
        if (entry.is_default && entry.dtype == dtype && fit_.Accepts(entry, probe, lookup)) chosen = &entry;
      }
      if (chosen == nullptr) return false;
      candidate->steps.push_back(KernelInvocation{*chosen, StepInputs(*chosen, inputs), outputs});
    }
    return true;
  }

 private:
  const Node& node_;
  const Graph& graph_;
  const ArtifactRepository& repository_;
  KernelFit fit_;
};

std::string BaseArch(const std::string& full) { return full.substr(0, full.find(':')); }

// What every HIP node must satisfy before its pack entries are consulted.
Status ScreenHipNode(const Node& node, const Graph& graph, const BackendOptions& options,
                     const ArtifactRepository& repository) {
  if (options.device.type != DeviceType::kHIP) {
    return Status::Unsupported(std::string(kHipBackendName) + " requires a HIP device");
  }
  CUTRITON_RETURN_IF_ERROR(RegisterBuiltinOpSchemas());
  const auto schema = OpSchemaRegistry::Global().Find(node.op_type());
  if (schema == nullptr) return Status::Unsupported("no OpSchema is registered for " + node.op_type());
  const std::size_t inputs = node.inputs().size();
  if (inputs < schema->min_inputs || inputs > schema->max_inputs || node.outputs().size() != schema->outputs) {
    return Status::Unsupported(node.op_type() + " has an invalid input/output count");
  }
  for (const auto* names : {&node.inputs(), &node.outputs()}) {
    for (const auto& name : *names) {
      const ValueDesc* value = graph.FindValue(name);
      if (value == nullptr) return Status::NotFound("tensor description is missing: " + name);
      CUTRITON_RETURN_IF_ERROR(value->tensor.Validate());
      const DataType dtype = value->tensor.dtype;
      if (dtype != DataType::kFloat32 && dtype != DataType::kFloat16) {
        return Status::Unsupported("only float32/float16 tensors are supported: " + name);
      }
      if (value->tensor.device_type != options.device.type || value->tensor.device_id != options.device.id) {
        return Status::Unsupported("tensor is assigned to another device: " + name);
      }
    }
  }
  if (node.op_type() == "Flatten") {
    const auto& outputs = graph.outputs();
    if (std::find(outputs.begin(), outputs.end(), node.outputs().front()) != outputs.end()) {
      return Status::Unsupported("a Flatten graph output needs an explicit copy kernel");
    }
    return Status::OK();
  }
  const auto* entries = repository.Find(node.op_type());
  if (entries == nullptr || entries->empty()) return Status::Unsupported("no Kernel Pack entry for " + node.op_type());
  int capability = 0;
  std::string arch;
  CUTRITON_RETURN_IF_ERROR(DeviceArchitecture(options.device.id, &capability, &arch));
  const KernelFit fit(capability, arch);
  const ValueLookup lookup = [&](const std::string& name) { return graph.FindValue(name); };
  const bool any = std::any_of(entries->begin(), entries->end(),
                               [&](const KernelArtifact& entry) { return fit.Accepts(entry, node, lookup); });
  return any ? Status::OK()
             : Status::Unsupported("no Kernel Pack variant of " + node.op_type() +
                                   " matches dtype/layout/architecture/constraints");
}

class HipBackend final : public Backend {
 public:
  const char* name() const override { return kHipBackendName; }

  Status CheckSupport(const Node& node, const Graph& graph, const BackendOptions& options) const override {
    std::vector<std::string> paths = options.kernel_artifact_paths;
    if (paths.empty() && !options.kernel_artifact_dir.empty()) paths.push_back(options.kernel_artifact_dir);
    ArtifactRepository repository;
    CUTRITON_RETURN_IF_ERROR(repository.Load(paths));
    return ScreenHipNode(node, graph, options, repository);
  }

  Status Lower(const Node& node, const LoweringContext& context,
               std::vector<ExecutionCandidate>* candidates) const override {
    if (candidates == nullptr || context.graph == nullptr || context.options == nullptr ||
        context.artifacts == nullptr || context.catalog == nullptr) {
      return Status::InvalidArgument("HIP lowering context is incomplete");
    }
    CUTRITON_RETURN_IF_ERROR(ScreenHipNode(node, *context.graph, *context.options, *context.artifacts));
    candidates->clear();
    if (node.op_type() == "Flatten") {
      ExecutionCandidate view;
      view.candidate_id = "view:flatten";
      view.is_default = true;
      view.steps.push_back(ViewInvocation{node.inputs().front(), node.outputs().front()});
      candidates->push_back(std::move(view));
      return Status::OK();
    }
    int capability = 0;
    std::string arch;
    CUTRITON_RETURN_IF_ERROR(DeviceArchitecture(context.options->device.id, &capability, &arch));
    const HipLowering lowering(node, *context.graph, *context.artifacts, KernelFit(capability, arch));
    lowering.AddFusedEntries(*context.catalog, capability, candidates);
    CUTRITON_RETURN_IF_ERROR(RegisterBuiltinFusionAlternatives());
    for (const auto& alternative : FusionRegistry::Global().Find(node.op_type())) {
      ExecutionCandidate candidate;
      if (lowering.BuildDecomposition(alternative, &candidate)) candidates->push_back(std::move(candidate));
    }
    if (candidates->empty()) return Status::Unsupported("no compatible artifact for " + node.op_type());
    return Status::OK();
  }

  Status CreateKernel(const Node& node, const Graph&, const BackendOptions&,
                      std::unique_ptr<OpKernel>* kernel) const override {
    if (kernel == nullptr) return Status::InvalidArgument("OpKernel output pointer is null");
    if (node.op_type() != "Flatten") {
      return Status::Unsupported("artifact kernels are instantiated from KernelInvocations");
    }
    *kernel = std::make_unique<ViewKernel>();
    return Status::OK();
  }
};

Status RegisterOnce(std::shared_ptr<Backend> backend) {
  auto& registry = KernelRegistry::Global();
  if (registry.GetBackend(backend->name()) != nullptr) return Status::OK();
  const Status status = registry.RegisterBackend(std::move(backend));
  return status.code() == ErrorCode::kAlreadyExists ? Status::OK() : status;
}

}  // namespace

Status CheckCandidateShapes(const ExecutionCandidate& candidate, const Graph& graph) {
  // Temporaries take the shape of their "like" value; re-laid-out constant
  // copies keep their original's byte size.
  auto describe = [&](std::string name) -> const ValueDesc* {
    for (const auto& temporary : candidate.temporaries) {
      if (temporary.name == name) name = temporary.like_value;
    }
    const auto copy = name.rfind('#');
    return graph.FindValue(copy == std::string::npos ? name : name.substr(0, copy));
  };
  for (const auto& step : candidate.steps) {
    const auto* invocation = std::get_if<KernelInvocation>(&step);
    if (invocation == nullptr) continue;
    for (const auto& constraint : invocation->artifact.constraints) {
      if (constraint.kind != KernelConstraintKind::kTensorBytesAtMost) continue;
      for (const auto* names : {&invocation->inputs, &invocation->outputs}) {
        for (const auto& name : *names) {
          const ValueDesc* value = describe(name);
          if (value == nullptr) return Status::NotFound("tensor description is missing: " + name);
          if (static_cast<int64_t>(value->tensor.ByteSize()) > constraint.expected) {
            return Status::Unsupported(invocation->artifact.kernel_id + " addresses at most " +
                                       std::to_string(constraint.expected) + " bytes per tensor; " + name + " holds " +
                                       std::to_string(value->tensor.ByteSize()));
          }
        }
      }
    }
  }
  return Status::OK();
}

Status Backend::Lower(const Node& node, const LoweringContext& context,
                      std::vector<ExecutionCandidate>* candidates) const {
  if (candidates == nullptr || context.graph == nullptr || context.options == nullptr) {
    return Status::InvalidArgument("lowering context is incomplete");
  }
  CUTRITON_RETURN_IF_ERROR(CheckSupport(node, *context.graph, *context.options));
  ExecutionCandidate legacy;
  legacy.candidate_id = std::string(name()) + ":legacy:" + node.op_type();
  legacy.is_default = true;
  candidates->assign(1, std::move(legacy));
  return Status::OK();
}

KernelRegistry& KernelRegistry::Global() {
  static KernelRegistry registry;
  return registry;
}

Status KernelRegistry::RegisterBackend(std::shared_ptr<Backend> backend) {
  if (backend == nullptr) return Status::InvalidArgument("Backend must not be null");
  std::string key = backend->name();
  if (key.empty()) return Status::InvalidArgument("Backend name must not be empty");
  std::unique_lock<std::shared_mutex> lock(mutex_);
  if (!backends_.try_emplace(key, std::move(backend)).second) {
    return Status::AlreadyExists("Backend is already registered: " + key);
  }
  return Status::OK();
}

std::shared_ptr<Backend> KernelRegistry::GetBackend(const std::string& name) const {
  std::shared_lock<std::shared_mutex> lock(mutex_);
  const auto found = backends_.find(name);
  return found == backends_.end() ? nullptr : found->second;
}

std::vector<std::string> KernelRegistry::AvailableBackends() const {
  std::vector<std::string> names;
  {
    std::shared_lock<std::shared_mutex> lock(mutex_);
    for (const auto& entry : backends_) names.push_back(entry.first);
  }
  std::sort(names.begin(), names.end());
  return names;
}

void KernelRegistry::ClearForTests() {
  std::unique_lock<std::shared_mutex> lock(mutex_);
  backends_.clear();
}

std::shared_ptr<Backend> CreateCpuReferenceBackend() { return std::make_shared<CpuReferenceBackend>(); }
std::shared_ptr<Backend> CreateHipBackend() { return std::make_shared<HipBackend>(); }

Status RegisterBuiltinBackends() {
  CUTRITON_RETURN_IF_ERROR(RegisterOnce(CreateCpuReferenceBackend()));
  return RegisterOnce(CreateHipBackend());
}

Status DeviceArchitecture(int device_id, int* numeric_arch, std::string* arch_name) {
  if (numeric_arch == nullptr || arch_name == nullptr) return Status::InvalidArgument("architecture outputs are null");
  // CUTRITON_TARGET_ARCH (e.g. "gfx950") plans for a device that is not
  // attached: lowering and memory planning then run without a GPU.
  if (const char* forced = std::getenv("CUTRITON_TARGET_ARCH"); forced != nullptr && std::strncmp(forced, "gfx", 3) == 0) {
    *arch_name = BaseArch(forced);
    *numeric_arch = std::atoi(forced + 3);
    return Status::OK();
  }
  static std::mutex mutex;
  static std::map<int, std::pair<int, std::string>> known;
  std::lock_guard<std::mutex> lock(mutex);
  auto found = known.find(device_id);
  if (found == known.end()) {
    cth_device_info info;
    if (cth_device_query(device_id, &info) != 0) {
      return Status::RuntimeError(std::string("HIP device query failed: ") + cth_last_error());
    }
    found = known.emplace(device_id, std::make_pair(info.numeric_arch, BaseArch(info.arch_name))).first;
  }
  *numeric_arch = found->second.first;
  *arch_name = found->second.second;
  return Status::OK();
}

}  // namespace cutriton
