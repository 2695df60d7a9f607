// Backends and lowering. Behaviour follows reference
// src/backend/backend.cpp:22-453: the "cpu_reference" backend refuses every
// node, the artifact backend checks device/schema/tensors, lowers a node to
// one candidate per matching pack variant plus one FusionRegistry
// decomposition built from default variants with named temporaries, and
// Flatten lowers to a view. Device capability is the gfx architecture number.
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

// Flatten shares its input's memory; nothing is launched.
class ViewKernel final : public OpKernel {
 public:
  const char* backend_name() const override { return kHipBackendName; }
  const char* op_type() const override { return "Flatten"; }
  Status Compute(KernelContext* context) override {
    if (context == nullptr || context->node == nullptr || context->tensors == nullptr) {
      return Status::InvalidArgument("Flatten KernelContext is invalid");
    }
    return Status::OK();
  }
};

using ValueLookup = std::function<const ValueDesc*(const std::string&)>;

Status CheckTensor(const Graph& graph, const std::string& name, const Device& device) {
  const ValueDesc* value = graph.FindValue(name);
  if (value == nullptr) return Status::NotFound("tensor description is missing: " + name);
  CUTRITON_RETURN_IF_ERROR(value->tensor.Validate());
  if (value->tensor.dtype != DataType::kFloat32 && value->tensor.dtype != DataType::kFloat16) {
    return Status::Unsupported("only float32/float16 tensors are supported: " + name);
  }
  if (value->tensor.device_type != device.type || value->tensor.device_id != device.id) {
    return Status::Unsupported("tensor is assigned to another device: " + name);
  }
  return Status::OK();
}

std::vector<std::string> InvocationInputs(const KernelArtifact& artifact, std::vector<std::string> inputs) {
  for (const auto& argument : artifact.arguments) {
    const KernelArgumentSource& s = argument.source;
    if (s.layout.empty() || s.index < 0 || static_cast<std::size_t>(s.index) >= inputs.size()) continue;
    std::string& name = inputs[static_cast<std::size_t>(s.index)];
    name = LaidOutConstantName(name, s.layout);
  }
  return inputs;
}

std::string BaseArch(const std::string& full) {
  const auto colon = full.find(':');
  return colon == std::string::npos ? full : full.substr(0, colon);
}

bool ArtifactMatches(const KernelArtifact& artifact, const Node& node, const ValueLookup& lookup,
                     int capability, const std::string& arch) {
  if (capability < artifact.min_compute_capability) return false;
  if (!artifact.target_arch.empty() && artifact.target_arch != arch) return false;
  const std::string& reference_name =
      node.outputs().empty() ? node.inputs().front() : node.outputs().front();
  const ValueDesc* reference = lookup(reference_name);
  if (reference == nullptr || artifact.dtype != DataTypeName(reference->tensor.dtype)) return false;
  auto layout_ok = [&](const std::string& name) {
    const ValueDesc* v = lookup(name);
    return v != nullptr && (artifact.layout.empty() || v->tensor.layout == artifact.layout);
  };
  if (!node.inputs().empty() && !layout_ok(node.inputs().front())) return false;
  for (const auto& name : node.outputs()) {
    if (!layout_ok(name)) return false;
  }
  // An input read in another layout must be a constant (the engine re-lays
  // it out once, at constant upload): rank-4 FP32 for OHWI, rank 2 for NK and T.
  for (const auto& argument : artifact.arguments) {
    const KernelArgumentSource& s = argument.source;
    if (s.layout.empty()) continue;
    if (s.index < 0 || static_cast<std::size_t>(s.index) >= node.inputs().size()) return false;
    const ValueDesc* v = lookup(node.inputs()[static_cast<std::size_t>(s.index)]);
    if (v == nullptr || !v->is_constant) return false;
    const bool ohwi = s.layout == "OHWI" && v->tensor.shape.size() == 4 && v->tensor.dtype == DataType::kFloat32;
    const bool nk = (s.layout == "NK" || s.layout == "T") && v->tensor.shape.size() == 2;
    if (!ohwi && !nk) return false;
  }
  for (const auto& c : artifact.constraints) {
    switch (c.kind) {
      case KernelConstraintKind::kInputCountEquals:
        if (node.inputs().size() != static_cast<std::size_t>(c.expected)) return false;
        break;
      case KernelConstraintKind::kAttributeInt64Equals:
        if (GetIntAttribute(node, c.attribute_name, c.default_value) != c.expected) return false;
        break;
      case KernelConstraintKind::kTensorRankEquals: {
        const auto& names = c.tensor_is_output ? node.outputs() : node.inputs();
        if (c.tensor_index < 0 || static_cast<std::size_t>(c.tensor_index) >= names.size()) {
          return false;
        }
        const ValueDesc* v = lookup(names[static_cast<std::size_t>(c.tensor_index)]);
        if (v == nullptr || v->tensor.shape.size() != static_cast<std::size_t>(c.expected)) {
          return false;
        }
        break;
      }
      case KernelConstraintKind::kTensorDimAtMost: {
        const auto& names = c.tensor_is_output ? node.outputs() : node.inputs();
        if (c.tensor_index < 0 || static_cast<std::size_t>(c.tensor_index) >= names.size()) {
          return false;
        }
        const ValueDesc* v = lookup(names[static_cast<std::size_t>(c.tensor_index)]);
        if (v == nullptr || static_cast<std::size_t>(c.tensor_axis) >= v->tensor.shape.size() ||
            v->tensor.shape[static_cast<std::size_t>(c.tensor_axis)] > c.expected) {
          return false;
        }
        break;
      }
    }
  }
  return true;
}

Status CheckHipNode(const Node& node, const Graph& graph, const BackendOptions& options,
                    const ArtifactRepository& repository) {
  if (options.device.type != DeviceType::kHIP) {
    return Status::Unsupported(std::string(kHipBackendName) + " requires a HIP device");
  }
  CUTRITON_RETURN_IF_ERROR(RegisterBuiltinOpSchemas());
  const auto schema = OpSchemaRegistry::Global().Find(node.op_type());
  if (schema == nullptr) return Status::Unsupported("no OpSchema is registered for " + node.op_type());
  if (node.inputs().size() < schema->min_inputs || node.inputs().size() > schema->max_inputs ||
      node.outputs().size() != schema->outputs) {
    return Status::Unsupported(node.op_type() + " has an invalid input/output count");
  }
  for (const auto& name : node.inputs()) CUTRITON_RETURN_IF_ERROR(CheckTensor(graph, name, options.device));
  for (const auto& name : node.outputs()) CUTRITON_RETURN_IF_ERROR(CheckTensor(graph, name, options.device));
  if (node.op_type() == "Flatten") {
    const auto& outs = graph.outputs();
    if (std::find(outs.begin(), outs.end(), node.outputs().front()) != outs.end()) {
      return Status::Unsupported("a Flatten graph output needs an explicit copy kernel");
    }
    return Status::OK();
  }
  const auto* artifacts = repository.Find(node.op_type());
  if (artifacts == nullptr || artifacts->empty()) {
    return Status::Unsupported("no Kernel Pack entry for " + node.op_type());
  }
  int capability = 0;
  std::string arch;
  CUTRITON_RETURN_IF_ERROR(DeviceArchitecture(options.device.id, &capability, &arch));
  const ValueLookup lookup = [&](const std::string& n) { return graph.FindValue(n); };
  for (const auto& artifact : *artifacts) {
    if (ArtifactMatches(artifact, node, lookup, capability, arch)) return Status::OK();
  }
  return Status::Unsupported("no Kernel Pack variant of " + node.op_type() +
                             " matches dtype/layout/architecture/constraints");
}

class HipBackend final : public Backend {
 public:
  const char* name() const override { return kHipBackendName; }

  Status CheckSupport(const Node& node, const Graph& graph,
                      const BackendOptions& options) const override {
    std::vector<std::string> paths = options.kernel_artifact_paths;
    if (paths.empty() && !options.kernel_artifact_dir.empty()) paths.push_back(options.kernel_artifact_dir);
    ArtifactRepository repository;
    CUTRITON_RETURN_IF_ERROR(repository.Load(paths));
    return CheckHipNode(node, graph, options, repository);
  }

  Status Lower(const Node& node, const LoweringContext& context,
               std::vector<ExecutionCandidate>* candidates) const override {
    if (candidates == nullptr || context.graph == nullptr || context.options == nullptr ||
        context.artifacts == nullptr || context.catalog == nullptr) {
      return Status::InvalidArgument("HIP lowering context is incomplete");
    }
    const Graph& graph = *context.graph;
    CUTRITON_RETURN_IF_ERROR(CheckHipNode(node, graph, *context.options, *context.artifacts));
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
    const ValueDesc* out = graph.FindValue(node.outputs().front());
    if (out == nullptr) return Status::NotFound("lowered node output description is missing");
    const std::string dtype = DataTypeName(out->tensor.dtype);
    const std::string layout =
        node.inputs().empty() ? std::string() : graph.FindValue(node.inputs().front())->tensor.layout;
    const ValueLookup graph_lookup = [&](const std::string& n) { return graph.FindValue(n); };
    for (const KernelArtifact* artifact : context.catalog->Query(node.op_type(), dtype, layout, capability)) {
      if (!ArtifactMatches(*artifact, node, graph_lookup, capability, arch)) continue;
      ExecutionCandidate candidate;
      candidate.candidate_id = artifact->identity();
      candidate.is_default = artifact->is_default;
      candidate.steps.push_back(
          KernelInvocation{*artifact, InvocationInputs(*artifact, node.inputs()), node.outputs()});
      candidates->push_back(std::move(candidate));
    }
    CUTRITON_RETURN_IF_ERROR(RegisterBuiltinFusionAlternatives());
    for (const auto& alternative : FusionRegistry::Global().Find(node.op_type())) {
      ExecutionCandidate candidate;
      candidate.candidate_id = alternative.candidate_id;
      if (Decompose(node, graph, *context.artifacts, dtype, capability, arch, &candidate)) {
        candidates->push_back(std::move(candidate));
      }
    }
    return candidates->empty() ? Status::Unsupported("no compatible artifact for " + node.op_type())
                               : Status::OK();
  }

  Status CreateKernel(const Node& node, const Graph&, const BackendOptions&,
                      std::unique_ptr<OpKernel>* kernel) const override {
    if (kernel == nullptr) return Status::InvalidArgument("OpKernel output pointer is null");
    if (node.op_type() == "Flatten") {
      *kernel = std::make_unique<ViewKernel>();
      return Status::OK();
    }
    return Status::Unsupported("artifact kernels are instantiated from KernelInvocations");
  }

 private:
  // Builds the unfused step sequence of `node`. Each step uses the default
  // variant of its op whose constraints accept the step; temporaries take
  // the fused output's description and numbered workspace slots.
  static bool Decompose(const Node& node, const Graph& graph, const ArtifactRepository& repository,
                        const std::string& dtype, int capability, const std::string& arch,
                        ExecutionCandidate* candidate) {
    const std::string& out = node.outputs().front();
    std::map<std::string, std::string> temporaries;  // name -> like value
    const ValueLookup lookup = [&](const std::string& n) -> const ValueDesc* {
      const auto t = temporaries.find(n);
      return graph.FindValue(t == temporaries.end() ? n : t->second);
    };
    auto step = [&](const char* op, std::vector<std::string> inputs, std::string output) -> bool {
      Node probe(node.name(), op, inputs, {output});
      for (const auto& attribute : node.attributes()) probe.SetAttribute(attribute.first, attribute.second);
      const auto* list = repository.Find(op);
      if (list == nullptr) return false;
      for (const auto& artifact : *list) {
        if (artifact.is_default && artifact.dtype == dtype &&
            ArtifactMatches(artifact, probe, lookup, capability, arch)) {
          candidate->steps.push_back(
              KernelInvocation{artifact, InvocationInputs(artifact, std::move(inputs)), {std::move(output)}});
          return true;
        }
      }
      return false;
    };
    auto temporary = [&](const std::string& suffix, std::size_t slot) {
      const std::string name = node.name() + "::__" + suffix;
      temporaries[name] = out;
      candidate->temporaries.push_back(CandidateTemporary{name, out, slot});
      return name;
    };
    const auto& in = node.inputs();
    const std::string& op = node.op_type();
    bool ok = false;
    if (op == "FusedConvBatchNormRelu" || op == "FusedConvBatchNorm") {
      const bool relu = op == "FusedConvBatchNormRelu";
      const std::string conv = temporary("conv", 0);
      const std::string bn = relu ? temporary("bn", 1) : out;
      ok = step("Conv", {in[0], in[1]}, conv) &&
           step("BatchNormalization", {conv, in[2], in[3], in[4], in[5]}, bn) &&
           (!relu || step("Relu", {bn}, out));
    } else if (op == "FusedConvBatchNormAddRelu") {
      const std::string conv_bn = temporary("conv_bn", 0);
      ok = step("FusedConvBatchNorm", {in[0], in[1], in[2], in[3], in[4], in[5]}, conv_bn) &&
           step("AddRelu", {conv_bn, in[6]}, out);
    } else if (op == "AddRelu") {
      const std::string sum = temporary("add", 0);
      ok = step("Add", in, sum) && step("Relu", {sum}, out);
    } else if (op == "GemmGelu") {
      const std::string projected = temporary("gemm", 0);
      ok = step("Gemm", in, projected) && step("Gelu", {projected}, out);
    } else if (op == "SkipLayerNormalization") {
      const std::string sum = temporary("add", 0);
      ok = step("Add", {in[0], in[1]}, sum) && step("LayerNormalization", {sum, in[2], in[3]}, out);
    }
    if (!ok) {
      candidate->steps.clear();
      candidate->temporaries.clear();
    }
    return ok;
  }
};

Status RegisterBuiltin(std::shared_ptr<Backend> backend) {
  auto& registry = KernelRegistry::Global();
  if (registry.GetBackend(backend->name()) != nullptr) return Status::OK();
  const Status status = registry.RegisterBackend(std::move(backend));
  return status.code() == ErrorCode::kAlreadyExists ? Status::OK() : status;
}

}  // namespace

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
  const std::string key = backend->name();
  if (key.empty()) return Status::InvalidArgument("Backend name must not be empty");
  std::unique_lock<std::shared_mutex> lock(mutex_);
  if (!backends_.emplace(key, std::move(backend)).second) {
    return Status::AlreadyExists("Backend is already registered: " + key);
  }
  return Status::OK();
}

std::shared_ptr<Backend> KernelRegistry::GetBackend(const std::string& name) const {
  std::shared_lock<std::shared_mutex> lock(mutex_);
  const auto it = backends_.find(name);
  return it == backends_.end() ? nullptr : it->second;
}

std::vector<std::string> KernelRegistry::AvailableBackends() const {
  std::shared_lock<std::shared_mutex> lock(mutex_);
  std::vector<std::string> names;
  for (const auto& entry : backends_) names.push_back(entry.first);
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
  CUTRITON_RETURN_IF_ERROR(RegisterBuiltin(CreateCpuReferenceBackend()));
  CUTRITON_RETURN_IF_ERROR(RegisterBuiltin(CreateHipBackend()));
  return Status::OK();
}

Status DeviceArchitecture(int device_id, int* numeric_arch, std::string* arch_name) {
  if (numeric_arch == nullptr || arch_name == nullptr) {
    return Status::InvalidArgument("architecture outputs are null");
  }
  // CUTRITON_TARGET_ARCH (e.g. "gfx950") plans for a device that is not
  // attached: lowering and memory planning then run without a GPU.
  if (const char* forced = std::getenv("CUTRITON_TARGET_ARCH")) {
    if (std::strncmp(forced, "gfx", 3) == 0) {
      *arch_name = BaseArch(forced);
      *numeric_arch = std::atoi(forced + 3);
      return Status::OK();
    }
  }
  static std::mutex mutex;
  static std::map<int, std::pair<int, std::string>> cache;
  std::lock_guard<std::mutex> lock(mutex);
  auto it = cache.find(device_id);
  if (it == cache.end()) {
    cth_device_info info;
    if (cth_device_query(device_id, &info) != 0) {
      return Status::RuntimeError(std::string("HIP device query failed: ") + cth_last_error());
    }
    it = cache.emplace(device_id, std::make_pair(info.numeric_arch, BaseArch(info.arch_name))).first;
  }
  *numeric_arch = it->second.first;
  *arch_name = it->second.second;
  return Status::OK();
}

}  // namespace cutriton
