// Compiler. Behaviour follows reference src/compiler/compiler.cpp:22-284:
// profile validation, opt-point shapes, pass pipeline, device assignment,
// pack loading, lowering with default-candidate selection, memory planning
// (static, or per profile at the max point) plus candidate scratch slots.
#include "cutriton/compiler/compiler.h"

#include <algorithm>
#include <utility>

#include "cutriton/backend/backend.h"
#include "cutriton/ir/pass.h"
#include "cutriton/runtime/memory_planner.h"

namespace cutriton {
namespace {

enum class ProfilePoint { kMin, kOpt, kMax };

const std::vector<int64_t>& PointOf(const ShapeRange& range, ProfilePoint point) {
  return point == ProfilePoint::kMin ? range.min : point == ProfilePoint::kMax ? range.max : range.opt;
}

Status ValidateProfiles(const Graph& graph, const std::vector<ShapeProfile>& profiles) {
  for (const auto& profile : profiles) {
    if (profile.name.empty()) return Status::InvalidArgument("ShapeProfile name must not be empty");
    for (const auto& input : graph.inputs()) {
      const auto range = profile.inputs.find(input);
      if (range == profile.inputs.end()) {
        return Status::InvalidArgument("ShapeProfile is missing input: " + input);
      }
      const ShapeRange& r = range->second;
      if (r.min.empty() || r.min.size() != r.opt.size() || r.min.size() != r.max.size()) {
        return Status::ShapeError("ShapeProfile ranks differ for " + input);
      }
      for (std::size_t axis = 0; axis < r.min.size(); ++axis) {
        if (r.min[axis] <= 0 || r.min[axis] > r.opt[axis] || r.opt[axis] > r.max[axis]) {
          return Status::ShapeError("ShapeProfile min/opt/max is invalid for " + input);
        }
      }
    }
  }
  return Status::OK();
}

Status ApplyProfilePoint(Graph* graph, const ShapeProfile& profile, ProfilePoint point) {
  for (const auto& input : graph->inputs()) {
    const ValueDesc* value = graph->FindValue(input);
    if (value == nullptr) return Status::NotFound("graph input is missing: " + input);
    TensorDesc desc = value->tensor;
    desc.shape = PointOf(profile.inputs.at(input), point);
    CUTRITON_RETURN_IF_ERROR(graph->SetValueDesc(input, std::move(desc)));
  }
  return Status::OK();
}

Status ResolveProfileGraph(const Graph& optimized, const ShapeProfile& profile, ProfilePoint point,
                           Graph* out) {
  *out = optimized;
  CUTRITON_RETURN_IF_ERROR(ApplyProfilePoint(out, profile, point));
  return CreateShapeInferencePass()->Run(out);
}

std::size_t Align256(std::size_t value) { return (value + 255u) & ~std::size_t{255u}; }

// Every candidate temporary gets a slot sized by the largest "like" value
// among the temporaries sharing that slot; slots follow the planned region.
Status AddCandidateTemporaries(const Graph& graph, const std::vector<PlanOp>& ops, MemoryPlan* plan) {
  std::vector<std::size_t> slot_bytes;
  for (const auto& op : ops) {
    for (const auto& candidate : op.candidates) {
      for (const auto& temporary : candidate.temporaries) {
        const ValueDesc* like = graph.FindValue(temporary.like_value);
        if (like == nullptr || like->tensor.ByteSize() == 0) {
          return Status::ShapeError("candidate temporary has no concrete shape: " + temporary.name);
        }
        if (slot_bytes.size() <= temporary.slot) slot_bytes.resize(temporary.slot + 1, 0);
        slot_bytes[temporary.slot] = std::max(slot_bytes[temporary.slot], like->tensor.ByteSize());
      }
    }
  }
  std::vector<std::size_t> slot_offset(slot_bytes.size());
  std::size_t cursor = Align256(plan->workspace_size_bytes);
  for (std::size_t slot = 0; slot < slot_bytes.size(); ++slot) {
    slot_offset[slot] = cursor;
    cursor += Align256(slot_bytes[slot]);
  }
  for (const auto& op : ops) {
    for (const auto& candidate : op.candidates) {
      for (const auto& temporary : candidate.temporaries) {
        const bool present = std::any_of(plan->allocations.begin(), plan->allocations.end(),
                                         [&](const Allocation& a) { return a.value_name == temporary.name; });
        if (present) continue;
        const ValueDesc* like = graph.FindValue(temporary.like_value);
        plan->allocations.push_back(
            Allocation{temporary.name, like->tensor.ByteSize(), slot_offset[temporary.slot], true, ""});
      }
    }
  }
  plan->workspace_size_bytes = Align256(cursor);
  return Status::OK();
}

}  // namespace

Status Compiler::Compile(const Model& model, const CompileOptions& options, ExecutablePlan* plan) const {
  if (plan == nullptr) return Status::InvalidArgument("ExecutablePlan output pointer is null");
  const bool hip_target = options.target == kHipBackendName;
  if (options.allow_cpu_fallback && hip_target) {
    return Status::Unsupported("CPU fallback inside a HIP plan needs transfer nodes and is not implemented");
  }
  CUTRITON_RETURN_IF_ERROR(RegisterBuiltinBackends());

  ExecutablePlan result;
  result.mutable_graph() = model.graph();
  result.mutable_constants() = model.constants();
  CUTRITON_RETURN_IF_ERROR(ValidateProfiles(result.graph(), options.shape_profiles));
  if (!options.shape_profiles.empty()) {
    CUTRITON_RETURN_IF_ERROR(
        ApplyProfilePoint(&result.mutable_graph(), options.shape_profiles.front(), ProfilePoint::kOpt));
  }
  result.set_target(options.target);
  result.set_enable_cuda_graph(options.enable_cuda_graph);
  result.set_enable_profiling(options.enable_profiling);
  TuningConfig& tuning = result.mutable_tuning_config();
  tuning.mode = options.tuning_mode;
  tuning.cache_dir = options.tuning_cache_dir;
  tuning.warmup_iterations = options.tuning_warmup_iterations;
  tuning.measurement_iterations = options.tuning_measurement_iterations;
  result.set_cuda_graph_cache_capacity(options.cuda_graph_cache_capacity);
  BackendOptions& backend_options = result.mutable_backend_options();
  backend_options.device = hip_target ? Device::HIP(options.device_id) : Device::CPU();
  backend_options.kernel_artifact_dir = options.kernel_artifact_dir;
  backend_options.kernel_artifact_paths = options.kernel_artifact_paths;
  if (backend_options.kernel_artifact_paths.empty() && !options.kernel_artifact_dir.empty()) {
    backend_options.kernel_artifact_paths.push_back(options.kernel_artifact_dir);
  }
  if (tuning.cache_dir.empty() && !backend_options.kernel_artifact_paths.empty()) {
    tuning.cache_dir = backend_options.kernel_artifact_paths.front() + "/tuning";
  }
  for (const auto& entry : result.graph().values()) {
    if (entry.second.is_constant && result.constants().count(entry.first) == 0) {
      return Status::InvalidArgument("constant value has no tensor data: " + entry.first);
    }
  }

  CUTRITON_RETURN_IF_ERROR(CreateDefaultCompilePasses(options.enable_transformer_fusions,
                                                      options.enable_residual_epilogue_fusion)
                               .Run(&result.mutable_graph()));

  if (hip_target) {
    for (const auto& entry : result.graph().values()) {
      TensorDesc desc = entry.second.tensor;
      if (desc.dtype == DataType::kUnknown) continue;
      desc.device_type = DeviceType::kHIP;
      desc.device_id = options.device_id;
      CUTRITON_RETURN_IF_ERROR(result.mutable_graph().SetValueDesc(entry.first, std::move(desc)));
    }
  }

  auto backend = KernelRegistry::Global().GetBackend(options.target);
  if (backend == nullptr) return Status::NotFound("target backend is not registered: " + options.target);

  ArtifactRepository artifacts;
  const ArtifactRepository* repository = nullptr;
  if (hip_target) {
    CUTRITON_RETURN_IF_ERROR(artifacts.Load(backend_options.kernel_artifact_paths));
    repository = &artifacts;
  }
  const KernelCatalog catalog(repository);
  const LoweringContext lowering{&result.graph(), &result.backend_options(), repository,
                                 repository == nullptr ? nullptr : &catalog};
  for (const auto& node : result.graph().nodes()) {
    PlanOp op{node.id(), node.name(), node.op_type(), backend->name(), node.inputs(), node.outputs(), {}, 0};
    const Status lowered = backend->Lower(node, lowering, &op.candidates);
    if (!lowered.ok()) {
      return Status::Unsupported("node " + node.name() + " (" + node.op_type() + ") is not supported by " +
                                 options.target + ": " + lowered.message());
    }
    if (op.candidates.empty()) return Status::Internal("backend produced no candidate for " + node.name());
    for (std::size_t i = 0; i < op.candidates.size(); ++i) {
      if (op.candidates[i].is_default) {
        op.selected_candidate = i;
        break;
      }
    }
    result.mutable_ops().push_back(std::move(op));
  }

  const MemoryPlanner planner;
  if (options.shape_profiles.empty()) {
    CUTRITON_RETURN_IF_ERROR(planner.Plan(result.graph(), &result.mutable_memory_plan()));
    CUTRITON_RETURN_IF_ERROR(
        AddCandidateTemporaries(result.graph(), result.ops(), &result.mutable_memory_plan()));
  } else {
    for (const auto& profile : options.shape_profiles) {
      ProfilePlan pp;
      pp.profile = profile;
      CUTRITON_RETURN_IF_ERROR(ResolveProfileGraph(result.graph(), profile, ProfilePoint::kMin, &pp.min_graph));
      CUTRITON_RETURN_IF_ERROR(ResolveProfileGraph(result.graph(), profile, ProfilePoint::kOpt, &pp.opt_graph));
      CUTRITON_RETURN_IF_ERROR(ResolveProfileGraph(result.graph(), profile, ProfilePoint::kMax, &pp.max_graph));
      CUTRITON_RETURN_IF_ERROR(planner.Plan(pp.max_graph, &pp.max_memory_plan));
      CUTRITON_RETURN_IF_ERROR(AddCandidateTemporaries(pp.max_graph, result.ops(), &pp.max_memory_plan));
      result.mutable_profile_plans().push_back(std::move(pp));
    }
    result.mutable_memory_plan() = result.profile_plans().front().max_memory_plan;
  }
  *plan = std::move(result);
  return Status::OK();
}

Status BuildEngine(const Model& model, const CompileOptions& options, std::unique_ptr<Engine>* engine) {
  if (engine == nullptr) return Status::InvalidArgument("Engine output pointer is null");
  ExecutablePlan plan;
  CUTRITON_RETURN_IF_ERROR(Compiler{}.Compile(model, options, &plan));
  *engine = std::make_unique<Engine>(std::move(plan));
  return Status::OK();
}

}  // namespace cutriton
