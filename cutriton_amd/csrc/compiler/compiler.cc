// Model -> ExecutablePlan.
//
// The compile is a short pipeline over one working plan:
//   1. check the request: shape profiles well formed, every constant value
//      backed by data;
//   2. settle the plan's options (target device, graph capture, tuning);
//   3. optimise the graph at the first profile's opt shapes (the pass
//      pipeline) and place its values on the target device;
//   4. lower every node to its execution candidates, default selected;
//   5. resolve each profile at its min, opt and max shapes and drop the
//      candidates whose kernels cannot take the tensors of some point
//      (tensor_bytes_le); a node left without a candidate fails the compile;
//   6. plan the workspace: for the static graph, or per profile at its max
//      shapes, with each candidate's temporaries live during its op only.
// Observable behaviour follows the reference's compiler
// (src/compiler/compiler.cpp): the same error kinds for malformed profiles,
// missing constant data, unregistered targets and unsupported nodes, the
// default tuning-cache folder "<first pack path>/tuning", and profile plans
// holding min/opt/max graphs with a max-shape workspace.
#include "cutriton/compiler/compiler.h"

#include <algorithm>
#include <map>
#include <utility>

#include "cutriton/backend/backend.h"
#include "cutriton/ir/pass.h"
#include "cutriton/runtime/memory_planner.h"

namespace cutriton {
namespace {

// The three shapes a profile names for every graph input.
enum class ProfileCorner { kMin, kOpt, kMax };

const std::vector<int64_t>& CornerShape(const ShapeRange& range, ProfileCorner corner) {
  switch (corner) {
    case ProfileCorner::kMin:
      return range.min;
    case ProfileCorner::kMax:
      return range.max;
    case ProfileCorner::kOpt:
      break;
  }
  return range.opt;
}

// A profile must name every graph input with three shapes of one rank,
// min <= opt <= max on every axis and every dimension positive.
Status CheckProfile(const Graph& graph, const ShapeProfile& profile) {
  if (profile.name.empty()) return Status::InvalidArgument("ShapeProfile name must not be empty");
  for (const auto& input : graph.inputs()) {
    const auto range = profile.inputs.find(input);
    if (range == profile.inputs.end()) {
      return Status::InvalidArgument("ShapeProfile " + profile.name + " is missing input: " + input);
    }
    const ShapeRange& r = range->second;
    const std::size_t rank = r.opt.size();
    if (rank == 0 || r.min.size() != rank || r.max.size() != rank) {
      return Status::ShapeError("ShapeProfile ranks differ for " + input);
    }
    for (std::size_t axis = 0; axis < rank; ++axis) {
      const bool ordered = 0 < r.min[axis] && r.min[axis] <= r.opt[axis] && r.opt[axis] <= r.max[axis];
      if (!ordered) return Status::ShapeError("ShapeProfile min/opt/max is invalid for " + input);
    }
  }
  return Status::OK();
}

// Gives every graph input the profile's shape at `corner`.
Status SetInputsAt(Graph* graph, const ShapeProfile& profile, ProfileCorner corner) {
  for (const auto& input : graph->inputs()) {
    const ValueDesc* value = graph->FindValue(input);
    if (value == nullptr) return Status::NotFound("graph input is missing: " + input);
    TensorDesc desc = value->tensor;
    desc.shape = CornerShape(profile.inputs.at(input), corner);
    CUTRITON_RETURN_IF_ERROR(graph->SetValueDesc(input, std::move(desc)));
  }
  return Status::OK();
}

// The optimised graph with every value's shape re-inferred at `corner`.
Status GraphAt(const Graph& optimized, const ShapeProfile& profile, ProfileCorner corner, Graph* out) {
  Graph graph = optimized;
  CUTRITON_RETURN_IF_ERROR(SetInputsAt(&graph, profile, corner));
  CUTRITON_RETURN_IF_ERROR(CreateShapeInferencePass()->Run(&graph));
  *out = std::move(graph);
  return Status::OK();
}

// One request per (op, temporary slot): the candidates of an op never run
// together, so the temporaries of one slot share a block sized for the
// largest of them.
Status TemporaryRequests(const Graph& graph, const std::vector<PlanOp>& ops,
                         std::vector<WorkspaceRequest>* requests) {
  requests->clear();
  for (std::size_t step = 0; step < ops.size(); ++step) {
    std::map<std::size_t, WorkspaceRequest> by_slot;
    for (const auto& candidate : ops[step].candidates) {
      for (const auto& temporary : candidate.temporaries) {
        const ValueDesc* like = graph.FindValue(temporary.like_value);
        if (like == nullptr || like->tensor.ByteSize() == 0) {
          return Status::ShapeError("candidate temporary has no concrete shape: " + temporary.name);
        }
        WorkspaceRequest& request = by_slot[temporary.slot];
        request.step = static_cast<int>(step);
        request.size_bytes = std::max(request.size_bytes, like->tensor.ByteSize());
        if (std::find(request.names.begin(), request.names.end(), temporary.name) == request.names.end()) {
          request.names.push_back(temporary.name);
        }
      }
    }
    for (auto& entry : by_slot) requests->push_back(std::move(entry.second));
  }
  return Status::OK();
}

Status PlanWorkspace(const Graph& graph, const std::vector<PlanOp>& ops, MemoryPlan* plan) {
  std::vector<WorkspaceRequest> temporaries;
  CUTRITON_RETURN_IF_ERROR(TemporaryRequests(graph, ops, &temporaries));
  return MemoryPlanner{}.Plan(graph, temporaries, plan);
}

class CompilePipeline {
 public:
  CompilePipeline(const Model& model, const CompileOptions& options) : model_(model), options_(options) {}

  Status Run(ExecutablePlan* out) {
    CUTRITON_RETURN_IF_ERROR(CheckRequest());
    CUTRITON_RETURN_IF_ERROR(RegisterBuiltinBackends());
    backend_ = KernelRegistry::Global().GetBackend(options_.target);
    ConfigurePlan();
    CUTRITON_RETURN_IF_ERROR(OptimizeGraph());
    if (backend_ == nullptr) return Status::NotFound("target backend is not registered: " + options_.target);
    CUTRITON_RETURN_IF_ERROR(LowerNodes());
    CUTRITON_RETURN_IF_ERROR(ResolveProfiles());
    CUTRITON_RETURN_IF_ERROR(PlanMemory());
    *out = std::move(plan_);
    return Status::OK();
  }

 private:
  bool OnHip() const { return options_.target == kHipBackendName; }

  Status CheckRequest() const {
    if (OnHip() && options_.allow_cpu_fallback) {
      return Status::Unsupported("CPU fallback inside a HIP plan needs transfer nodes and is not implemented");
    }
    for (const auto& profile : options_.shape_profiles) CUTRITON_RETURN_IF_ERROR(CheckProfile(model_.graph(), profile));
    for (const auto& [name, value] : model_.graph().values()) {
      if (value.is_constant && model_.constants().count(name) == 0) {
        return Status::InvalidArgument("constant value has no tensor data: " + name);
      }
    }
    return Status::OK();
  }

  void ConfigurePlan() {
    plan_.mutable_graph() = model_.graph();
    plan_.mutable_constants() = model_.constants();
    plan_.set_target(options_.target);
    plan_.set_enable_cuda_graph(options_.enable_cuda_graph);
    plan_.set_enable_profiling(options_.enable_profiling);
    plan_.set_cuda_graph_cache_capacity(options_.cuda_graph_cache_capacity);

    BackendOptions& backend = plan_.mutable_backend_options();
    backend.device = OnHip() ? Device::HIP(options_.device_id) : Device::CPU();
    backend.kernel_artifact_dir = options_.kernel_artifact_dir;
    backend.kernel_artifact_paths = options_.kernel_artifact_paths;
    if (backend.kernel_artifact_paths.empty() && !backend.kernel_artifact_dir.empty()) {
      backend.kernel_artifact_paths.push_back(backend.kernel_artifact_dir);
    }

    TuningConfig& tuning = plan_.mutable_tuning_config();
    tuning.mode = options_.tuning_mode;
    tuning.warmup_iterations = options_.tuning_warmup_iterations;
    tuning.measurement_iterations = options_.tuning_measurement_iterations;
    tuning.cache_dir = options_.tuning_cache_dir;
    if (tuning.cache_dir.empty() && !backend.kernel_artifact_paths.empty()) {
      tuning.cache_dir = backend.kernel_artifact_paths.front() + "/tuning";
    }
  }

  Status OptimizeGraph() {
    Graph& graph = plan_.mutable_graph();
    if (!options_.shape_profiles.empty()) {
      CUTRITON_RETURN_IF_ERROR(SetInputsAt(&graph, options_.shape_profiles.front(), ProfileCorner::kOpt));
    }
    CUTRITON_RETURN_IF_ERROR(
        CreateDefaultCompilePasses(options_.enable_transformer_fusions, options_.enable_residual_epilogue_fusion)
            .Run(&graph));
    if (!OnHip()) return Status::OK();
    // Typed values move to the device; untyped ones (never produced) stay put.
    std::vector<std::pair<std::string, TensorDesc>> placed;
    for (const auto& [name, value] : graph.values()) {
      if (value.tensor.dtype == DataType::kUnknown) continue;
      TensorDesc desc = value.tensor;
      desc.device_type = DeviceType::kHIP;
      desc.device_id = options_.device_id;
      placed.emplace_back(name, std::move(desc));
    }
    for (auto& [name, desc] : placed) CUTRITON_RETURN_IF_ERROR(graph.SetValueDesc(name, std::move(desc)));
    return Status::OK();
  }

  Status LowerNodes() {
    const ArtifactRepository* repository = nullptr;
    if (OnHip()) {
      CUTRITON_RETURN_IF_ERROR(artifacts_.Load(plan_.backend_options().kernel_artifact_paths));
      repository = &artifacts_;
    }
    const KernelCatalog catalog(repository);
    const LoweringContext context{&plan_.graph(), &plan_.backend_options(), repository,
                                  repository != nullptr ? &catalog : nullptr};
    for (const auto& node : plan_.graph().nodes()) {
      PlanOp op{node.id(), node.name(), node.op_type(), backend_->name(), node.inputs(), node.outputs(), {}, 0};
      const Status lowered = backend_->Lower(node, context, &op.candidates);
      if (!lowered.ok()) {
        return Status::Unsupported("node " + node.name() + " (" + node.op_type() + ") is not supported by " +
                                   options_.target + ": " + lowered.message());
      }
      if (op.candidates.empty()) return Status::Internal("backend produced no candidate for " + node.name());
      SelectDefault(&op);
      plan_.mutable_ops().push_back(std::move(op));
    }
    return Status::OK();
  }

  // The first candidate flagged default, else the first.
  static void SelectDefault(PlanOp* op) {
    const auto flagged = std::find_if(op->candidates.begin(), op->candidates.end(),
                                      [](const ExecutionCandidate& c) { return c.is_default; });
    op->selected_candidate = flagged == op->candidates.end() ? 0 : static_cast<std::size_t>(flagged - op->candidates.begin());
  }

  // Size limits of the kernels hold at every corner of every profile, not
  // only at the opt shapes the nodes were lowered at.
  Status ResolveProfiles() {
    std::vector<const Graph*> corners;
    if (options_.shape_profiles.empty()) {
      corners.push_back(&plan_.graph());
    } else {
      for (const auto& profile : options_.shape_profiles) {
        ProfilePlan pp;
        pp.profile = profile;
        CUTRITON_RETURN_IF_ERROR(GraphAt(plan_.graph(), profile, ProfileCorner::kMin, &pp.min_graph));
        CUTRITON_RETURN_IF_ERROR(GraphAt(plan_.graph(), profile, ProfileCorner::kOpt, &pp.opt_graph));
        CUTRITON_RETURN_IF_ERROR(GraphAt(plan_.graph(), profile, ProfileCorner::kMax, &pp.max_graph));
        plan_.mutable_profile_plans().push_back(std::move(pp));
      }
      for (const auto& pp : plan_.profile_plans()) {
        corners.insert(corners.end(), {&pp.min_graph, &pp.opt_graph, &pp.max_graph});
      }
    }
    for (PlanOp& op : plan_.mutable_ops()) {
      const std::string selected = op.candidates[op.selected_candidate].candidate_id;
      std::string refusal;
      std::vector<ExecutionCandidate> kept;
      for (auto& candidate : op.candidates) {
        Status fits = Status::OK();
        for (const Graph* graph : corners) {
          fits = CheckCandidateShapes(candidate, *graph);
          if (!fits.ok()) break;
        }
        if (fits.ok()) {
          kept.push_back(std::move(candidate));
        } else if (refusal.empty()) {
          refusal = fits.message();
        }
      }
      if (kept.empty()) {
        return Status::Unsupported("node " + op.node_name + " (" + op.op_type + ") has no kernel for the shapes of " +
                                   "its profile: " + refusal);
      }
      op.candidates = std::move(kept);
      const auto still = std::find_if(op.candidates.begin(), op.candidates.end(),
                                      [&](const ExecutionCandidate& c) { return c.candidate_id == selected; });
      if (still != op.candidates.end()) {
        op.selected_candidate = static_cast<std::size_t>(still - op.candidates.begin());
      } else {
        SelectDefault(&op);
      }
    }
    return Status::OK();
  }

  Status PlanMemory() {
    if (plan_.profile_plans().empty()) {
      return PlanWorkspace(plan_.graph(), plan_.ops(), &plan_.mutable_memory_plan());
    }
    for (ProfilePlan& pp : plan_.mutable_profile_plans()) {
      CUTRITON_RETURN_IF_ERROR(PlanWorkspace(pp.max_graph, plan_.ops(), &pp.max_memory_plan));
    }
    plan_.mutable_memory_plan() = plan_.profile_plans().front().max_memory_plan;
    return Status::OK();
  }

  const Model& model_;
  const CompileOptions& options_;
  ExecutablePlan plan_;
  ArtifactRepository artifacts_;
  std::shared_ptr<Backend> backend_;
};

}  // namespace

Status Compiler::Compile(const Model& model, const CompileOptions& options, ExecutablePlan* plan) const {
  if (plan == nullptr) return Status::InvalidArgument("ExecutablePlan output pointer is null");
  return CompilePipeline(model, options).Run(plan);
}

Status BuildEngine(const Model& model, const CompileOptions& options, std::unique_ptr<Engine>* engine) {
  if (engine == nullptr) return Status::InvalidArgument("Engine output pointer is null");
  ExecutablePlan plan;
  CUTRITON_RETURN_IF_ERROR(Compiler{}.Compile(model, options, &plan));
  *engine = std::make_unique<Engine>(std::move(plan));
  return Status::OK();
}

}  // namespace cutriton
