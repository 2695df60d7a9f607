// Engine and ExecutionContext over HIP.
//
// An Engine holds the compiled plan and, shared by all its contexts, the
// device copies of the constants (uploaded once, with re-laid-out copies made
// on the GPU) and the cache of loaded code objects. An ExecutionContext is one
// run session: its bindings, its shapes (static, or a point of a shape
// profile), the tensors of the current run (constants, bindings, and the
// intermediates placed in its workspace), the selected candidate and kernels
// of every op, and the HIP state (stream, per-op events, captured graphs).
//
// Preparation is lazy and layered: a binding change invalidates the tensor
// table; a shape change also the kernels and tuning choices (and the
// bindings, whose shapes no longer fit); a profile change also the workspace
// and the captured graphs. A run prepares what is stale: tensors, then tuning
// choices, then kernels; then it replays (or captures) the hipGraph keyed by
// profile, workspace, bound buffers, shapes and candidates - the key the
// reference's graph cache uses (src/runtime/engine.cpp:1003-1024), so its
// least-recently-used eviction behaves alike.
//
// The tuner (TuneOnMiss / ForceRetune) first runs the current selection of
// every op once, so that intermediate inputs hold values derived from the
// bound inputs, then times every candidate of each op in back-to-back batches
// of about 0.2 ms, rejects candidates whose output strays from the first
// candidate's by more than the numeric gate, and records the fastest.
#include "cutriton/runtime/engine.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <mutex>
#include <optional>
#include <sstream>

#include "cutriton/core/buffer.h"
#include "cutriton/ir/pass.h"
#include "cutriton_hip_runtime.h"
#include "runtime/relayout.h"
#include "runtime/static_scratch.h"
#include "runtime/tuning_store.h"

namespace cutriton {
namespace {

Status RuntimeStatus(int code, const char* operation) {
  if (code == 0) return Status::OK();
  return Status::RuntimeError(std::string(operation) + ": " + cth_last_error());
}

// binary16 -> binary32, exact for every input including subnormals.
float WidenHalf(std::uint16_t bits) {
  const int exponent = (bits >> 10) & 0x1f;
  const int fraction = bits & 0x3ff;
  float magnitude;
  if (exponent == 0) {
    magnitude = std::ldexp(static_cast<float>(fraction), -24);
  } else if (exponent == 0x1f) {
    magnitude = fraction == 0 ? std::numeric_limits<float>::infinity() : std::numeric_limits<float>::quiet_NaN();
  } else {
    magnitude = std::ldexp(static_cast<float>(fraction | 0x400), exponent - 25);
  }
  return (bits & 0x8000) ? -magnitude : magnitude;
}

// The tensor's elements on the host as floats (the tuner's numeric gate).
Status ReadBackAsFloats(const Tensor& tensor, std::vector<float>* out) {
  const auto count = static_cast<std::size_t>(tensor.desc().NumElements());
  switch (tensor.desc().dtype) {
    case DataType::kFloat32:
      out->resize(count);
      return tensor.buffer()->CopyToHost(out->data(), tensor.desc().ByteSize(), tensor.byte_offset());
    case DataType::kFloat16: {
      std::vector<std::uint16_t> bits(count);
      CUTRITON_RETURN_IF_ERROR(tensor.buffer()->CopyToHost(bits.data(), tensor.desc().ByteSize(), tensor.byte_offset()));
      out->resize(count);
      std::transform(bits.begin(), bits.end(), out->begin(), WidenHalf);
      return Status::OK();
    }
    default:
      return Status::Unsupported("tuning comparison supports float32/float16 only");
  }
}

// A caller's tensor for graph value `name`, whose plan description is `want`.
Status CheckBinding(const std::string& name, const TensorDesc& want, const Tensor& tensor) {
  CUTRITON_RETURN_IF_ERROR(tensor.desc().Validate());
  if (!tensor.defined() || tensor.buffer()->empty()) return Status::InvalidArgument("tensor Buffer is not defined: " + name);
  const TensorDesc& have = tensor.desc();
  const bool same = have.shape == want.shape && have.dtype == want.dtype && have.layout == want.layout &&
                    have.device_type == want.device_type && have.device_id == want.device_id;
  if (!same) return Status::InvalidArgument("tensor description does not match the plan: " + name);
  const Buffer& buffer = *tensor.buffer();
  if (buffer.device_type() != want.device_type || buffer.device_id() != want.device_id) {
    return Status::InvalidArgument("tensor Buffer is on another device: " + name);
  }
  if (tensor.byte_offset() > buffer.size_bytes() || want.ByteSize() > buffer.size_bytes() - tensor.byte_offset()) {
    return Status::InvalidArgument("tensor Buffer is too small: " + name);
  }
  return Status::OK();
}

struct EventPair {
  cth_event start{nullptr};
  cth_event end{nullptr};
  bool timed{false};
};

struct GraphEntry {
  std::string key;
  cth_graph exec{nullptr};
  std::uint64_t last_used{0};
};

struct HipExecutionState {
  int device{0};
  cth_stream owned_stream{nullptr};
  cth_stream active_stream{nullptr};
  std::vector<GraphEntry> graphs;
  std::uint64_t clock{0};
  std::vector<EventPair> events;
};

void DestroyGraphs(HipExecutionState* state) {
  for (auto& entry : state->graphs) cth_graph_destroy(entry.exec);
  state->graphs.clear();
}

void DestroyHipState(HipExecutionState* state) {
  if (state == nullptr) return;
  cth_set_device(state->device);
  DestroyGraphs(state);
  for (auto& pair : state->events) {
    cth_event_destroy(pair.start);
    cth_event_destroy(pair.end);
  }
  cth_stream_destroy(state->owned_stream);
  delete state;
}

Status CreateHipState(int device, std::size_t op_count, bool profiling, HipExecutionState** out) {
  auto* state = new HipExecutionState();
  state->device = device;
  Status status = RuntimeStatus(cth_stream_create(&state->owned_stream, device), "hipStreamCreate");
  state->events.resize(op_count);
  for (std::size_t i = 0; status.ok() && profiling && i < op_count; ++i) {
    status = RuntimeStatus(cth_event_create(&state->events[i].start), "hipEventCreate");
    if (status.ok()) status = RuntimeStatus(cth_event_create(&state->events[i].end), "hipEventCreate");
  }
  if (!status.ok()) {
    DestroyHipState(state);
    return status;
  }
  *out = state;
  return Status::OK();
}

std::optional<std::size_t> CandidateIndex(const PlanOp& op, const std::string& id) {
  for (std::size_t i = 0; i < op.candidates.size(); ++i) {
    if (op.candidates[i].candidate_id == id) return i;
  }
  return std::nullopt;
}

}  // namespace

// CUTRITON_INIT_LOG=1 prints the wall time of each one-time stage of a
// context's first run: constant upload and re-layout, tuning, kernel
// loading, graph capture.
class StageTimer {
 public:
  explicit StageTimer(const char* stage) : stage_(stage), start_(std::chrono::steady_clock::now()) {}
  ~StageTimer() {
    static const bool enabled = std::getenv("CUTRITON_INIT_LOG") != nullptr;
    if (!enabled) return;
    const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - start_).count();
    if (ms >= 0.05) std::fprintf(stderr, "[cutriton init] %s: %.2f ms\n", stage_, ms);
  }

 private:
  const char* stage_;
  std::chrono::steady_clock::time_point start_;
};

class EngineState {
 public:
  explicit EngineState(ExecutablePlan p) : plan(std::move(p)) {}

  Status InitializeConstants() {
    std::call_once(constants_once_, [&] {
      constants_status_ = UploadConstants();
      constants_ready_ = constants_status_.ok();
    });
    return constants_status_;
  }
  bool ConstantsReady() const { return constants_ready_; }

  Status InitializeModuleCache() {
    if (plan.backend_options().device.type != DeviceType::kHIP) return Status::OK();
    std::call_once(module_once_, [&] {
      module_status_ = CreateHipModuleCache(plan.backend_options().device.id, &module_cache);
    });
    return module_status_;
  }

  ExecutablePlan plan;
  std::unordered_map<std::string, Tensor> device_constants;
  std::shared_ptr<HipModuleCache> module_cache;

 private:
  Status UploadConstants() {
    const Device& device = plan.backend_options().device;
    {
      StageTimer timer("constant upload");
      for (const auto& entry : plan.constants()) {
        const ValueDesc* value = plan.graph().FindValue(entry.first);
        if (value == nullptr || !value->is_constant) {
          return Status::Internal("plan constant is missing from the graph: " + entry.first);
        }
        if (device.type == DeviceType::kCPU) {
          device_constants.emplace(entry.first, entry.second);
          continue;
        }
        std::shared_ptr<Buffer> buffer;
        CUTRITON_RETURN_IF_ERROR(Buffer::AllocateHip(value->tensor.ByteSize(), device.id, &buffer));
        const Tensor& host = entry.second;
        const auto* bytes = static_cast<const std::uint8_t*>(host.buffer()->data()) + host.byte_offset();
        CUTRITON_RETURN_IF_ERROR(buffer->CopyFromHost(bytes, value->tensor.ByteSize()));
        device_constants.emplace(entry.first, Tensor(value->tensor, std::move(buffer)));
      }
    }
    return UploadLaidOutConstants();
  }

  // Copies of constants in the layout a selected kernel reads them in (the
  // KernelInvocation input "<constant>#<layout>"), made once per engine on
  // the device from the uploaded original. The copy keeps the logical
  // shape; only the element order changes.
  Status UploadLaidOutConstants() {
    const Device& device = plan.backend_options().device;
    if (device.type != DeviceType::kHIP) return Status::OK();
    StageTimer timer("constant re-layout");
    bool launched = false;
    for (const PlanOp& op : plan.ops()) {
      for (const ExecutionCandidate& candidate : op.candidates) {
        for (const PlanStep& step : candidate.steps) {
          const auto* inv = std::get_if<KernelInvocation>(&step);
          if (inv == nullptr) continue;
          for (const auto& argument : inv->artifact.arguments) {
            const KernelArgumentSource& src = argument.source;
            if (src.layout.empty() || src.index < 0 || static_cast<std::size_t>(src.index) >= inv->inputs.size()) {
              continue;
            }
            const std::string& name = inv->inputs[static_cast<std::size_t>(src.index)];
            if (device_constants.count(name) != 0) continue;
            const std::string base = name.substr(0, name.rfind('#'));
            const auto original = device_constants.find(base);
            if (original == device_constants.end() || !IsInputLayout(src.layout)) {
              return Status::Internal("no constant to lay out as " + name);
            }
            const TensorDesc& desc = original->second.desc();
            TensorDesc laid_out = desc;
            laid_out.layout = src.layout;
            if (src.layout == "OHWI") {
              if (desc.shape.size() != 4 || desc.dtype != DataType::kFloat32) {
                return Status::InvalidArgument("OHWI needs a rank-4 float32 constant: " + base);
              }
              if (desc.shape[2] * desc.shape[3] == 1) {  // [K][C][1][1]: both orders are the same bytes
                device_constants.emplace(name, Tensor(laid_out, original->second.buffer(),
                                                      original->second.byte_offset()));
                continue;
              }
            }
            std::shared_ptr<Buffer> buffer;
            CUTRITON_RETURN_IF_ERROR(Buffer::AllocateHip(desc.ByteSize(), device.id, &buffer));
            const auto* in = static_cast<const std::uint8_t*>(original->second.buffer()->data()) +
                             original->second.byte_offset();
            CUTRITON_RETURN_IF_ERROR(RelayoutOnDevice(src.layout, desc, in, buffer->data(), device.id));
            launched = true;
            device_constants.emplace(name, Tensor(laid_out, std::move(buffer)));
          }
        }
      }
    }
    if (launched) CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_device_synchronize(device.id), "hipDeviceSynchronize"));
    return Status::OK();
  }

  std::once_flag constants_once_;
  Status constants_status_;
  bool constants_ready_{false};
  std::once_flag module_once_;
  Status module_status_;
};

Engine::Engine(ExecutablePlan plan) : state_(std::make_shared<EngineState>(std::move(plan))) {}

const ExecutablePlan& Engine::plan() const { return state_->plan; }

std::unique_ptr<ExecutionContext> Engine::CreateExecutionContext() const {
  return std::make_unique<ExecutionContext>(state_);
}

ExecutionContext::ExecutionContext(std::shared_ptr<EngineState> state) : state_(std::move(state)) {
  // A plan with exactly one profile starts on it, at its opt shapes.
  if (state_ == nullptr || state_->plan.profile_plans().size() != 1) return;
  const ProfilePlan& only = state_->plan.profile_plans().front();
  selected_profile_ = 0;
  for (const auto& [input, range] : only.profile.inputs) input_shapes_[input] = range.opt;
  resolved_graph_ = only.opt_graph;
  shapes_resolved_ = true;
}

ExecutionContext::~ExecutionContext() {
  (void)Synchronize();
  DestroyHipState(static_cast<HipExecutionState*>(hip_state_));
}

// Captured graphs survive binding and shape changes: their keys name the
// bound buffers, shapes and candidates, so a later run with the same
// bindings replays its graph again (least recently used evicted first).
void ExecutionContext::Invalidate(Stale what) {
  tensors_prepared_ = false;
  if (what == Stale::kBindings) return;
  bound_.clear();
  kernels_.clear();
  kernels_prepared_ = false;
  tuning_prepared_ = false;
  if (what == Stale::kShapes) return;
  workspace_.reset();
  InvalidateHipGraph();
}

const Graph& ExecutionContext::ActiveGraph() const { return shapes_resolved_ ? resolved_graph_ : state_->plan.graph(); }

const MemoryPlan& ExecutionContext::ActiveMemoryPlan() const {
  if (selected_profile_ < 0) return state_->plan.memory_plan();
  return state_->plan.profile_plans().at(static_cast<std::size_t>(selected_profile_)).max_memory_plan;
}

Status ExecutionContext::BindInput(const std::string& name, Tensor tensor) {
  if (state_ == nullptr) return Status::InvalidArgument("ExecutionContext has no EngineState");
  if (run_pending_) return Status::RuntimeError("cannot bind a tensor while a run is pending");
  if (!state_->plan.profile_plans().empty() && !shapes_resolved_) {
    return Status::RuntimeError("ResolveShapes must be called before binding");
  }
  const auto& inputs = ActiveGraph().inputs();
  const ValueDesc* value = ActiveGraph().FindValue(name);
  if (std::find(inputs.begin(), inputs.end(), name) == inputs.end()) return Status::NotFound("name is not a graph input: " + name);
  if (value == nullptr) return Status::NotFound("graph input description is missing: " + name);
  CUTRITON_RETURN_IF_ERROR(CheckBinding(name, value->tensor, tensor));
  bound_[name] = std::move(tensor);
  Invalidate(Stale::kBindings);
  return Status::OK();
}

Status ExecutionContext::BindOutput(const std::string& name, Tensor tensor) {
  if (state_ == nullptr) return Status::InvalidArgument("ExecutionContext has no EngineState");
  if (run_pending_) return Status::RuntimeError("cannot bind a tensor while a run is pending");
  if (!state_->plan.profile_plans().empty() && !shapes_resolved_) {
    return Status::RuntimeError("ResolveShapes must be called before binding");
  }
  const auto& outputs = ActiveGraph().outputs();
  const ValueDesc* value = ActiveGraph().FindValue(name);
  if (std::find(outputs.begin(), outputs.end(), name) == outputs.end()) return Status::NotFound("name is not a graph output: " + name);
  if (value == nullptr) return Status::NotFound("graph output description is missing: " + name);
  CUTRITON_RETURN_IF_ERROR(CheckBinding(name, value->tensor, tensor));
  bound_[name] = std::move(tensor);
  Invalidate(Stale::kBindings);
  return Status::OK();
}

Status ExecutionContext::SelectShapeProfile(const std::string& name) {
  if (run_pending_) return Status::RuntimeError("cannot change the profile while a run is pending");
  const auto& profiles = state_->plan.profile_plans();
  const auto found = std::find_if(profiles.begin(), profiles.end(), [&](const ProfilePlan& p) { return p.profile.name == name; });
  if (found == profiles.end()) return Status::NotFound("ShapeProfile is not defined: " + name);
  selected_profile_ = static_cast<int>(found - profiles.begin());
  input_shapes_.clear();
  for (const auto& [input, range] : found->profile.inputs) input_shapes_[input] = range.opt;
  resolved_graph_ = found->opt_graph;
  shapes_resolved_ = true;
  Invalidate(Stale::kProfile);
  return Status::OK();
}

Status ExecutionContext::SetInputShape(const std::string& name, std::vector<int64_t> shape) {
  if (run_pending_) return Status::RuntimeError("cannot change a shape while a run is pending");
  if (selected_profile_ < 0) return Status::RuntimeError("select a ShapeProfile before setting shapes");
  const ShapeProfile& profile = state_->plan.profile_plans().at(static_cast<std::size_t>(selected_profile_)).profile;
  const auto range = profile.inputs.find(name);
  if (range == profile.inputs.end()) return Status::NotFound("name is not a profiled graph input: " + name);
  const ShapeRange& r = range->second;
  if (shape.size() != r.min.size()) return Status::ShapeError("input rank does not match the profile: " + name);
  for (std::size_t axis = 0; axis < shape.size(); ++axis) {
    if (shape[axis] < r.min[axis] || shape[axis] > r.max[axis]) {
      return Status::ShapeError("input shape is outside the profile range: " + name);
    }
  }
  input_shapes_[name] = std::move(shape);
  shapes_resolved_ = false;
  Invalidate(Stale::kShapes);
  return Status::OK();
}

Status ExecutionContext::ResolveShapes() {
  if (selected_profile_ < 0) return Status::RuntimeError("select a ShapeProfile before resolving shapes");
  Graph graph = state_->plan.profile_plans().at(static_cast<std::size_t>(selected_profile_)).opt_graph;
  for (const auto& input : graph.inputs()) {
    const auto shape = input_shapes_.find(input);
    if (shape == input_shapes_.end()) return Status::InvalidArgument("input shape is not set: " + input);
    TensorDesc desc = graph.FindValue(input)->tensor;
    desc.shape = shape->second;
    CUTRITON_RETURN_IF_ERROR(graph.SetValueDesc(input, std::move(desc)));
  }
  CUTRITON_RETURN_IF_ERROR(CreateShapeInferencePass()->Run(&graph));
  resolved_graph_ = std::move(graph);
  shapes_resolved_ = true;
  return Status::OK();
}

const TensorDesc* ExecutionContext::GetResolvedTensorDesc(const std::string& name) const {
  if (!shapes_resolved_) return nullptr;
  const ValueDesc* value = resolved_graph_.FindValue(name);
  return value == nullptr ? nullptr : &value->tensor;
}

std::size_t ExecutionContext::cached_cuda_graph_count() const {
  const auto* hip = static_cast<const HipExecutionState*>(hip_state_);
  return hip == nullptr ? 0 : hip->graphs.size();
}

std::size_t ExecutionContext::loaded_cuda_module_count() const {
  return state_ == nullptr ? 0 : LoadedModuleCount(state_->module_cache);
}

// The largest runtime scratch any candidate declares (tuning may run each).
std::size_t ExecutionContext::RuntimeScratchNeed() const {
  std::size_t need = 0;
  for (const auto& op : state_->plan.ops()) {
    for (const auto& candidate : op.candidates) {
      for (const auto& step : candidate.steps) {
        if (const auto* inv = std::get_if<KernelInvocation>(&step)) {
          need = std::max(need, static_cast<std::size_t>(std::max<int64_t>(0, inv->artifact.runtime_scratch_bytes)));
        }
      }
    }
  }
  return need;
}

// The run's tensor table: device constants, the caller's bindings, and every
// planned intermediate (values, Flatten views, candidate temporaries) at its
// workspace offset.
Status ExecutionContext::PrepareTensors(bool may_allocate) {
  if (tensors_prepared_) return Status::OK();
  if (state_ == nullptr) return Status::InvalidArgument("ExecutionContext has no EngineState");
  if (!may_allocate && !state_->ConstantsReady()) {
    return Status::RuntimeError("constants are not on the device yet: run the context once with RunAsync first");
  }
  CUTRITON_RETURN_IF_ERROR(state_->InitializeConstants());
  const Device& device = state_->plan.backend_options().device;
  const MemoryPlan& memory = ActiveMemoryPlan();
  const bool workspace_short = workspace_ == nullptr || workspace_->size_bytes() < memory.workspace_size_bytes;
  if (memory.workspace_size_bytes != 0 && workspace_short) {
    if (!may_allocate) {
      return Status::RuntimeError("the context has no workspace of " + std::to_string(memory.workspace_size_bytes) +
                                  " bytes: run it once with RunAsync first");
    }
    if (device.type == DeviceType::kHIP) {
      CUTRITON_RETURN_IF_ERROR(Buffer::AllocateHip(memory.workspace_size_bytes, device.id, &workspace_));
    } else {
      workspace_ = Buffer::AllocateHost(memory.workspace_size_bytes);
    }
  }

  std::unordered_map<std::string, Tensor> table = state_->device_constants;
  for (const auto& [name, tensor] : bound_) table[name] = tensor;
  // Temporaries are described like the value their candidate names.
  std::unordered_map<std::string, std::string> temporary_like;
  for (const auto& op : state_->plan.ops()) {
    for (const auto& candidate : op.candidates) {
      for (const auto& temporary : candidate.temporaries) temporary_like.emplace(temporary.name, temporary.like_value);
    }
  }
  const Graph& graph = ActiveGraph();
  for (const Allocation& allocation : memory.allocations) {
    const ValueDesc* value = graph.FindValue(allocation.value_name);
    if (value == nullptr) {
      const auto like = temporary_like.find(allocation.value_name);
      value = like == temporary_like.end() ? nullptr : graph.FindValue(like->second);
      if (value == nullptr) return Status::Internal("allocation references an unknown value: " + allocation.value_name);
    }
    if (!allocation.alias_of.empty()) {
      const auto source = table.find(allocation.alias_of);
      if (source == table.end()) return Status::Internal("alias source tensor is missing: " + allocation.alias_of);
      if (value->tensor.ByteSize() != source->second.desc().ByteSize()) {
        return Status::ShapeError("alias changes the byte size of " + allocation.value_name);
      }
      table[allocation.value_name] = Tensor(value->tensor, source->second.buffer(), source->second.byte_offset());
      continue;
    }
    const std::size_t bytes = value->tensor.ByteSize();
    if (workspace_ == nullptr || allocation.offset > workspace_->size_bytes() ||
        bytes > workspace_->size_bytes() - allocation.offset) {
      return Status::Internal("allocation exceeds the workspace: " + allocation.value_name);
    }
    table[allocation.value_name] = Tensor(value->tensor, workspace_, allocation.offset);
  }
  tensors_ = std::move(table);

  const std::size_t scratch = RuntimeScratchNeed();
  const bool scratch_short = runtime_scratch_ == nullptr || runtime_scratch_->size_bytes() < scratch;
  if (may_allocate && scratch > 0 && device.type == DeviceType::kHIP && scratch_short) {
    CUTRITON_RETURN_IF_ERROR(Buffer::AllocateHip(scratch, device.id, &runtime_scratch_));
    CUTRITON_RETURN_IF_ERROR(
        RuntimeStatus(cth_memset(runtime_scratch_->data(), 0, runtime_scratch_->size_bytes(), device.id), "hipMemset"));
    InvalidateHipGraph();
  }
  tensors_prepared_ = true;
  return Status::OK();
}

Status ExecutionContext::PrepareKernels(bool may_load) {
  if (kernels_prepared_) return Status::OK();
  if (state_ == nullptr) return Status::InvalidArgument("ExecutionContext has no EngineState");
  CUTRITON_RETURN_IF_ERROR(RegisterBuiltinBackends());
  CUTRITON_RETURN_IF_ERROR(state_->InitializeModuleCache());
  const auto& ops = state_->plan.ops();
  if (selected_candidates_.size() != ops.size()) return Status::Internal("tuning selections are not prepared");
  const BackendOptions& options = state_->plan.backend_options();
  std::vector<std::vector<std::unique_ptr<OpKernel>>> kernels;
  for (std::size_t i = 0; i < ops.size(); ++i) {
    const PlanOp& op = ops[i];
    auto backend = KernelRegistry::Global().GetBackend(op.backend_name);
    if (backend == nullptr) return Status::NotFound("backend is not registered: " + op.backend_name);
    const Node& node = ActiveGraph().nodes().at(static_cast<std::size_t>(op.node_id));
    if (selected_candidates_[i] >= op.candidates.size()) return Status::Internal("selected candidate is out of range");
    const ExecutionCandidate& chosen = op.candidates[selected_candidates_[i]];
    std::vector<std::unique_ptr<OpKernel>> group;
    for (const auto& step : chosen.steps) {
      std::unique_ptr<OpKernel> kernel;
      if (const auto* inv = std::get_if<KernelInvocation>(&step)) {
        if (!may_load && !CodeObjectLoaded(state_->module_cache, inv->artifact)) {
          return Status::RuntimeError("code object of " + inv->artifact.identity() +
                                      " is not loaded: run the context once with RunAsync first");
        }
        CUTRITON_RETURN_IF_ERROR(CreateInvocationKernel(*inv, options.device.id, state_->module_cache, &kernel));
      } else {
        CUTRITON_RETURN_IF_ERROR(backend->CreateKernel(node, ActiveGraph(), options, &kernel));
      }
      if (kernel == nullptr) return Status::Internal("backend returned a null OpKernel");
      group.push_back(std::move(kernel));
    }
    if (group.empty()) {  // a legacy candidate: the backend's own kernel
      std::unique_ptr<OpKernel> kernel;
      CUTRITON_RETURN_IF_ERROR(backend->CreateKernel(node, ActiveGraph(), options, &kernel));
      if (kernel == nullptr) return Status::Internal("backend returned a null OpKernel");
      group.push_back(std::move(kernel));
    }
    kernels.push_back(std::move(group));
  }
  kernels_ = std::move(kernels);
  kernels_prepared_ = true;
  return Status::OK();
}

Status ExecutionContext::PrepareTuning(bool may_time) {
  if (tuning_prepared_) return Status::OK();
  const auto& ops = state_->plan.ops();
  selected_candidates_.clear();
  for (const auto& op : ops) selected_candidates_.push_back(op.selected_candidate);
  const TuningConfig& config = state_->plan.tuning_config();
  const Device& device = state_->plan.backend_options().device;
  if (device.type != DeviceType::kHIP || config.mode == TuningMode::kDisabled) {
    tuning_prepared_ = true;
    return Status::OK();
  }
  CUTRITON_RETURN_IF_ERROR(state_->InitializeModuleCache());
  const Graph& graph = ActiveGraph();
  const TuningStore store(config.cache_dir);

  // Resolve from the store first; collect the ops that still need timing.
  // Under UseCache a shape that was never tuned takes the profile opt
  // point's choice.
  std::vector<std::size_t> to_tune;
  std::vector<std::string> keys(ops.size());
  for (std::size_t i = 0; i < ops.size(); ++i) {
    const PlanOp& op = ops[i];
    if (op.candidates.size() < 2) continue;
    const Node& node = graph.nodes().at(static_cast<std::size_t>(op.node_id));
    keys[i] = TuningDecisionKey(op, node, graph, device.id);
    if (config.mode != TuningMode::kForceRetune) {
      std::optional<std::string> recorded = store.Lookup(keys[i]);
      if (!recorded && config.mode == TuningMode::kUseCache && selected_profile_ >= 0) {
        const Graph& opt = state_->plan.profile_plans().at(static_cast<std::size_t>(selected_profile_)).opt_graph;
        recorded = store.Lookup(TuningDecisionKey(op, opt.nodes().at(static_cast<std::size_t>(op.node_id)), opt, device.id));
      }
      if (recorded) {
        if (const auto index = CandidateIndex(op, *recorded)) {
          selected_candidates_[i] = *index;
          continue;
        }
      }
    }
    if (config.mode != TuningMode::kUseCache) to_tune.push_back(i);
  }
  if (to_tune.empty()) {
    tuning_prepared_ = true;
    return Status::OK();
  }
  if (!may_time) {
    return Status::RuntimeError(std::to_string(to_tune.size()) + " ops need tuning (" + ops[to_tune.front()].node_name +
                                " first): run the context once with RunAsync first");
  }

  cth_stream stream = nullptr;
  cth_event start = nullptr;
  cth_event end = nullptr;
  CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_stream_create(&stream, device.id), "hipStreamCreate"));
  struct Cleanup {
    cth_stream* s;
    cth_event* a;
    cth_event* b;
    ~Cleanup() {
      cth_event_destroy(*a);
      cth_event_destroy(*b);
      cth_stream_destroy(*s);
    }
  } cleanup{&stream, &start, &end};
  CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_event_create(&start), "hipEventCreate"));
  CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_event_create(&end), "hipEventCreate"));
  void* scratch = runtime_scratch_ ? runtime_scratch_->data() : nullptr;
  const std::size_t scratch_bytes = runtime_scratch_ ? runtime_scratch_->size_bytes() : 0;

  auto build_kernels = [&](const ExecutionCandidate& candidate, std::vector<std::unique_ptr<OpKernel>>* out) -> Status {
    out->clear();
    for (const auto& step : candidate.steps) {
      const auto* inv = std::get_if<KernelInvocation>(&step);
      if (inv == nullptr) continue;
      std::unique_ptr<OpKernel> kernel;
      CUTRITON_RETURN_IF_ERROR(CreateInvocationKernel(*inv, device.id, state_->module_cache, &kernel));
      out->push_back(std::move(kernel));
    }
    return Status::OK();
  };

  // One pass of the current selection, so that every intermediate tensor an
  // op reads holds data derived from the bound inputs.
  for (std::size_t i = 0; i < ops.size(); ++i) {
    const Node& node = graph.nodes().at(static_cast<std::size_t>(ops[i].node_id));
    std::vector<std::unique_ptr<OpKernel>> kernels;
    CUTRITON_RETURN_IF_ERROR(build_kernels(ops[i].candidates[selected_candidates_[i]], &kernels));
    KernelContext context{&node, &tensors_, stream, nullptr, scratch, scratch_bytes};
    for (auto& kernel : kernels) CUTRITON_RETURN_IF_ERROR(kernel->Compute(&context));
  }
  CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_stream_synchronize(stream), "hipStreamSynchronize"));

  // CUTRITON_TUNING_LOG=1 prints every candidate's median and every
  // numeric-gate rejection to stderr.
  const bool tuning_log = std::getenv("CUTRITON_TUNING_LOG") != nullptr;
  for (const std::size_t op_index : to_tune) {
    const PlanOp& op = ops[op_index];
    const Node& node = graph.nodes().at(static_cast<std::size_t>(op.node_id));
    KernelContext context{&node, &tensors_, stream, nullptr, scratch, scratch_bytes};
    double best_ms = std::numeric_limits<double>::infinity();
    std::size_t best = op.selected_candidate;
    std::vector<float> reference;
    float reference_rms = 0.0f;
    for (std::size_t c = 0; c < op.candidates.size(); ++c) {
      std::vector<std::unique_ptr<OpKernel>> kernels;
      CUTRITON_RETURN_IF_ERROR(build_kernels(op.candidates[c], &kernels));
      if (kernels.empty()) continue;
      for (int w = 0; w < config.warmup_iterations; ++w) {
        for (auto& kernel : kernels) CUTRITON_RETURN_IF_ERROR(kernel->Compute(&context));
      }
      CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_stream_synchronize(stream), "hipStreamSynchronize"));
      const Tensor& output = tensors_.at(op.outputs.front());
      std::vector<float> produced;
      CUTRITON_RETURN_IF_ERROR(ReadBackAsFloats(output, &produced));
      if (reference.empty()) {
        reference = std::move(produced);
        double sum_sq = 0.0;
        for (const float v : reference) sum_sq += static_cast<double>(v) * v;
        reference_rms = reference.empty() ? 0.0f : static_cast<float>(std::sqrt(sum_sq / reference.size()));
      } else {
        // Candidates differ only in summation order, so an element may
        // differ by a relative amount of the output's scale, not of its own
        // value: the absolute floor is rel * max(1, rms of the output).
        const float rel = output.desc().dtype == DataType::kFloat16 ? 1e-2f : 1e-4f;
        const float floor = rel * std::max(1.0f, reference_rms);
        bool agrees = true;
        std::size_t e = 0;
        for (; e < produced.size() && agrees; ++e) {
          const float tolerance = floor + rel * std::fabs(reference[e]);
          agrees = std::isfinite(produced[e]) && std::fabs(produced[e] - reference[e]) <= tolerance;
        }
        if (!agrees) {
          if (tuning_log) {
            std::fprintf(stderr, "[cutriton tuning] %s: %s rejected (element %zu: %g vs %g)\n",
                         op.node_name.c_str(), op.candidates[c].candidate_id.c_str(), e - 1,
                         static_cast<double>(produced[e - 1]), static_cast<double>(reference[e - 1]));
          }
          continue;
        }
      }
      // A sample is `launches` back-to-back runs of the candidate between
      // one event pair, enough to last about kSampleMs, so that launch
      // overhead and the idle gap after each synchronisation weigh the
      // same for every candidate; the sample's time per run enters the
      // median. Candidates are safe to rerun: graph replay relies on it.
      constexpr double kSampleMs = 0.2;
      auto time_runs = [&](int launches, float* ms) -> Status {
        CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_event_record(start, stream), "hipEventRecord"));
        for (int r = 0; r < launches; ++r) {
          for (auto& kernel : kernels) CUTRITON_RETURN_IF_ERROR(kernel->Compute(&context));
        }
        CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_event_record(end, stream), "hipEventRecord"));
        CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_event_synchronize(end), "hipEventSynchronize"));
        CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_event_elapsed_ms(ms, start, end), "hipEventElapsedTime"));
        *ms /= static_cast<float>(launches);
        return Status::OK();
      };
      float probe_ms = 0.0f;
      CUTRITON_RETURN_IF_ERROR(time_runs(1, &probe_ms));
      const int launches = static_cast<int>(std::clamp(std::ceil(kSampleMs / std::max(probe_ms, 1e-4f)), 1.0, 64.0));
      std::vector<float> samples;
      for (int it = 0; it < std::max(1, config.measurement_iterations); ++it) {
        float ms = 0.0f;
        CUTRITON_RETURN_IF_ERROR(time_runs(launches, &ms));
        samples.push_back(ms);
      }
      std::sort(samples.begin(), samples.end());
      const double median = samples[samples.size() / 2];
      if (tuning_log) {
        std::fprintf(stderr, "[cutriton tuning] %s: %s %.4f ms\n", op.node_name.c_str(),
                     op.candidates[c].candidate_id.c_str(), median);
      }
      if (median < best_ms) {
        best_ms = median;
        best = c;
      }
    }
    if (!std::isfinite(best_ms)) return Status::RuntimeError("no numerically valid tuning candidate for " + op.node_name);
    selected_candidates_[op_index] = best;
    // Leave the op's output as the chosen candidate computes it.
    std::vector<std::unique_ptr<OpKernel>> kernels;
    CUTRITON_RETURN_IF_ERROR(build_kernels(op.candidates[best], &kernels));
    for (auto& kernel : kernels) CUTRITON_RETURN_IF_ERROR(kernel->Compute(&context));
    CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_stream_synchronize(stream), "hipStreamSynchronize"));
    CUTRITON_RETURN_IF_ERROR(store.Record(keys[op_index], op.candidates[best].candidate_id, best_ms));
  }
  tuning_prepared_ = true;
  return Status::OK();
}

Status ExecutionContext::ValidateBindings() const {
  const Graph& graph = ActiveGraph();
  for (const auto* names : {&graph.inputs(), &graph.outputs()}) {
    for (const auto& name : *names) {
      if (bound_.count(name) == 0) return Status::InvalidArgument("graph value is not bound: " + name);
    }
  }
  for (const auto& node : graph.nodes()) {
    for (const auto* names : {&node.inputs(), &node.outputs()}) {
      for (const auto& name : *names) {
        if (tensors_.count(name) == 0) return Status::InvalidArgument("node tensor is missing: " + name);
      }
    }
  }
  return Status::OK();
}

Status ExecutionContext::Run() {
  CUTRITON_RETURN_IF_ERROR(RunAsync(nullptr));
  return Synchronize();
}

Status ExecutionContext::EnqueueOps(void* stream, bool capture, void* scratch, std::size_t scratch_bytes) {
  auto* hip = static_cast<HipExecutionState*>(hip_state_);
  const bool profiling = state_->plan.enable_profiling() && hip != nullptr;
  for (std::size_t i = 0; i < kernels_.size(); ++i) {
    const PlanOp& op = state_->plan.ops()[i];
    const Node& node = ActiveGraph().nodes().at(static_cast<std::size_t>(op.node_id));
    // Events inside a capture are graph nodes placed by CaptureGraph.
    const bool timed = profiling && node.op_type() != "Flatten";
    if (hip != nullptr) hip->events[i].timed = timed;
    if (timed && !capture) CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_event_record(hip->events[i].start, stream), "hipEventRecord"));
    KernelContext context{&node, &tensors_, stream, nullptr, scratch, scratch_bytes};
    for (auto& kernel : kernels_[i]) CUTRITON_RETURN_IF_ERROR(kernel->Compute(&context));
    if (timed && !capture) CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_event_record(hip->events[i].end, stream), "hipEventRecord"));
  }
  return Status::OK();
}

// Records the op sequence into an executable hipGraph. Without profiling the
// whole sequence is one stream capture. With profiling every op is captured
// on its own and chained as a child graph between two hipEvent record nodes,
// so each replay times every op (HIP refuses external event records inside a
// stream capture, the mechanism of reference src/runtime/engine.cpp:971-980).
Status ExecutionContext::CaptureGraph(void* stream, void** exec) {
  auto* hip = static_cast<HipExecutionState*>(hip_state_);
  *exec = nullptr;
  void* scratch = runtime_scratch_ ? runtime_scratch_->data() : nullptr;
  const std::size_t scratch_bytes = runtime_scratch_ ? runtime_scratch_->size_bytes() : 0;
  if (!state_->plan.enable_profiling()) {
    CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_stream_begin_capture(stream), "hipStreamBeginCapture"));
    const Status enqueued = EnqueueOps(stream, true, scratch, scratch_bytes);
    cth_graph graph = nullptr;
    const Status ended = RuntimeStatus(cth_stream_end_capture(stream, &graph), "hipStreamEndCapture");
    if (!enqueued.ok()) {
      cth_graph_destroy(graph);
      return enqueued;
    }
    CUTRITON_RETURN_IF_ERROR(ended);
    *exec = graph;
    return Status::OK();
  }
  cth_graph_template parent = nullptr;
  CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_graph_template_create(&parent), "hipGraphCreate"));
  struct ParentGuard {
    cth_graph_template graph;
    ~ParentGuard() { cth_graph_template_destroy(graph); }
  } guard{parent};
  cth_graph_node previous = nullptr;
  for (std::size_t i = 0; i < kernels_.size(); ++i) {
    const PlanOp& op = state_->plan.ops()[i];
    const Node& node = ActiveGraph().nodes().at(static_cast<std::size_t>(op.node_id));
    EventPair& events = hip->events[i];
    events.timed = node.op_type() != "Flatten";
    if (!events.timed) continue;  // a view launches nothing
    CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_graph_add_event_record(parent, previous, events.start, &previous),
                                           "hipGraphAddEventRecordNode"));
    CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_stream_begin_capture(stream), "hipStreamBeginCapture"));
    KernelContext context{&node, &tensors_, stream, nullptr, scratch, scratch_bytes};
    Status launched = Status::OK();
    for (auto& kernel : kernels_[i]) {
      launched = kernel->Compute(&context);
      if (!launched.ok()) break;
    }
    cth_graph_template child = nullptr;
    const Status ended = RuntimeStatus(cth_stream_end_capture_template(stream, &child), "hipStreamEndCapture");
    if (launched.ok() && ended.ok()) {
      launched = RuntimeStatus(cth_graph_add_child(parent, previous, child, &previous), "hipGraphAddChildGraphNode");
    }
    cth_graph_template_destroy(child);
    CUTRITON_RETURN_IF_ERROR(launched);
    CUTRITON_RETURN_IF_ERROR(ended);
    CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_graph_add_event_record(parent, previous, events.end, &previous),
                                           "hipGraphAddEventRecordNode"));
  }
  cth_graph graph = nullptr;
  CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_graph_instantiate(parent, &graph), "hipGraphInstantiate"));
  *exec = graph;
  return Status::OK();
}

Status ExecutionContext::RunAsync(void* stream) {
  if (run_pending_) return Status::RuntimeError("a run is already pending");
  {
    StageTimer timer("tensors");
    CUTRITON_RETURN_IF_ERROR(PrepareTensors(true));
  }
  CUTRITON_RETURN_IF_ERROR(ValidateBindings());
  {
    StageTimer timer("tuning");
    CUTRITON_RETURN_IF_ERROR(PrepareTuning(true));
  }
  {
    StageTimer timer("kernel loading");
    CUTRITON_RETURN_IF_ERROR(PrepareKernels(true));
  }
  void* scratch = runtime_scratch_ ? runtime_scratch_->data() : nullptr;
  const std::size_t scratch_bytes = runtime_scratch_ ? runtime_scratch_->size_bytes() : 0;

  const Device& device = state_->plan.backend_options().device;
  if (device.type != DeviceType::kHIP) {
    profiler_.Clear();
    for (std::size_t i = 0; i < kernels_.size(); ++i) {
      const PlanOp& op = state_->plan.ops()[i];
      const Node& node = ActiveGraph().nodes().at(static_cast<std::size_t>(op.node_id));
      KernelContext context{&node, &tensors_, stream, state_->plan.enable_profiling() ? &profiler_ : nullptr,
                            scratch, scratch_bytes};
      for (auto& kernel : kernels_[i]) CUTRITON_RETURN_IF_ERROR(kernel->Compute(&context));
    }
    run_pending_ = true;
    return Status::OK();
  }

  auto* hip = static_cast<HipExecutionState*>(hip_state_);
  if (hip == nullptr) {
    CUTRITON_RETURN_IF_ERROR(CreateHipState(device.id, kernels_.size(), state_->plan.enable_profiling(), &hip));
    hip_state_ = hip;
  }
  CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_set_device(device.id), "hipSetDevice"));
  hip->active_stream = stream == nullptr ? hip->owned_stream : stream;

  if (!state_->plan.enable_cuda_graph()) {
    CUTRITON_RETURN_IF_ERROR(EnqueueOps(hip->active_stream, false, scratch, scratch_bytes));
    run_pending_ = true;
    return Status::OK();
  }

  std::ostringstream key;
  key << "profile:" << selected_profile_ << "|workspace:" << (workspace_ == nullptr ? nullptr : workspace_->data());
  for (const auto& name : ActiveGraph().inputs()) {
    const Tensor& t = tensors_.at(name);
    key << "|in:" << name << ':' << t.buffer()->data() << ':' << t.byte_offset();
    for (const int64_t d : t.desc().shape) key << ':' << d;
  }
  for (const auto& name : ActiveGraph().outputs()) {
    const Tensor& t = tensors_.at(name);
    key << "|out:" << name << ':' << t.buffer()->data() << ':' << t.byte_offset();
  }
  for (std::size_t i = 0; i < selected_candidates_.size(); ++i) {
    key << "|candidate:" << state_->plan.ops()[i].candidates[selected_candidates_[i]].candidate_id;
  }
  const std::string graph_key = key.str();
  auto entry = std::find_if(hip->graphs.begin(), hip->graphs.end(), [&](const GraphEntry& e) { return e.key == graph_key; });
  if (entry == hip->graphs.end()) {
    GraphEntry created;
    created.key = graph_key;
    StageTimer timer("graph capture");
    CUTRITON_RETURN_IF_ERROR(CaptureGraph(hip->active_stream, &created.exec));
    const std::size_t capacity = std::max<std::size_t>(1, state_->plan.cuda_graph_cache_capacity());
    if (hip->graphs.size() >= capacity) {
      auto oldest = std::min_element(hip->graphs.begin(), hip->graphs.end(),
                                     [](const GraphEntry& a, const GraphEntry& b) { return a.last_used < b.last_used; });
      cth_graph_destroy(oldest->exec);
      hip->graphs.erase(oldest);
    }
    hip->graphs.push_back(std::move(created));
    entry = std::prev(hip->graphs.end());
  }
  entry->last_used = ++hip->clock;
  CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_graph_launch(entry->exec, hip->active_stream), "hipGraphLaunch"));
  run_pending_ = true;
  return Status::OK();
}

// The allocation-free run: the same preparation with every allocating step
// refused, then the ops enqueued straight onto the caller's stream with the
// static scratch as their runtime scratch.
Status ExecutionContext::RunAsyncWithoutAllocation(void* stream) {
  if (run_pending_) return Status::RuntimeError("a run is already pending");
  if (stream == nullptr) return Status::InvalidArgument("the allocation-free run needs the caller's stream");
  if (state_ == nullptr) return Status::InvalidArgument("ExecutionContext has no EngineState");
  const Device& device = state_->plan.backend_options().device;
  if (device.type != DeviceType::kHIP) return Status::Unsupported("the allocation-free run needs a HIP plan");
  const std::size_t need = RuntimeScratchNeed();
  if (need > kStaticScratchBytes) {
    return Status::InvalidArgument("kernels of this plan declare " + std::to_string(need) +
                                     " bytes of runtime scratch; the static scratch holds " +
                                     std::to_string(kStaticScratchBytes));
  }
  CUTRITON_RETURN_IF_ERROR(PrepareTensors(false));
  CUTRITON_RETURN_IF_ERROR(ValidateBindings());
  CUTRITON_RETURN_IF_ERROR(PrepareTuning(false));
  CUTRITON_RETURN_IF_ERROR(PrepareKernels(false));
  void* scratch = nullptr;
  if (StaticScratchAddress(device.id, &scratch) != 0) {
    return Status::RuntimeError(std::string("static scratch: ") + StaticScratchError());
  }
  CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_set_device(device.id), "hipSetDevice"));
  // The array keeps the last call's contents: the split-K tile counters must
  // start at zero.
  if (need > 0 && ClearStaticScratchCounters(scratch, stream) != 0) {
    return Status::RuntimeError(std::string("static scratch: ") + StaticScratchError());
  }
  if (auto* hip = static_cast<HipExecutionState*>(hip_state_)) {
    for (auto& pair : hip->events) pair.timed = false;  // no per-op events on this path
  }
  for (std::size_t i = 0; i < kernels_.size(); ++i) {
    const PlanOp& op = state_->plan.ops()[i];
    const Node& node = ActiveGraph().nodes().at(static_cast<std::size_t>(op.node_id));
    KernelContext context{&node, &tensors_, stream, nullptr, scratch, kStaticScratchBytes};
    for (auto& kernel : kernels_[i]) CUTRITON_RETURN_IF_ERROR(kernel->Compute(&context));
  }
  unmanaged_stream_ = stream;
  run_pending_ = true;
  return Status::OK();
}

Status ExecutionContext::TimeOp(std::size_t op_index, int iterations, void* stream, double* ms_per_launch) {
  if (ms_per_launch == nullptr || iterations < 1) return Status::InvalidArgument("TimeOp needs iterations >= 1");
  if (run_pending_) return Status::RuntimeError("TimeOp while a run is pending");
  auto* hip = static_cast<HipExecutionState*>(hip_state_);
  if (!kernels_prepared_ || hip == nullptr) return Status::RuntimeError("TimeOp needs a completed HIP run first");
  if (op_index >= kernels_.size()) return Status::InvalidArgument("TimeOp: op index out of range");
  *ms_per_launch = 0.0;
  const PlanOp& op = state_->plan.ops()[op_index];
  const Node& node = ActiveGraph().nodes().at(static_cast<std::size_t>(op.node_id));
  // Flatten is a view: no launch, not timed (as in the profiled graph).
  if (kernels_[op_index].empty() || node.op_type() == "Flatten") return Status::OK();
  void* s = stream == nullptr ? hip->owned_stream : stream;
  KernelContext context{&node, &tensors_, s, nullptr, runtime_scratch_ ? runtime_scratch_->data() : nullptr,
                        runtime_scratch_ ? runtime_scratch_->size_bytes() : 0};
  cth_event start = nullptr;
  cth_event end = nullptr;
  CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_set_device(state_->plan.backend_options().device.id), "hipSetDevice"));
  CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_event_create(&start), "hipEventCreate"));
  Status status = RuntimeStatus(cth_event_create(&end), "hipEventCreate");
  for (auto& kernel : kernels_[op_index]) {
    if (status.ok()) status = kernel->Compute(&context);
  }
  if (status.ok()) status = RuntimeStatus(cth_event_record(start, s), "hipEventRecord");
  for (int it = 0; it < iterations && status.ok(); ++it) {
    for (auto& kernel : kernels_[op_index]) {
      if (status.ok()) status = kernel->Compute(&context);
    }
  }
  if (status.ok()) status = RuntimeStatus(cth_event_record(end, s), "hipEventRecord");
  if (status.ok()) status = RuntimeStatus(cth_event_synchronize(end), "hipEventSynchronize");
  float ms = 0.0f;
  if (status.ok()) status = RuntimeStatus(cth_event_elapsed_ms(&ms, start, end), "hipEventElapsedTime");
  cth_event_destroy(start);
  if (end != nullptr) cth_event_destroy(end);
  CUTRITON_RETURN_IF_ERROR(status);
  *ms_per_launch = static_cast<double>(ms) / iterations;
  return Status::OK();
}

Status ExecutionContext::Synchronize() {
  if (!run_pending_) return Status::OK();
  run_pending_ = false;
  if (state_->plan.backend_options().device.type != DeviceType::kHIP) return Status::OK();
  profiler_.Clear();
  if (unmanaged_stream_ != nullptr) {  // an allocation-free run: no events were recorded
    void* stream = unmanaged_stream_;
    unmanaged_stream_ = nullptr;
    return RuntimeStatus(cth_stream_synchronize(stream), "hipStreamSynchronize");
  }
  auto* hip = static_cast<HipExecutionState*>(hip_state_);
  CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_stream_synchronize(hip->active_stream), "hipStreamSynchronize"));
  if (state_->plan.enable_profiling()) {
    for (std::size_t i = 0; i < state_->plan.ops().size(); ++i) {
      const PlanOp& op = state_->plan.ops()[i];
      float ms = 0.0f;
      if (hip->events[i].timed) {
        CUTRITON_RETURN_IF_ERROR(
            RuntimeStatus(cth_event_elapsed_ms(&ms, hip->events[i].start, hip->events[i].end), "hipEventElapsedTime"));
      }
      profiler_.Record(op.node_name, op.backend_name, static_cast<double>(ms));
    }
  }
  return Status::OK();
}

void ExecutionContext::InvalidateHipGraph() {
  if (auto* hip = static_cast<HipExecutionState*>(hip_state_)) {
    cth_set_device(hip->device);
    DestroyGraphs(hip);
  }
}

}  // namespace cutriton
