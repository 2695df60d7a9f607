// Engine and ExecutionContext over HIP. Behaviour follows reference
// src/runtime/engine.cpp:
//   * EngineState: constants uploaded once, module cache created once
//     (340-395);
//   * binding validation (79-110, 404-454), profiles and shape resolution
//     (462-576), tensor placement in the planned workspace (593-668), kernel
//     creation (670-723);
//   * tuner: FNV-1a-64 key over op, tensors, attributes, candidates, artifact
//     identity, device and driver (215-295); cache files written atomically
//     (297-335); warm-up, numerical check against candidate 0 (1e-4 FP32,
//     1e-2 FP16, relative + absolute), median of timed runs (725-891);
//   * RunAsync: per-op event pairs (event record nodes around per-op child
//     graphs when capturing), graph
//     capture keyed by profile, workspace, bound tensors and selected
//     candidates, LRU eviction of the least recently used graph (925-1079);
//   * Synchronize: stream sync, then per-op durations into the Profiler
//     (1081-1119).
// Two deliberate differences: before timing candidates, the tuner runs the
// default candidate of every op once, so that intermediate inputs hold the
// values of the current inputs rather than uninitialised workspace memory;
// and each timed sample is a back-to-back batch of runs (about 0.2 ms),
// not one run between synchronisations, whose launch and idle overheads
// are as large as a short kernel.
#include "cutriton/runtime/engine.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <iomanip>
#include <limits>
#include <mutex>
#include <optional>
#include <sstream>
#include <type_traits>
#include <variant>

#include "cutriton/core/buffer.h"
#include "cutriton/ir/pass.h"
#include "cutriton_hip_runtime.h"
#include "runtime/relayout.h"

namespace cutriton {
namespace {

Status RuntimeStatus(int code, const char* operation) {
  if (code == 0) return Status::OK();
  return Status::RuntimeError(std::string(operation) + ": " + cth_last_error());
}

bool Contains(const std::vector<std::string>& names, const std::string& name) {
  return std::find(names.begin(), names.end(), name) != names.end();
}

// IEEE binary16 -> binary32 (exact).
float HalfToFloat(std::uint16_t h) {
  const std::uint32_t sign = static_cast<std::uint32_t>(h & 0x8000u) << 16;
  const std::uint32_t exponent = (h >> 10) & 0x1fu;
  std::uint32_t mantissa = h & 0x3ffu;
  std::uint32_t bits;
  if (exponent == 0x1fu) {
    bits = sign | 0x7f800000u | (mantissa << 13);
  } else if (exponent != 0) {
    bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
  } else if (mantissa == 0) {
    bits = sign;
  } else {
    int shift = 0;
    while ((mantissa & 0x400u) == 0) {
      mantissa <<= 1;
      ++shift;
    }
    bits = sign | (static_cast<std::uint32_t>(113 - shift) << 23) | ((mantissa & 0x3ffu) << 13);
  }
  float value;
  std::memcpy(&value, &bits, sizeof(value));
  return value;
}

Status TensorToHostFloats(const Tensor& tensor, std::vector<float>* out) {
  const auto count = static_cast<std::size_t>(tensor.desc().NumElements());
  out->assign(count, 0.0f);
  if (tensor.desc().dtype == DataType::kFloat32) {
    return tensor.buffer()->CopyToHost(out->data(), tensor.desc().ByteSize(), tensor.byte_offset());
  }
  if (tensor.desc().dtype == DataType::kFloat16) {
    std::vector<std::uint16_t> halves(count);
    CUTRITON_RETURN_IF_ERROR(
        tensor.buffer()->CopyToHost(halves.data(), tensor.desc().ByteSize(), tensor.byte_offset()));
    for (std::size_t i = 0; i < count; ++i) (*out)[i] = HalfToFloat(halves[i]);
    return Status::OK();
  }
  return Status::Unsupported("tuning comparison supports float32/float16 only");
}

Status ValidateBoundTensor(const std::string& name, const TensorDesc& expected, const Tensor& tensor) {
  CUTRITON_RETURN_IF_ERROR(tensor.desc().Validate());
  if (!tensor.defined() || tensor.buffer()->empty()) {
    return Status::InvalidArgument("tensor Buffer is not defined: " + name);
  }
  const TensorDesc& actual = tensor.desc();
  if (actual.shape != expected.shape || actual.dtype != expected.dtype ||
      actual.layout != expected.layout || actual.device_type != expected.device_type ||
      actual.device_id != expected.device_id) {
    return Status::InvalidArgument("tensor description does not match the plan: " + name);
  }
  if (tensor.buffer()->device_type() != expected.device_type ||
      tensor.buffer()->device_id() != expected.device_id) {
    return Status::InvalidArgument("tensor Buffer is on another device: " + name);
  }
  const std::size_t capacity = tensor.buffer()->size_bytes();
  if (tensor.byte_offset() > capacity || expected.ByteSize() > capacity - tensor.byte_offset()) {
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

std::string TuningKey(const PlanOp& op, const Node& node, const Graph& graph, int device_id) {
  std::ostringstream m;
  m << op.op_type << '|' << device_id;
  auto tensors = [&](const char* role, const std::vector<std::string>& names) {
    for (const auto& name : names) {
      m << '|' << role << ':' << name;
      if (const ValueDesc* v = graph.FindValue(name)) {
        m << ':' << static_cast<int>(v->tensor.dtype) << ':' << v->tensor.layout;
        for (const int64_t d : v->tensor.shape) m << ':' << d;
      }
    }
  };
  tensors("input", op.inputs);
  tensors("output", op.outputs);
  std::vector<std::string> keys;
  for (const auto& attribute : node.attributes()) keys.push_back(attribute.first);
  std::sort(keys.begin(), keys.end());
  for (const auto& key : keys) {
    const Attribute& a = node.attributes().at(key);
    m << "|attribute:" << key << ':' << a.index();
    std::visit(
        [&](const auto& value) {
          using T = std::decay_t<decltype(value)>;
          if constexpr (std::is_same_v<T, std::vector<int64_t>> || std::is_same_v<T, std::vector<double>>) {
            for (const auto item : value) m << ':' << item;
          } else {
            m << ':' << value;
          }
        },
        a);
  }
  for (const auto& candidate : op.candidates) {
    m << '|' << candidate.candidate_id;
    for (const auto& step : candidate.steps) {
      if (const auto* inv = std::get_if<KernelInvocation>(&step)) {
        const KernelArtifact& a = inv->artifact;
        m << "|pack:" << a.pack_name << ':' << a.pack_version << "|kernel:" << a.kernel_id << ':'
          << a.kernel_version << ':' << a.variant_id << "|abi:" << a.abi_schema_version
          << "|generator:" << a.generator_version << "|toolchain:" << a.triton_version
          << "|code:" << a.sha256;
      } else {
        m << "|view";
      }
    }
  }
  cth_device_info info;
  if (cth_device_query(device_id, &info) == 0) {
    m << "|arch:" << info.arch_name << "|cu:" << info.compute_units << "|uuid:";
    for (const unsigned char byte : info.uuid) m << std::hex << static_cast<int>(byte) << std::dec;
    m << "|driver:" << info.driver_version << "|runtime:" << info.runtime_version;
  }
  std::uint64_t hash = 0xcbf29ce484222325ull;  // FNV-1a 64 offset basis
  for (const unsigned char c : m.str()) {
    hash ^= c;
    hash *= 0x100000001b3ull;  // FNV-1a 64 prime
  }
  std::ostringstream hex;
  hex << std::hex << std::setw(16) << std::setfill('0') << hash;
  return hex.str();
}

std::optional<std::string> ReadTuningChoice(const std::filesystem::path& path) {
  std::ifstream in(path);
  if (!in) return std::nullopt;
  std::ostringstream contents;
  contents << in.rdbuf();
  const std::string text = contents.str();
  const std::string marker = "\"candidate_id\": \"";
  const auto begin = text.find(marker);
  if (begin == std::string::npos) return std::nullopt;
  const auto first = begin + marker.size();
  const auto last = text.find('"', first);
  if (last == std::string::npos) return std::nullopt;
  return text.substr(first, last - first);
}

Status WriteTuningChoice(const std::filesystem::path& path, const std::string& key,
                         const std::string& candidate_id, double median_ms) {
  std::error_code error;
  std::filesystem::create_directories(path.parent_path(), error);
  if (error) return Status::RuntimeError("cannot create the tuning cache directory: " + error.message());
  const std::string staging = path.string() + ".tmp";
  {
    std::ofstream out(staging, std::ios::trunc);
    out << "{\n  \"schema_version\": 1,\n  \"tuning_key\": \"" << key << "\",\n  \"candidate_id\": \""
        << candidate_id << "\",\n  \"median_ms\": " << median_ms << "\n}\n";
    if (!out) return Status::RuntimeError("cannot write the tuning cache");
  }
  std::filesystem::rename(staging, path, error);
  if (error) {
    std::filesystem::remove(path, error);
    error.clear();
    std::filesystem::rename(staging, path, error);
  }
  return error ? Status::RuntimeError("cannot publish the tuning cache: " + error.message()) : Status::OK();
}

std::optional<std::size_t> FindCandidate(const PlanOp& op, const std::string& id) {
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
    std::call_once(constants_once_, [&] { constants_status_ = UploadConstants(); });
    return constants_status_;
  }

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
  std::once_flag module_once_;
  Status module_status_;
};

Engine::Engine(ExecutablePlan plan) : state_(std::make_shared<EngineState>(std::move(plan))) {}

const ExecutablePlan& Engine::plan() const { return state_->plan; }

std::unique_ptr<ExecutionContext> Engine::CreateExecutionContext() const {
  return std::make_unique<ExecutionContext>(state_);
}

ExecutionContext::ExecutionContext(std::shared_ptr<EngineState> state) : state_(std::move(state)) {
  if (state_ != nullptr && state_->plan.profile_plans().size() == 1) {
    selected_profile_ = 0;
    const ProfilePlan& pp = state_->plan.profile_plans().front();
    resolved_graph_ = pp.opt_graph;
    shapes_resolved_ = true;
    for (const auto& entry : pp.profile.inputs) input_shapes_[entry.first] = entry.second.opt;
  }
}

ExecutionContext::~ExecutionContext() {
  (void)Synchronize();
  DestroyHipState(static_cast<HipExecutionState*>(hip_state_));
}

const Graph& ExecutionContext::ActiveGraph() const {
  return shapes_resolved_ ? resolved_graph_ : state_->plan.graph();
}

const MemoryPlan& ExecutionContext::ActiveMemoryPlan() const {
  if (selected_profile_ >= 0) {
    return state_->plan.profile_plans().at(static_cast<std::size_t>(selected_profile_)).max_memory_plan;
  }
  return state_->plan.memory_plan();
}

Status ExecutionContext::BindInput(const std::string& name, Tensor tensor) {
  if (state_ == nullptr) return Status::InvalidArgument("ExecutionContext has no EngineState");
  if (run_pending_) return Status::RuntimeError("cannot bind a tensor while a run is pending");
  if (!state_->plan.profile_plans().empty() && !shapes_resolved_) {
    return Status::RuntimeError("ResolveShapes must be called before binding");
  }
  const Graph& graph = ActiveGraph();
  if (!Contains(graph.inputs(), name)) return Status::NotFound("name is not a graph input: " + name);
  const ValueDesc* value = graph.FindValue(name);
  if (value == nullptr) return Status::NotFound("graph input description is missing: " + name);
  CUTRITON_RETURN_IF_ERROR(ValidateBoundTensor(name, value->tensor, tensor));
  tensors_[name] = std::move(tensor);
  tensors_prepared_ = false;
  return Status::OK();
}

Status ExecutionContext::BindOutput(const std::string& name, Tensor tensor) {
  if (state_ == nullptr) return Status::InvalidArgument("ExecutionContext has no EngineState");
  if (run_pending_) return Status::RuntimeError("cannot bind a tensor while a run is pending");
  if (!state_->plan.profile_plans().empty() && !shapes_resolved_) {
    return Status::RuntimeError("ResolveShapes must be called before binding");
  }
  const Graph& graph = ActiveGraph();
  if (!Contains(graph.outputs(), name)) return Status::NotFound("name is not a graph output: " + name);
  const ValueDesc* value = graph.FindValue(name);
  if (value == nullptr) return Status::NotFound("graph output description is missing: " + name);
  CUTRITON_RETURN_IF_ERROR(ValidateBoundTensor(name, value->tensor, tensor));
  tensors_[name] = std::move(tensor);
  tensors_prepared_ = false;
  return Status::OK();
}

Status ExecutionContext::SelectShapeProfile(const std::string& name) {
  if (run_pending_) return Status::RuntimeError("cannot change the profile while a run is pending");
  const auto& profiles = state_->plan.profile_plans();
  const auto found = std::find_if(profiles.begin(), profiles.end(),
                                  [&](const ProfilePlan& p) { return p.profile.name == name; });
  if (found == profiles.end()) return Status::NotFound("ShapeProfile is not defined: " + name);
  selected_profile_ = static_cast<int>(found - profiles.begin());
  input_shapes_.clear();
  for (const auto& entry : found->profile.inputs) input_shapes_[entry.first] = entry.second.opt;
  resolved_graph_ = found->opt_graph;
  shapes_resolved_ = true;
  tensors_.clear();
  workspace_.reset();
  tensors_prepared_ = false;
  kernels_.clear();
  kernels_prepared_ = false;
  tuning_prepared_ = false;
  InvalidateHipGraph();
  return Status::OK();
}

Status ExecutionContext::SetInputShape(const std::string& name, std::vector<int64_t> shape) {
  if (run_pending_) return Status::RuntimeError("cannot change a shape while a run is pending");
  if (selected_profile_ < 0) return Status::RuntimeError("select a ShapeProfile before setting shapes");
  const ShapeProfile& profile =
      state_->plan.profile_plans().at(static_cast<std::size_t>(selected_profile_)).profile;
  const auto range = profile.inputs.find(name);
  if (range == profile.inputs.end()) return Status::NotFound("name is not a profiled graph input: " + name);
  if (shape.size() != range->second.min.size()) {
    return Status::ShapeError("input rank does not match the profile: " + name);
  }
  for (std::size_t axis = 0; axis < shape.size(); ++axis) {
    if (shape[axis] < range->second.min[axis] || shape[axis] > range->second.max[axis]) {
      return Status::ShapeError("input shape is outside the profile range: " + name);
    }
  }
  input_shapes_[name] = std::move(shape);
  shapes_resolved_ = false;
  tensors_.clear();
  tensors_prepared_ = false;
  kernels_.clear();
  kernels_prepared_ = false;
  tuning_prepared_ = false;
  return Status::OK();
}

Status ExecutionContext::ResolveShapes() {
  if (selected_profile_ < 0) return Status::RuntimeError("select a ShapeProfile before resolving shapes");
  const ProfilePlan& pp = state_->plan.profile_plans().at(static_cast<std::size_t>(selected_profile_));
  resolved_graph_ = pp.opt_graph;
  for (const auto& input : resolved_graph_.inputs()) {
    const auto shape = input_shapes_.find(input);
    if (shape == input_shapes_.end()) return Status::InvalidArgument("input shape is not set: " + input);
    TensorDesc desc = resolved_graph_.FindValue(input)->tensor;
    desc.shape = shape->second;
    CUTRITON_RETURN_IF_ERROR(resolved_graph_.SetValueDesc(input, std::move(desc)));
  }
  CUTRITON_RETURN_IF_ERROR(CreateShapeInferencePass()->Run(&resolved_graph_));
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

Status ExecutionContext::PrepareTensors() {
  if (tensors_prepared_) return Status::OK();
  if (state_ == nullptr) return Status::InvalidArgument("ExecutionContext has no EngineState");
  CUTRITON_RETURN_IF_ERROR(state_->InitializeConstants());
  for (const auto& entry : state_->device_constants) tensors_[entry.first] = entry.second;
  const MemoryPlan& memory = ActiveMemoryPlan();
  const Device& device = state_->plan.backend_options().device;
  if (memory.workspace_size_bytes != 0 &&
      (workspace_ == nullptr || workspace_->size_bytes() < memory.workspace_size_bytes)) {
    if (device.type == DeviceType::kHIP) {
      CUTRITON_RETURN_IF_ERROR(Buffer::AllocateHip(memory.workspace_size_bytes, device.id, &workspace_));
    } else {
      workspace_ = Buffer::AllocateHost(memory.workspace_size_bytes);
    }
  }
  const Graph& graph = ActiveGraph();
  for (const auto& allocation : memory.allocations) {
    const ValueDesc* value = graph.FindValue(allocation.value_name);
    if (value == nullptr) {
      // A candidate temporary: described like its "like" value.
      const ValueDesc* like = nullptr;
      for (const auto& op : state_->plan.ops()) {
        for (const auto& candidate : op.candidates) {
          for (const auto& temporary : candidate.temporaries) {
            if (temporary.name == allocation.value_name) like = graph.FindValue(temporary.like_value);
          }
          if (like != nullptr) break;
        }
        if (like != nullptr) break;
      }
      if (like == nullptr) return Status::Internal("allocation references an unknown value: " + allocation.value_name);
      tensors_[allocation.value_name] = Tensor(like->tensor, workspace_, allocation.offset);
      continue;
    }
    if (!allocation.alias_of.empty()) {
      const auto source = tensors_.find(allocation.alias_of);
      if (source == tensors_.end()) {
        return Status::Internal("alias source tensor is missing: " + allocation.alias_of);
      }
      if (value->tensor.ByteSize() != source->second.desc().ByteSize()) {
        return Status::ShapeError("alias changes the byte size of " + allocation.value_name);
      }
      tensors_[allocation.value_name] =
          Tensor(value->tensor, source->second.buffer(), source->second.byte_offset());
      continue;
    }
    if (workspace_ == nullptr || allocation.offset > workspace_->size_bytes() ||
        allocation.size_bytes > workspace_->size_bytes() - allocation.offset) {
      return Status::Internal("allocation exceeds the workspace: " + allocation.value_name);
    }
    tensors_[allocation.value_name] = Tensor(value->tensor, workspace_, allocation.offset);
  }
  // One zero-initialised runtime scratch buffer per context, sized for the
  // largest declared need of any candidate (tuning may run every one).
  std::int64_t scratch = 0;
  for (const auto& op : state_->plan.ops()) {
    for (const auto& candidate : op.candidates) {
      for (const auto& step : candidate.steps) {
        if (const auto* inv = std::get_if<KernelInvocation>(&step)) {
          scratch = std::max(scratch, inv->artifact.runtime_scratch_bytes);
        }
      }
    }
  }
  if (scratch > 0 && device.type == DeviceType::kHIP &&
      (runtime_scratch_ == nullptr || runtime_scratch_->size_bytes() < static_cast<std::size_t>(scratch))) {
    CUTRITON_RETURN_IF_ERROR(Buffer::AllocateHip(static_cast<std::size_t>(scratch), device.id, &runtime_scratch_));
    CUTRITON_RETURN_IF_ERROR(RuntimeStatus(
        cth_memset(runtime_scratch_->data(), 0, runtime_scratch_->size_bytes(), device.id), "hipMemset"));
    InvalidateHipGraph();
  }
  tensors_prepared_ = true;
  return Status::OK();
}

Status ExecutionContext::PrepareKernels() {
  if (kernels_prepared_) return Status::OK();
  if (state_ == nullptr) return Status::InvalidArgument("ExecutionContext has no EngineState");
  CUTRITON_RETURN_IF_ERROR(RegisterBuiltinBackends());
  CUTRITON_RETURN_IF_ERROR(state_->InitializeModuleCache());
  if (selected_candidates_.size() != state_->plan.ops().size()) {
    return Status::Internal("tuning selections are not prepared");
  }
  kernels_.clear();
  const int device_id = state_->plan.backend_options().device.id;
  for (std::size_t i = 0; i < state_->plan.ops().size(); ++i) {
    const PlanOp& op = state_->plan.ops()[i];
    auto backend = KernelRegistry::Global().GetBackend(op.backend_name);
    if (backend == nullptr) return Status::NotFound("backend is not registered: " + op.backend_name);
    const Node& node = ActiveGraph().nodes().at(static_cast<std::size_t>(op.node_id));
    const std::size_t selected = selected_candidates_[i];
    if (selected >= op.candidates.size()) return Status::Internal("selected candidate is out of range");
    std::vector<std::unique_ptr<OpKernel>> group;
    for (const auto& step : op.candidates[selected].steps) {
      std::unique_ptr<OpKernel> kernel;
      if (const auto* inv = std::get_if<KernelInvocation>(&step)) {
        CUTRITON_RETURN_IF_ERROR(CreateInvocationKernel(*inv, device_id, state_->module_cache, &kernel));
      } else {
        CUTRITON_RETURN_IF_ERROR(
            backend->CreateKernel(node, ActiveGraph(), state_->plan.backend_options(), &kernel));
      }
      if (kernel == nullptr) return Status::Internal("backend returned a null OpKernel");
      group.push_back(std::move(kernel));
    }
    if (group.empty()) {
      std::unique_ptr<OpKernel> kernel;
      CUTRITON_RETURN_IF_ERROR(backend->CreateKernel(node, ActiveGraph(), state_->plan.backend_options(), &kernel));
      if (kernel == nullptr) return Status::Internal("backend returned a null OpKernel");
      group.push_back(std::move(kernel));
    }
    kernels_.push_back(std::move(group));
  }
  kernels_prepared_ = true;
  return Status::OK();
}

Status ExecutionContext::PrepareTuning() {
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

  // Resolve from the cache first; remember which ops still need timing.
  std::vector<std::size_t> to_tune;
  std::vector<std::string> keys(ops.size());
  for (std::size_t i = 0; i < ops.size(); ++i) {
    const PlanOp& op = ops[i];
    if (op.candidates.size() < 2) continue;
    const Node& node = graph.nodes().at(static_cast<std::size_t>(op.node_id));
    keys[i] = TuningKey(op, node, graph, device.id);
    if (config.mode != TuningMode::kForceRetune) {
      const auto cached = ReadTuningChoice(std::filesystem::path(config.cache_dir) / (keys[i] + ".json"));
      if (cached) {
        if (const auto index = FindCandidate(op, *cached)) {
          selected_candidates_[i] = *index;
          continue;
        }
      }
      if (config.mode == TuningMode::kUseCache && selected_profile_ >= 0) {
        const Graph& opt = state_->plan.profile_plans().at(static_cast<std::size_t>(selected_profile_)).opt_graph;
        const std::string opt_key =
            TuningKey(op, opt.nodes().at(static_cast<std::size_t>(op.node_id)), opt, device.id);
        const auto choice = ReadTuningChoice(std::filesystem::path(config.cache_dir) / (opt_key + ".json"));
        if (choice) {
          if (const auto index = FindCandidate(op, *choice)) {
            selected_candidates_[i] = *index;
            continue;
          }
        }
      }
    }
    if (config.mode != TuningMode::kUseCache) to_tune.push_back(i);
  }
  if (to_tune.empty()) {
    tuning_prepared_ = true;
    return Status::OK();
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

  auto build_kernels = [&](const ExecutionCandidate& candidate,
                           std::vector<std::unique_ptr<OpKernel>>* out) -> Status {
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
    KernelContext context{&node, &tensors_, stream, nullptr, ScratchPointer(), ScratchBytes()};
    for (auto& kernel : kernels) CUTRITON_RETURN_IF_ERROR(kernel->Compute(&context));
  }
  CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_stream_synchronize(stream), "hipStreamSynchronize"));

  // CUTRITON_TUNING_LOG=1 prints every candidate's median and every
  // numeric-gate rejection to stderr.
  const bool tuning_log = std::getenv("CUTRITON_TUNING_LOG") != nullptr;
  for (const std::size_t op_index : to_tune) {
    const PlanOp& op = ops[op_index];
    const Node& node = graph.nodes().at(static_cast<std::size_t>(op.node_id));
    KernelContext context{&node, &tensors_, stream, nullptr, ScratchPointer(), ScratchBytes()};
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
      CUTRITON_RETURN_IF_ERROR(TensorToHostFloats(output, &produced));
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
    if (!std::isfinite(best_ms)) {
      return Status::RuntimeError("no numerically valid tuning candidate for " + op.node_name);
    }
    selected_candidates_[op_index] = best;
    // Leave the op's output as the chosen candidate computes it.
    std::vector<std::unique_ptr<OpKernel>> kernels;
    CUTRITON_RETURN_IF_ERROR(build_kernels(op.candidates[best], &kernels));
    for (auto& kernel : kernels) CUTRITON_RETURN_IF_ERROR(kernel->Compute(&context));
    CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_stream_synchronize(stream), "hipStreamSynchronize"));
    CUTRITON_RETURN_IF_ERROR(WriteTuningChoice(std::filesystem::path(config.cache_dir) / (keys[op_index] + ".json"),
                                               keys[op_index], op.candidates[best].candidate_id, best_ms));
  }
  tuning_prepared_ = true;
  return Status::OK();
}

Status ExecutionContext::ValidateBindings() const {
  const Graph& graph = ActiveGraph();
  for (const auto& name : graph.inputs()) {
    if (tensors_.count(name) == 0) return Status::InvalidArgument("graph input is not bound: " + name);
  }
  for (const auto& name : graph.outputs()) {
    if (tensors_.count(name) == 0) return Status::InvalidArgument("graph output is not bound: " + name);
  }
  for (const auto& node : graph.nodes()) {
    for (const auto& name : node.inputs()) {
      if (tensors_.count(name) == 0) return Status::InvalidArgument("node input tensor is missing: " + name);
    }
    for (const auto& name : node.outputs()) {
      if (tensors_.count(name) == 0) return Status::InvalidArgument("node output tensor is missing: " + name);
    }
  }
  return Status::OK();
}

Status ExecutionContext::Run() {
  CUTRITON_RETURN_IF_ERROR(RunAsync(nullptr));
  return Synchronize();
}

Status ExecutionContext::EnqueueOps(void* stream, bool capture) {
  auto* hip = static_cast<HipExecutionState*>(hip_state_);
  const bool profiling = state_->plan.enable_profiling();
  for (std::size_t i = 0; i < kernels_.size(); ++i) {
    const PlanOp& op = state_->plan.ops()[i];
    const Node& node = ActiveGraph().nodes().at(static_cast<std::size_t>(op.node_id));
    EventPair& events = hip->events[i];
    // Events inside a capture are graph nodes placed by CaptureGraph.
    events.timed = profiling && node.op_type() != "Flatten";
    if (events.timed && !capture) CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_event_record(events.start, stream), "hipEventRecord"));
    KernelContext context{&node, &tensors_, stream, nullptr, ScratchPointer(), ScratchBytes()};
    for (auto& kernel : kernels_[i]) CUTRITON_RETURN_IF_ERROR(kernel->Compute(&context));
    if (events.timed && !capture) CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_event_record(events.end, stream), "hipEventRecord"));
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
  if (!state_->plan.enable_profiling()) {
    CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_stream_begin_capture(stream), "hipStreamBeginCapture"));
    const Status enqueued = EnqueueOps(stream, true);
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
    KernelContext context{&node, &tensors_, stream, nullptr, ScratchPointer(), ScratchBytes()};
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
    CUTRITON_RETURN_IF_ERROR(PrepareTensors());
  }
  CUTRITON_RETURN_IF_ERROR(ValidateBindings());
  {
    StageTimer timer("tuning");
    CUTRITON_RETURN_IF_ERROR(PrepareTuning());
  }
  {
    StageTimer timer("kernel loading");
    CUTRITON_RETURN_IF_ERROR(PrepareKernels());
  }

  const Device& device = state_->plan.backend_options().device;
  if (device.type != DeviceType::kHIP) {
    profiler_.Clear();
    for (std::size_t i = 0; i < kernels_.size(); ++i) {
      const PlanOp& op = state_->plan.ops()[i];
      const Node& node = ActiveGraph().nodes().at(static_cast<std::size_t>(op.node_id));
      KernelContext context{&node, &tensors_, stream,
                            state_->plan.enable_profiling() ? &profiler_ : nullptr, ScratchPointer(), ScratchBytes()};
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
    CUTRITON_RETURN_IF_ERROR(EnqueueOps(hip->active_stream, false));
    run_pending_ = true;
    return Status::OK();
  }

  std::ostringstream key;
  key << "profile:" << selected_profile_ << "|workspace:"
      << (workspace_ == nullptr ? nullptr : workspace_->data());
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
  auto entry = std::find_if(hip->graphs.begin(), hip->graphs.end(),
                            [&](const GraphEntry& e) { return e.key == graph_key; });
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
  KernelContext context{&node, &tensors_, s, nullptr, ScratchPointer(), ScratchBytes()};
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
  if (state_->plan.backend_options().device.type != DeviceType::kHIP) {
    run_pending_ = false;
    return Status::OK();
  }
  auto* hip = static_cast<HipExecutionState*>(hip_state_);
  run_pending_ = false;
  CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_stream_synchronize(hip->active_stream), "hipStreamSynchronize"));
  profiler_.Clear();
  if (state_->plan.enable_profiling()) {
    for (std::size_t i = 0; i < state_->plan.ops().size(); ++i) {
      const PlanOp& op = state_->plan.ops()[i];
      float ms = 0.0f;
      if (hip->events[i].timed) {
        CUTRITON_RETURN_IF_ERROR(RuntimeStatus(
            cth_event_elapsed_ms(&ms, hip->events[i].start, hip->events[i].end), "hipEventElapsedTime"));
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
