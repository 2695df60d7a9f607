// Artifact launcher. Behaviour follows reference
// src/backend/cuda_launcher.cpp:47-468: a module cache keyed by code-object
// SHA-256 (functions by SHA+symbol), an argument binder over the manifest's
// argument sources, the grid-AST evaluator with positivity/overflow checks,
// and an OpKernel that launches one invocation. Launch goes through the
// C-ABI runtime layer (hipModuleLoadData / hipModuleLaunchKernel);
// workgroups have num_warps * 64 threads.
#include <array>
#include <cstring>
#include <fstream>
#include <limits>
#include <mutex>
#include <sstream>
#include <unordered_map>

#include "cutriton/backend/backend.h"
#include "cutriton/core/buffer.h"
#include "cutriton_hip_runtime.h"

namespace cutriton {

namespace {

Status RuntimeStatus(int code, const char* operation) {
  if (code == 0) return Status::OK();
  return Status::RuntimeError(std::string(operation) + ": " + cth_last_error());
}

}  // namespace

class HipModuleCache {
 public:
  explicit HipModuleCache(int device_id) : device_id_(device_id) {}
  ~HipModuleCache() {
    std::lock_guard<std::mutex> lock(mutex_);
    for (auto& entry : modules_) cth_module_unload(entry.second);
  }
  HipModuleCache(const HipModuleCache&) = delete;
  HipModuleCache& operator=(const HipModuleCache&) = delete;

  Status GetFunction(const KernelArtifact& artifact, cth_function* function) {
    if (function == nullptr) return Status::InvalidArgument("function output is null");
    std::lock_guard<std::mutex> lock(mutex_);
    const std::string function_key = artifact.sha256 + ":" + artifact.symbol;
    const auto cached = functions_.find(function_key);
    if (cached != functions_.end()) {
      *function = cached->second;
      return Status::OK();
    }
    auto module = modules_.find(artifact.sha256);
    if (module == modules_.end()) {
      std::ifstream in(artifact.binary_path, std::ios::binary);
      if (!in) return Status::NotFound("kernel binary not found: " + artifact.binary_path.string());
      std::ostringstream image;
      image << in.rdbuf();
      const std::string bytes = image.str();
      cth_module loaded = nullptr;
      CUTRITON_RETURN_IF_ERROR(RuntimeStatus(
          cth_module_load_data(&loaded, bytes.data(), bytes.size(), device_id_), "hipModuleLoadData"));
      module = modules_.emplace(artifact.sha256, loaded).first;
    }
    cth_function loaded = nullptr;
    CUTRITON_RETURN_IF_ERROR(RuntimeStatus(
        cth_module_get_function(&loaded, module->second, artifact.symbol.c_str()),
        ("hipModuleGetFunction(" + artifact.symbol + ")").c_str()));
    functions_.emplace(function_key, loaded);
    *function = loaded;
    return Status::OK();
  }

  std::size_t size() const {
    std::lock_guard<std::mutex> lock(mutex_);
    return modules_.size();
  }

  bool HasCodeObject(const std::string& sha256) const {
    std::lock_guard<std::mutex> lock(mutex_);
    return modules_.count(sha256) != 0;
  }

 private:
  int device_id_;
  mutable std::mutex mutex_;
  std::unordered_map<std::string, cth_module> modules_;
  std::unordered_map<std::string, cth_function> functions_;
};

namespace {

// One kernel argument as HIP reads it: 8-byte pointers, 4-byte i32/f32.
union ArgumentSlot {
  void* pointer;
  int32_t i32;
  float f32;
};

const Tensor* LookupTensor(const std::vector<std::string>& names, int index,
                           const KernelContext& context, Status* status) {
  if (index < 0 || static_cast<std::size_t>(index) >= names.size()) {
    *status = Status::InvalidArgument("kernel tensor index is out of range");
    return nullptr;
  }
  const auto it = context.tensors->find(names[static_cast<std::size_t>(index)]);
  if (it == context.tensors->end() || !it->second.defined()) {
    *status = Status::NotFound("kernel tensor is not bound: " + names[static_cast<std::size_t>(index)]);
    return nullptr;
  }
  return &it->second;
}

Status NarrowToI32(int64_t value, bool require_positive, int32_t* out, const char* what) {
  if ((require_positive && value <= 0) || value > std::numeric_limits<int32_t>::max() ||
      value < std::numeric_limits<int32_t>::min()) {
    return Status::ShapeError(std::string("kernel ") + what + " does not fit an i32");
  }
  *out = static_cast<int32_t>(value);
  return Status::OK();
}

int64_t IntegerAttribute(const Node& node, const KernelArgumentSource& source) {
  if (auto list = node.GetAttribute<std::vector<int64_t>>(source.attribute_name)) {
    if (source.attribute_index >= 0 && static_cast<std::size_t>(source.attribute_index) < list->size()) {
      return (*list)[static_cast<std::size_t>(source.attribute_index)];
    }
  }
  if (auto scalar = node.GetAttribute<int64_t>(source.attribute_name)) return *scalar;
  return source.default_int;
}

Status BindArguments(const KernelInvocation& invocation, const KernelContext& context,
                     std::vector<ArgumentSlot>* slots) {
  slots->assign(invocation.artifact.arguments.size(), ArgumentSlot{nullptr});
  const Node& node = *context.node;
  bool scratch_bound = false;
  for (std::size_t i = 0; i < invocation.artifact.arguments.size(); ++i) {
    const KernelArgumentSource& s = invocation.artifact.arguments[i].source;
    ArgumentSlot& slot = (*slots)[i];
    Status status;
    switch (s.kind) {
      case KernelArgumentSourceKind::kInput:
      case KernelArgumentSourceKind::kOutput: {
        const auto& names = s.kind == KernelArgumentSourceKind::kInput ? invocation.inputs
                                                                       : invocation.outputs;
        const Tensor* t = LookupTensor(names, s.index, context, &status);
        if (t == nullptr) return status;
        slot.pointer = static_cast<std::uint8_t*>(t->buffer()->data()) + t->byte_offset();
        break;
      }
      case KernelArgumentSourceKind::kInputDim:
      case KernelArgumentSourceKind::kOutputDim: {
        const auto& names = s.kind == KernelArgumentSourceKind::kInputDim ? invocation.inputs
                                                                          : invocation.outputs;
        const Tensor* t = LookupTensor(names, s.index, context, &status);
        if (t == nullptr) return status;
        const auto& shape = t->desc().shape;
        if (s.axis < 0 || static_cast<std::size_t>(s.axis) >= shape.size()) {
          return Status::ShapeError("kernel dimension axis is out of range");
        }
        CUTRITON_RETURN_IF_ERROR(NarrowToI32(shape[static_cast<std::size_t>(s.axis)], false, &slot.i32, "dimension"));
        break;
      }
      case KernelArgumentSourceKind::kInputDimProduct: {
        const Tensor* t = LookupTensor(invocation.inputs, s.index, context, &status);
        if (t == nullptr) return status;
        const auto& shape = t->desc().shape;
        if (s.begin_axis < 0 || static_cast<std::size_t>(s.begin_axis) > shape.size()) {
          return Status::ShapeError("kernel dimension-product axis is out of range");
        }
        int64_t product = 1;
        for (std::size_t a = static_cast<std::size_t>(s.begin_axis); a < shape.size(); ++a) product *= shape[a];
        CUTRITON_RETURN_IF_ERROR(NarrowToI32(product, true, &slot.i32, "dimension product"));
        break;
      }
      case KernelArgumentSourceKind::kOutputNumElements: {
        const Tensor* t = LookupTensor(invocation.outputs, s.index, context, &status);
        if (t == nullptr) return status;
        CUTRITON_RETURN_IF_ERROR(NarrowToI32(t->desc().NumElements(), true, &slot.i32, "element count"));
        break;
      }
      case KernelArgumentSourceKind::kAttributeInt64:
        slot.i32 = static_cast<int32_t>(IntegerAttribute(node, s));
        break;
      case KernelArgumentSourceKind::kAttributeFloat64: {
        double value = s.default_float;
        if (auto primary = node.GetAttribute<double>(s.attribute_name)) {
          value = *primary;
        } else if (!s.alternate_attribute_name.empty()) {
          value = node.GetAttribute<double>(s.alternate_attribute_name).value_or(s.default_float);
        }
        slot.f32 = static_cast<float>(value);
        break;
      }
      case KernelArgumentSourceKind::kLiteralInt32:
        slot.i32 = static_cast<int32_t>(s.default_int);
        break;
      case KernelArgumentSourceKind::kRuntimeReserved:
        slot.pointer = nullptr;
        if (invocation.artifact.runtime_scratch_bytes > 0 && !scratch_bound) {
          if (context.runtime_scratch == nullptr ||
              context.runtime_scratch_bytes < static_cast<std::size_t>(invocation.artifact.runtime_scratch_bytes)) {
            return Status::RuntimeError("kernel " + invocation.artifact.symbol + " needs " +
                                        std::to_string(invocation.artifact.runtime_scratch_bytes) +
                                        " bytes of runtime scratch");
          }
          slot.pointer = context.runtime_scratch;
          scratch_bound = true;
        }
        break;
    }
  }
  return Status::OK();
}

Status EvaluateGrid(const GridExpression& e, const KernelInvocation& invocation,
                    const KernelContext& context, int64_t* out) {
  Status status;
  switch (e.kind) {
    case GridExpressionKind::kLiteral:
      *out = e.literal;
      break;
    case GridExpressionKind::kVariantMeta: {
      const auto it = invocation.artifact.launch_meta.find(e.meta_name);
      if (it == invocation.artifact.launch_meta.end()) {
        return Status::InvalidArgument("launch grid references missing variant meta: " + e.meta_name);
      }
      *out = it->second;
      break;
    }
    case GridExpressionKind::kInputDim:
    case GridExpressionKind::kOutputDim: {
      const auto& names = e.kind == GridExpressionKind::kInputDim ? invocation.inputs : invocation.outputs;
      const Tensor* t = LookupTensor(names, e.tensor_index, context, &status);
      if (t == nullptr) return status;
      const auto& shape = t->desc().shape;
      if (e.axis < 0 || static_cast<std::size_t>(e.axis) >= shape.size()) {
        return Status::ShapeError("launch grid axis is out of range");
      }
      *out = shape[static_cast<std::size_t>(e.axis)];
      break;
    }
    case GridExpressionKind::kInputNumElements:
    case GridExpressionKind::kOutputNumElements: {
      const auto& names =
          e.kind == GridExpressionKind::kInputNumElements ? invocation.inputs : invocation.outputs;
      const Tensor* t = LookupTensor(names, e.tensor_index, context, &status);
      if (t == nullptr) return status;
      *out = t->desc().NumElements();
      break;
    }
    case GridExpressionKind::kCeilDiv:
    case GridExpressionKind::kMultiply: {
      if (e.operands.size() != 2) return Status::InvalidArgument("launch grid operator is malformed");
      int64_t lhs = 0;
      int64_t rhs = 0;
      CUTRITON_RETURN_IF_ERROR(EvaluateGrid(e.operands[0], invocation, context, &lhs));
      CUTRITON_RETURN_IF_ERROR(EvaluateGrid(e.operands[1], invocation, context, &rhs));
      if (lhs <= 0 || rhs <= 0) return Status::ShapeError("launch grid operands must be positive");
      if (e.kind == GridExpressionKind::kCeilDiv) {
        *out = (lhs + rhs - 1) / rhs;
      } else {
        if (lhs > std::numeric_limits<int64_t>::max() / rhs) {
          return Status::ShapeError("launch grid multiplication overflows");
        }
        *out = lhs * rhs;
      }
      break;
    }
  }
  return *out > 0 ? Status::OK() : Status::ShapeError("launch grid dimension is not positive");
}

class InvocationKernel final : public OpKernel {
 public:
  InvocationKernel(KernelInvocation invocation, std::shared_ptr<HipModuleCache> cache,
                   cth_function function)
      : invocation_(std::move(invocation)), cache_(std::move(cache)), function_(function) {}

  const char* backend_name() const override { return kHipBackendName; }
  const char* op_type() const override { return invocation_.artifact.op_type.c_str(); }

  Status Compute(KernelContext* context) override {
    if (context == nullptr || context->node == nullptr || context->tensors == nullptr) {
      return Status::InvalidArgument("invalid artifact KernelContext");
    }
    CUTRITON_RETURN_IF_ERROR(BindArguments(invocation_, *context, &slots_));
    params_.resize(slots_.size());
    for (std::size_t i = 0; i < slots_.size(); ++i) params_[i] = &slots_[i];
    unsigned int grid[3];
    for (int axis = 0; axis < 3; ++axis) {
      int64_t value = 0;
      CUTRITON_RETURN_IF_ERROR(EvaluateGrid(invocation_.artifact.launch_grid[static_cast<std::size_t>(axis)],
                                            invocation_, *context, &value));
      if (value > static_cast<int64_t>(std::numeric_limits<int32_t>::max())) {
        return Status::ShapeError("launch grid dimension exceeds the HIP limit");
      }
      grid[axis] = static_cast<unsigned int>(value);
    }
    const unsigned int block[3] = {static_cast<unsigned int>(invocation_.artifact.block_threads()), 1, 1};
    return RuntimeStatus(
        cth_launch(function_, grid, block,
                   static_cast<unsigned int>(invocation_.artifact.shared_memory_bytes), context->stream,
                   params_.data()),
        ("hipModuleLaunchKernel(" + invocation_.artifact.symbol + ")").c_str());
  }

 private:
  KernelInvocation invocation_;
  std::shared_ptr<HipModuleCache> cache_;  // keeps the module loaded
  cth_function function_;
  std::vector<ArgumentSlot> slots_;
  std::vector<void*> params_;
};

}  // namespace

Status CreateHipModuleCache(int device_id, std::shared_ptr<HipModuleCache>* cache) {
  if (cache == nullptr) return Status::InvalidArgument("module cache output is null");
  CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_set_device(device_id), "hipSetDevice"));
  *cache = std::make_shared<HipModuleCache>(device_id);
  return Status::OK();
}

Status CreateInvocationKernel(const KernelInvocation& invocation, int device_id,
                              std::shared_ptr<HipModuleCache> cache,
                              std::unique_ptr<OpKernel>* kernel) {
  (void)device_id;
  if (kernel == nullptr || cache == nullptr) {
    return Status::InvalidArgument("invocation kernel arguments are invalid");
  }
  cth_function function = nullptr;
  CUTRITON_RETURN_IF_ERROR(cache->GetFunction(invocation.artifact, &function));
  *kernel = std::make_unique<InvocationKernel>(invocation, std::move(cache), function);
  return Status::OK();
}

std::size_t LoadedModuleCount(const std::shared_ptr<HipModuleCache>& cache) {
  return cache == nullptr ? 0 : cache->size();
}

bool CodeObjectLoaded(const std::shared_ptr<HipModuleCache>& cache, const KernelArtifact& artifact) {
  return cache != nullptr && cache->HasCodeObject(artifact.sha256);
}

}  // namespace cutriton
