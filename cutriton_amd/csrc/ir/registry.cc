// OpSchemaRegistry and FusionRegistry. Behaviour follows reference
// src/ir/op_schema.cpp:8-46 and src/ir/fusion.cpp:8-60; the fusion table adds
// the decomposition of FusedConvBatchNormAddRelu used by this backend.
#include <algorithm>
#include <mutex>

#include "cutriton/ir/fusion.h"
#include "cutriton/ir/op_schema.h"

namespace cutriton {

OpSchemaRegistry& OpSchemaRegistry::Global() {
  static OpSchemaRegistry registry;
  return registry;
}

Status OpSchemaRegistry::Register(OpSchema schema) {
  if (schema.op_type.empty() || !schema.infer || schema.min_inputs > schema.max_inputs ||
      schema.outputs == 0) {
    return Status::InvalidArgument("OpSchema is incomplete");
  }
  std::unique_lock<std::shared_mutex> lock(mutex_);
  const std::string key = schema.op_type;
  if (schemas_.count(key) != 0) return Status::AlreadyExists("OpSchema already registered: " + key);
  schemas_.emplace(key, std::make_shared<const OpSchema>(std::move(schema)));
  return Status::OK();
}

std::shared_ptr<const OpSchema> OpSchemaRegistry::Find(const std::string& op_type) const {
  std::shared_lock<std::shared_mutex> lock(mutex_);
  const auto it = schemas_.find(op_type);
  return it == schemas_.end() ? nullptr : it->second;
}

std::vector<std::string> OpSchemaRegistry::AvailableOps() const {
  std::shared_lock<std::shared_mutex> lock(mutex_);
  std::vector<std::string> names;
  names.reserve(schemas_.size());
  for (const auto& entry : schemas_) names.push_back(entry.first);
  std::sort(names.begin(), names.end());
  return names;
}

void OpSchemaRegistry::ClearForTests() {
  std::unique_lock<std::shared_mutex> lock(mutex_);
  schemas_.clear();
}

FusionRegistry& FusionRegistry::Global() {
  static FusionRegistry registry;
  return registry;
}

Status FusionRegistry::Register(FusionAlternative alternative) {
  if (alternative.fused_op_type.empty() || alternative.candidate_id.empty() ||
      alternative.decomposed_ops.empty()) {
    return Status::InvalidArgument("FusionAlternative is incomplete");
  }
  std::unique_lock<std::shared_mutex> lock(mutex_);
  auto& list = alternatives_[alternative.fused_op_type];
  for (const auto& existing : list) {
    if (existing.candidate_id == alternative.candidate_id) {
      return Status::AlreadyExists("fusion alternative already registered: " +
                                   alternative.candidate_id);
    }
  }
  list.push_back(std::move(alternative));
  return Status::OK();
}

std::vector<FusionAlternative> FusionRegistry::Find(const std::string& fused_op_type) const {
  std::shared_lock<std::shared_mutex> lock(mutex_);
  const auto it = alternatives_.find(fused_op_type);
  return it == alternatives_.end() ? std::vector<FusionAlternative>{} : it->second;
}

void FusionRegistry::ClearForTests() {
  std::unique_lock<std::shared_mutex> lock(mutex_);
  alternatives_.clear();
}

Status RegisterBuiltinFusionAlternatives() {
  const FusionAlternative table[] = {
      {"FusedConvBatchNormRelu", "unfused:conv_bn_relu", {"Conv", "BatchNormalization", "Relu"}},
      {"FusedConvBatchNorm", "unfused:conv_bn", {"Conv", "BatchNormalization"}},
      {"FusedConvBatchNormAddRelu", "unfused:conv_bn_add_relu",
       {"FusedConvBatchNorm", "AddRelu"}},
      {"AddRelu", "unfused:add_relu", {"Add", "Relu"}},
      {"GemmGelu", "unfused:gemm_gelu", {"Gemm", "Gelu"}},
      {"SkipLayerNormalization", "unfused:add_layer_norm", {"Add", "LayerNormalization"}},
  };
  auto& registry = FusionRegistry::Global();
  for (const auto& entry : table) {
    const Status status = registry.Register(entry);
    if (!status.ok() && status.code() != ErrorCode::kAlreadyExists) return status;
  }
  return Status::OK();
}

}  // namespace cutriton
