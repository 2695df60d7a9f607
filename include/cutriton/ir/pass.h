// Graph passes and the default compile pipeline.
// Mirrors include/cutriton/ir/pass.h:14-68 of the reference, plus the
// conv-epilogue residual fusion (FusedConvBatchNorm + AddRelu) of this backend.
#pragma once

#include <memory>
#include <string>
#include <vector>

#include "cutriton/core/status.h"
#include "cutriton/ir/graph.h"

namespace cutriton {

class GraphPass {
 public:
  virtual ~GraphPass() = default;
  virtual const char* name() const = 0;
  virtual Status Run(Graph* graph) const = 0;
};

class PassManager {
 public:
  void Add(std::unique_ptr<GraphPass> pass);
  Status Run(Graph* graph) const;
  const std::vector<std::string>& executed_passes() const { return executed_passes_; }

 private:
  std::vector<std::unique_ptr<GraphPass>> passes_;
  mutable std::vector<std::string> executed_passes_;
};

std::unique_ptr<GraphPass> CreateTopologicalSortPass();
std::unique_ptr<GraphPass> CreateShapeInferencePass();
std::unique_ptr<GraphPass> CreateConstantFoldingPass();
std::unique_ptr<GraphPass> CreateDeadNodeEliminationPass();
// Conv -> BatchNormalization [-> Relu] becomes FusedConvBatchNorm[Relu].
std::unique_ptr<GraphPass> CreateConvBatchNormReluFusionPass();
// Add -> Relu becomes AddRelu.
std::unique_ptr<GraphPass> CreateAddReluFusionPass();
// FusedConvBatchNorm -> AddRelu(conv, residual) becomes
// FusedConvBatchNormAddRelu(x, w, scale, bias, mean, var, residual): the
// residual join is applied in the convolution epilogue.
std::unique_ptr<GraphPass> CreateConvBatchNormAddReluFusionPass();
// Gemm -> Gelu becomes GemmGelu when the Gemm output is private.
std::unique_ptr<GraphPass> CreateGemmGeluFusionPass();
// Add -> LayerNormalization becomes SkipLayerNormalization.
std::unique_ptr<GraphPass> CreateSkipLayerNormalizationFusionPass();
std::unique_ptr<GraphPass> CreateFlattenGemmNormalizationPass();
// Attention's default scale 1 / sqrt(head dimension) (no counterpart in the
// reference, which has no attention).
std::unique_ptr<GraphPass> CreateAttentionScalePass();
std::unique_ptr<GraphPass> CreateStaticShapeValidationPass();

// The default pipeline. `enable_transformer_fusions` toggles GemmGelu and
// SkipLayerNormalization fusion; `enable_residual_epilogue_fusion` toggles the
// conv-epilogue residual fusion.
PassManager CreateDefaultCompilePasses(bool enable_transformer_fusions = true,
                                       bool enable_residual_epilogue_fusion = true);

}  // namespace cutriton
