// Kernel Pack v2: manifest types, loader and catalog.
// Mirrors include/cutriton/backend/kernel_artifact.h:14-154 of the reference.
// Differences that belong to the gfx950 target:
//   * binary_format is "hsaco" (an AMDGPU code object), never "ptx";
//   * min_compute_capability carries the numeric gfx architecture (950 for
//     gfx950) and the optional target_arch names it ("gfx950");
//   * num_warps counts 64-lane wavefronts, so a launch uses num_warps*64
//     threads per workgroup.
#pragma once

#include <array>
#include <cstdint>
#include <filesystem>
#include <string>
#include <unordered_map>
#include <vector>

#include "cutriton/core/status.h"

namespace cutriton {

enum class KernelArgumentSourceKind {
  kInput,
  kOutput,
  kInputDim,
  kInputDimProduct,
  kOutputDim,
  kOutputNumElements,
  kAttributeInt64,
  kAttributeFloat64,
  kLiteralInt32,
  kRuntimeReserved,
};

struct KernelArgumentSource {
  KernelArgumentSourceKind kind{KernelArgumentSourceKind::kRuntimeReserved};
  int index{0};
  int axis{0};
  int begin_axis{0};
  std::string attribute_name;
  std::string alternate_attribute_name;
  int attribute_index{0};
  int64_t default_int{0};
  double default_float{0.0};
  // "input" only: the kernel reads this input in another memory layout of
  // the same logical shape. Three layouts are defined:
  //   "OHWI": a rank-4 FP32 OIHW weight stored as [out][kh][kw][in];
  //   "NK":   a rank-2 [K][N] GEMM weight stored transposed, as [N][K];
  //   "T":    any rank-2 constant stored transposed (the same copy as "NK",
  //           named for a weight that is [N][K] already, e.g. a Gemm with
  //           transB = 1, read by a kernel that wants [K][N]).
  // The input must be a constant; the engine keeps the re-laid-out copy
  // beside the original.
  std::string layout;
};

// The layouts an input argument may request.
inline bool IsInputLayout(const std::string& layout) {
  return layout == "OHWI" || layout == "NK" || layout == "T";
}

// Name of the re-laid-out copy of constant `name` in `layout`.
inline std::string LaidOutConstantName(const std::string& name, const std::string& layout) {
  return name + "#" + layout;
}

struct KernelArgumentSpec {
  std::string name;
  std::string type;
  KernelArgumentSource source;
};

enum class KernelConstraintKind {
  kAttributeInt64Equals,
  kInputCountEquals,
  kTensorRankEquals,
  kTensorDimAtMost,  // "dim_le": shape[axis] of an input/output <= value
  // "tensor_bytes_le": every input and output the kernel binds holds at most
  // value bytes (kernels that address tensors through 32-bit buffer
  // resources declare 2^31 - 1).
  kTensorBytesAtMost,
};

// Declarative constraint; packs cannot inject code.
struct KernelConstraint {
  KernelConstraintKind kind{KernelConstraintKind::kInputCountEquals};
  std::string attribute_name;
  bool tensor_is_output{false};
  int tensor_index{0};
  int tensor_axis{0};
  int64_t expected{0};
  int64_t default_value{0};
};

enum class GridExpressionKind {
  kLiteral,
  kInputDim,
  kOutputDim,
  kInputNumElements,
  kOutputNumElements,
  kVariantMeta,
  kCeilDiv,
  kMultiply,
};

// Bounded launch-grid expression tree (depth <= 8). Only these node kinds
// exist; anything else in a manifest is rejected at load time.
struct GridExpression {
  GridExpressionKind kind{GridExpressionKind::kLiteral};
  int64_t literal{1};
  int tensor_index{0};
  int axis{0};
  std::string meta_name;
  std::vector<GridExpression> operands;
};

struct KernelArtifact {
  std::string pack_name;
  int pack_version{0};
  std::string generator_version;
  // Schema field kept for compatibility; holds the generator toolchain id.
  std::string triton_version;
  int abi_schema_version{0};
  std::string kernel_id;
  std::string op_type;
  int kernel_version{0};
  std::string variant_id;
  bool is_default{false};
  std::string symbol;
  std::filesystem::path binary_path;
  std::string binary_format;
  std::string sha256;
  std::string dtype;
  std::string layout;
  std::string target_arch;
  int min_compute_capability{950};
  int num_warps{4};
  int num_stages{1};
  int shared_memory_bytes{0};
  // Device scratch the kernel needs through its first runtime_reserved
  // argument (0: the argument is null, as in the reference ABI).
  std::int64_t runtime_scratch_bytes{0};
  std::array<GridExpression, 3> launch_grid{};
  std::unordered_map<std::string, int64_t> launch_meta;
  // ABI v1 compatibility: grid = ceil(output_numel / grid_divisor).
  int grid_divisor{1};
  std::vector<KernelArgumentSpec> arguments;
  std::vector<KernelConstraint> constraints;
  // Threads per workgroup on a wave64 device.
  int block_threads() const { return num_warps * 64; }
  std::string identity() const { return pack_name + ":" + kernel_id + ":" + variant_id; }
};

// Immutable, validated view over one or more packs (pack.json or its folder).
class ArtifactRepository {
 public:
  Status Load(const std::vector<std::string>& paths);
  const std::vector<KernelArtifact>* Find(const std::string& op_type) const;
  const std::vector<KernelArtifact>& artifacts() const { return artifacts_; }
  const std::string& repository_hash() const { return repository_hash_; }

 private:
  std::vector<KernelArtifact> artifacts_;
  std::unordered_map<std::string, std::vector<KernelArtifact>> by_op_type_;
  std::string repository_hash_;
};

// op/dtype/layout/architecture filter shared by every lowering.
class KernelCatalog {
 public:
  explicit KernelCatalog(const ArtifactRepository* repository) : repository_(repository) {}
  std::vector<const KernelArtifact*> Query(const std::string& op_type,
                                           const std::string& dtype,
                                           const std::string& layout,
                                           int compute_capability) const;

 private:
  const ArtifactRepository* repository_{nullptr};
};

// FIPS 180-4 SHA-256 of `data`, lowercase hex.
std::string Sha256Hex(const std::string& data);

}  // namespace cutriton
