// Backends, kernels and the registry.
// Mirrors include/cutriton/backend/backend.h:23-104 of the reference. The
// artifact backend of this build is "hip_gfx950": it lowers nodes to
// KernelInvocations over gfx950 code objects launched with
// hipModuleLaunchKernel.
#pragma once

#include <memory>
#include <shared_mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "cutriton/backend/kernel_artifact.h"
#include "cutriton/backend/kernel_invocation.h"
#include "cutriton/core/device.h"
#include "cutriton/core/status.h"
#include "cutriton/core/tensor.h"
#include "cutriton/ir/graph.h"

namespace cutriton {

class Profiler;
class HipModuleCache;

// Name of the built-in artifact backend.
inline constexpr const char* kHipBackendName = "hip_gfx950";

struct BackendOptions {
  Device device{};
  std::vector<std::string> kernel_artifact_paths;
  // Single-pack spelling, used when kernel_artifact_paths is empty.
  std::string kernel_artifact_dir;
};

struct LoweringContext {
  const Graph* graph{nullptr};
  const BackendOptions* options{nullptr};
  const ArtifactRepository* artifacts{nullptr};
  const KernelCatalog* catalog{nullptr};
};

// Valid only for the duration of OpKernel::Compute. `stream` is a
// hipStream_t for the HIP backend. `runtime_scratch` is the execution
// context's zero-initialised device scratch (runtime_scratch_bytes long),
// bound to the first runtime_reserved argument of kernels that declare a
// scratch size; such kernels leave it zeroed again when they finish.
struct KernelContext {
  const Node* node{nullptr};
  std::unordered_map<std::string, Tensor>* tensors{nullptr};
  void* stream{nullptr};
  Profiler* profiler{nullptr};
  void* runtime_scratch{nullptr};
  std::size_t runtime_scratch_bytes{0};
};

class OpKernel {
 public:
  virtual ~OpKernel() = default;
  virtual const char* backend_name() const = 0;
  virtual const char* op_type() const = 0;
  virtual Status Compute(KernelContext* context) = 0;
};

class Backend {
 public:
  virtual ~Backend() = default;
  virtual const char* name() const = 0;
  // Full check of dtype, shape, layout, attributes, device and artifacts.
  virtual Status CheckSupport(const Node& node, const Graph& graph,
                              const BackendOptions& options) const = 0;
  // Node -> execution candidates. The base version emits one legacy
  // candidate backed by CreateKernel (non-artifact backends, tests).
  virtual Status Lower(const Node& node, const LoweringContext& context,
                       std::vector<ExecutionCandidate>* candidates) const;
  virtual Status CreateKernel(const Node& node, const Graph& graph,
                              const BackendOptions& options,
                              std::unique_ptr<OpKernel>* kernel) const = 0;
};

class KernelRegistry {
 public:
  static KernelRegistry& Global();
  Status RegisterBackend(std::shared_ptr<Backend> backend);
  std::shared_ptr<Backend> GetBackend(const std::string& name) const;
  std::vector<std::string> AvailableBackends() const;
  void ClearForTests();

 private:
  mutable std::shared_mutex mutex_;
  std::unordered_map<std::string, std::shared_ptr<Backend>> backends_;
};

// "cpu_reference": always Unsupported (the reference's behaviour).
std::shared_ptr<Backend> CreateCpuReferenceBackend();
// "hip_gfx950": the artifact backend of this build.
std::shared_ptr<Backend> CreateHipBackend();
Status RegisterBuiltinBackends();

// Checks the size-dependent constraints (tensor_bytes_le) of every kernel
// step of `candidate` against the value shapes of `graph` (a graph resolved at
// some shape-profile point). Candidate temporaries are sized like their
// "like" value. Unsupported names the first tensor that is too large.
Status CheckCandidateShapes(const ExecutionCandidate& candidate, const Graph& graph);

// Numeric architecture of a HIP device (950 for gfx950), used against
// min_compute_capability; `arch_name` receives e.g. "gfx950".
Status DeviceArchitecture(int device_id, int* numeric_arch, std::string* arch_name);

// Module/function cache keyed by code-object SHA-256 (and SHA+symbol).
Status CreateHipModuleCache(int device_id, std::shared_ptr<HipModuleCache>* cache);
Status CreateInvocationKernel(const KernelInvocation& invocation, int device_id,
                              std::shared_ptr<HipModuleCache> cache,
                              std::unique_ptr<OpKernel>* kernel);
std::size_t LoadedModuleCount(const std::shared_ptr<HipModuleCache>& cache);
// Whether the code object of `artifact` is loaded (CreateInvocationKernel
// then loads nothing).
bool CodeObjectLoaded(const std::shared_ptr<HipModuleCache>& cache, const KernelArtifact& artifact);

}  // namespace cutriton
