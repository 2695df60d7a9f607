// Engine (shared read-only state) and ExecutionContext (one run session).
// Mirrors include/cutriton/runtime/engine.h:20-93 of the reference; the
// device side is HIP: hipStream, hipEvent pairs and a hipGraph LRU.
#pragma once

#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "cutriton/backend/backend.h"
#include "cutriton/core/buffer.h"
#include "cutriton/core/status.h"
#include "cutriton/runtime/executable_plan.h"
#include "cutriton/runtime/profiler.h"

namespace cutriton {

class ExecutionContext;
class EngineState;

class Engine {
 public:
  explicit Engine(ExecutablePlan plan);
  const ExecutablePlan& plan() const;
  // Each context owns its stream, workspace, profiler and graph cache.
  std::unique_ptr<ExecutionContext> CreateExecutionContext() const;

 private:
  std::shared_ptr<EngineState> state_;
};

// Not thread-safe; at most one pending run at a time.
class ExecutionContext {
 public:
  explicit ExecutionContext(std::shared_ptr<EngineState> state);
  ~ExecutionContext();

  // Name, shape, dtype, layout, device and buffer extent must match the plan.
  Status BindInput(const std::string& name, Tensor tensor);
  Status BindOutput(const std::string& name, Tensor tensor);
  Status SelectShapeProfile(const std::string& name);
  Status SetInputShape(const std::string& name, std::vector<int64_t> shape);
  Status ResolveShapes();
  const TensorDesc* GetResolvedTensorDesc(const std::string& name) const;
  // RunAsync(nullptr) followed by Synchronize().
  Status Run();
  // Enqueues on `stream` (a hipStream_t), or on the context's own stream.
  Status RunAsync(void* stream);
  // RunAsync for callers that cannot allocate device memory (no counterpart
  // in the reference). It enqueues the op sequence on `stream` (non-null)
  // without graph capture and without per-op events, binding the kernels'
  // runtime scratch to the library's static device array; it calls no
  // hipMalloc, loads no code object and times no candidate. What it needs
  // must already exist: constants uploaded, a workspace of the profile's
  // size, the code objects of the selected kernels loaded (one RunAsync of
  // the context, at any shape of its profile, provides all three) and
  // tuning choices that resolve without timing. Otherwise it fails with
  // RuntimeError and enqueues nothing. Runs of this kind that overlap on one
  // GPU share the static array and race.
  Status RunAsyncWithoutAllocation(void* stream);
  Status Synchronize();

  const Profiler& profiler() const { return profiler_; }
  std::size_t cached_cuda_graph_count() const;
  std::size_t loaded_cuda_module_count() const;
  const std::unordered_map<std::string, Tensor>& tensors() const { return tensors_; }
  // Index of the chosen candidate per plan op (valid after the first run).
  const std::vector<std::size_t>& selected_candidates() const { return selected_candidates_; }
  // Kernel time of plan op `op_index` as selected: one warm-up launch, then
  // `iterations` back-to-back launches between one hipEvent pair on `stream`
  // (the context's own stream when null), so that launch latency overlaps
  // execution. Needs a completed run; the op reads and rewrites its bound
  // tensors. Ops without a kernel (Flatten views) report 0.
  Status TimeOp(std::size_t op_index, int iterations, void* stream, double* ms_per_launch);

 private:
  // What a binding or shape change invalidates, from least to most.
  enum class Stale { kBindings, kShapes, kProfile };
  void Invalidate(Stale what);
  // The "may_*" flags are false on the allocation-free path: a step that
  // would allocate device memory, load a code object or time candidates
  // fails instead.
  Status PrepareKernels(bool may_load);
  Status PrepareTuning(bool may_time);
  Status PrepareTensors(bool may_allocate);
  Status ValidateBindings() const;
  Status EnqueueOps(void* stream, bool capture, void* scratch, std::size_t scratch_bytes);
  Status CaptureGraph(void* stream, void** exec);
  void InvalidateHipGraph();
  const Graph& ActiveGraph() const;
  const MemoryPlan& ActiveMemoryPlan() const;
  std::size_t RuntimeScratchNeed() const;

  std::shared_ptr<EngineState> state_;
  bool kernels_prepared_{false};
  bool tensors_prepared_{false};
  bool run_pending_{false};
  bool tuning_prepared_{false};
  std::vector<std::size_t> selected_candidates_;
  int selected_profile_{-1};
  std::unordered_map<std::string, std::vector<int64_t>> input_shapes_;
  Graph resolved_graph_;
  bool shapes_resolved_{false};
  std::vector<std::vector<std::unique_ptr<OpKernel>>> kernels_;
  std::unordered_map<std::string, Tensor> tensors_;
  // Caller-bound graph inputs and outputs (the rest of tensors_ is derived).
  std::unordered_map<std::string, Tensor> bound_;
  std::shared_ptr<Buffer> workspace_;
  // Zero-initialised device scratch for kernels that declare one.
  std::shared_ptr<Buffer> runtime_scratch_;
  Profiler profiler_;
  // HIP stream/event/graph state; its type lives in the implementation.
  void* hip_state_{nullptr};
  // Stream of a pending allocation-free run (Synchronize waits on it).
  void* unmanaged_stream_{nullptr};
};

}  // namespace cutriton
