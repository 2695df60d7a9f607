// Single-workspace planner for intermediates.
// Mirrors include/cutriton/runtime/memory_planner.h:13-29 of the reference.
#pragma once

#include <cstddef>
#include <string>
#include <vector>

#include "cutriton/core/status.h"
#include "cutriton/ir/graph.h"

namespace cutriton {

struct Allocation {
  std::string value_name;
  std::size_t size_bytes{0};
  std::size_t offset{0};
  bool reused{false};
  std::string alias_of;
};

struct MemoryPlan {
  std::size_t workspace_size_bytes{0};
  std::vector<Allocation> allocations;
};

// Workspace for the temporaries of one plan step (an execution candidate's
// private intermediates): every name in `names` shares one block of
// `size_bytes`, live during step `step` only. Candidates of one op never run
// at the same time, so their temporaries of one slot share a request.
struct WorkspaceRequest {
  std::vector<std::string> names;
  std::size_t size_bytes{0};
  int step{0};
};

class MemoryPlanner {
 public:
  // 256-byte aligned blocks for every intermediate value; blocks whose
  // lifetimes do not overlap share bytes; Flatten outputs alias their input.
  Status Plan(const Graph& graph, MemoryPlan* plan) const;
  // As above, plus blocks for step-private temporaries.
  Status Plan(const Graph& graph, const std::vector<WorkspaceRequest>& temporaries, MemoryPlan* plan) const;
};

}  // namespace cutriton
