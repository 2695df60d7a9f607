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

class MemoryPlanner {
 public:
  // 256-byte aligned best-fit placement with lifetime-based reuse; Flatten
  // outputs alias their input.
  Status Plan(const Graph& graph, MemoryPlan* plan) const;
};

}  // namespace cutriton
