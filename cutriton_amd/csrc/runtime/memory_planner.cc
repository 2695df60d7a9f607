// Workspace planner. Behaviour follows reference
// src/runtime/memory_planner.cpp:29-169: last-use lifetimes (graph outputs
// live to the end, Flatten aliases extend their source), release before each
// node, best-fit reuse of freed 256-byte-aligned blocks, else bump allocation.
#include "cutriton/runtime/memory_planner.h"

#include <algorithm>
#include <unordered_map>
#include <unordered_set>

namespace cutriton {
namespace {

constexpr std::size_t kAlignment = 256;

std::size_t AlignUp(std::size_t value) { return (value + kAlignment - 1) & ~(kAlignment - 1); }

struct Block {
  std::size_t offset{0};
  std::size_t size{0};
};

}  // namespace

Status MemoryPlanner::Plan(const Graph& graph, MemoryPlan* plan) const {
  if (plan == nullptr) return Status::InvalidArgument("MemoryPlan output pointer is null");
  *plan = MemoryPlan{};

  std::unordered_set<std::string> external(graph.inputs().begin(), graph.inputs().end());
  external.insert(graph.outputs().begin(), graph.outputs().end());

  std::unordered_map<std::string, std::string> alias_source;
  for (const auto& node : graph.nodes()) {
    if (node.op_type() == "Flatten" && node.inputs().size() == 1 && node.outputs().size() == 1) {
      alias_source[node.outputs()[0]] = node.inputs()[0];
    }
  }

  std::unordered_map<std::string, int> last_use;
  for (std::size_t i = 0; i < graph.nodes().size(); ++i) {
    const Node& node = graph.nodes()[i];
    for (const auto& name : node.inputs()) last_use[name] = static_cast<int>(i);
    for (const auto& name : node.outputs()) last_use.emplace(name, static_cast<int>(i));
  }
  const int end_of_graph = static_cast<int>(graph.nodes().size());
  for (const auto& name : graph.outputs()) last_use[name] = end_of_graph;
  for (const auto& alias : alias_source) {
    const auto use = last_use.find(alias.first);
    if (use != last_use.end()) {
      int& source_use = last_use[alias.second];
      source_use = std::max(source_use, use->second);
    }
  }

  std::vector<Block> free_blocks;
  std::vector<std::pair<std::string, Block>> live;
  std::unordered_map<std::string, Allocation> placed;
  std::size_t high_water = 0;

  for (std::size_t i = 0; i < graph.nodes().size(); ++i) {
    // Release every block whose value was last read before this node.
    for (auto it = live.begin(); it != live.end();) {
      const auto use = last_use.find(it->first);
      if (use != last_use.end() && use->second < static_cast<int>(i)) {
        free_blocks.push_back(it->second);
        it = live.erase(it);
      } else {
        ++it;
      }
    }
    for (const auto& name : graph.nodes()[i].outputs()) {
      if (external.count(name) != 0) continue;
      const auto alias = alias_source.find(name);
      if (alias != alias_source.end()) {
        const auto source = placed.find(alias->second);
        Allocation allocation;
        if (source != placed.end()) {
          allocation = source->second;
        } else if (external.count(alias->second) != 0) {
          const ValueDesc* source_value = graph.FindValue(alias->second);
          if (source_value == nullptr) {
            return Status::Internal("Flatten alias source is unknown: " + alias->second);
          }
          allocation.size_bytes = source_value->tensor.ByteSize();
        } else {
          return Status::Internal("Flatten alias source has no allocation: " + alias->second);
        }
        allocation.value_name = name;
        allocation.alias_of = alias->second;
        allocation.reused = true;
        const ValueDesc* value = graph.FindValue(name);
        if (value == nullptr || value->tensor.ByteSize() != allocation.size_bytes) {
          return Status::ShapeError("Flatten alias changes the byte size of " + name);
        }
        plan->allocations.push_back(allocation);
        placed.emplace(name, allocation);
        continue;
      }
      const ValueDesc* value = graph.FindValue(name);
      if (value == nullptr || value->is_constant) continue;
      const std::size_t bytes = value->tensor.ByteSize();
      if (bytes == 0) return Status::ShapeError("cannot plan a dynamically sized value: " + name);
      const std::size_t reserved = AlignUp(bytes);
      auto best = free_blocks.end();
      for (auto it = free_blocks.begin(); it != free_blocks.end(); ++it) {
        if (it->size >= reserved && (best == free_blocks.end() || it->size < best->size)) best = it;
      }
      Allocation allocation;
      allocation.value_name = name;
      allocation.size_bytes = bytes;
      if (best != free_blocks.end()) {
        allocation.offset = best->offset;
        allocation.reused = true;
        if (best->size > reserved) {
          best->offset += reserved;
          best->size -= reserved;
        } else {
          free_blocks.erase(best);
        }
      } else {
        allocation.offset = AlignUp(high_water);
        high_water = allocation.offset + reserved;
      }
      plan->allocations.push_back(allocation);
      placed.emplace(name, allocation);
      live.push_back({name, Block{allocation.offset, reserved}});
    }
  }
  plan->workspace_size_bytes = AlignUp(high_water);
  return Status::OK();
}

}  // namespace cutriton
