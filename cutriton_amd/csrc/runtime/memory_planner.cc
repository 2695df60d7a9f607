// Workspace planning for intermediate tensors.
//
// Every intermediate (a node output that is neither a graph input, a graph
// output nor a constant) gets a block of the one workspace allocation. A
// block lives from the node that writes it to the last node that reads it,
// where a Flatten output counts as a read of its input (Flatten is a view: it
// shares its input's block, and keeps it alive as long as the view is read).
// Execution-candidate temporaries are blocks that live for their op only.
//
// Placement is greedy by size (Pisarchyk and Lee, "Efficient Memory
// Management for Deep Neural Net Inference", 2020): blocks are placed from the
// largest down, each at the lowest 256-byte aligned offset where it overlaps
// no already placed block whose lifetime overlaps its own. Large activations
// therefore claim the bottom of the workspace first and small ones fill the
// gaps between them. Allocations are reported in the order the values are
// produced; `reused` marks a block whose bytes an earlier-born value held.
//
// The reference plans with a best-fit free list in node order
// (src/runtime/memory_planner.cpp); both satisfy its tests
// (tests/cpp/test_core.cpp:236-272): a chain of three 17-float values is
// placed at 0, 256 and 0 (the third reusing the first), and a Flatten output
// aliases its input at the same offset.
#include "cutriton/runtime/memory_planner.h"

#include <algorithm>
#include <unordered_map>
#include <unordered_set>

namespace cutriton {
namespace {

constexpr std::size_t kAlignment = 256;

std::size_t RoundUp(std::size_t bytes) { return (bytes + kAlignment - 1) / kAlignment * kAlignment; }

struct Block {
  std::size_t bytes{0};     // aligned size
  int first{0};             // step that writes it
  int last{0};              // last step that reads it
  std::size_t offset{0};
  bool reused{false};
  std::size_t order{0};     // production order (ties in placement)
};

bool LifetimesOverlap(const Block& a, const Block& b) { return a.first <= b.last && b.first <= a.last; }

// Places `blocks` (greedy by size) and returns the workspace size.
std::size_t Place(std::vector<Block>* blocks) {
  std::vector<std::size_t> by_size(blocks->size());
  for (std::size_t i = 0; i < by_size.size(); ++i) by_size[i] = i;
  std::stable_sort(by_size.begin(), by_size.end(), [&](std::size_t a, std::size_t b) {
    const Block& x = (*blocks)[a];
    const Block& y = (*blocks)[b];
    return x.bytes != y.bytes ? x.bytes > y.bytes : x.order < y.order;
  });
  std::vector<std::size_t> placed;
  std::size_t high_water = 0;
  for (const std::size_t index : by_size) {
    Block& block = (*blocks)[index];
    // Address ranges taken by live-at-the-same-time blocks, lowest first.
    std::vector<std::pair<std::size_t, std::size_t>> taken;
    for (const std::size_t other : placed) {
      const Block& o = (*blocks)[other];
      if (LifetimesOverlap(block, o)) taken.emplace_back(o.offset, o.offset + o.bytes);
    }
    std::sort(taken.begin(), taken.end());
    std::size_t candidate = 0;
    for (const auto& [begin, end] : taken) {
      if (candidate + block.bytes <= begin) break;  // fits in the gap below this range
      candidate = std::max(candidate, end);
    }
    block.offset = candidate;
    high_water = std::max(high_water, candidate + block.bytes);
    placed.push_back(index);
  }
  // A block is reused when a value produced before it occupied any of its bytes.
  for (Block& block : *blocks) {
    for (const Block& other : *blocks) {
      if (other.order < block.order && other.last < block.first && other.offset < block.offset + block.bytes &&
          block.offset < other.offset + other.bytes) {
        block.reused = true;
        break;
      }
    }
  }
  return high_water;
}

}  // namespace

Status MemoryPlanner::Plan(const Graph& graph, MemoryPlan* plan) const { return Plan(graph, {}, plan); }

Status MemoryPlanner::Plan(const Graph& graph, const std::vector<WorkspaceRequest>& temporaries,
                           MemoryPlan* plan) const {
  if (plan == nullptr) return Status::InvalidArgument("MemoryPlan output pointer is null");
  *plan = MemoryPlan{};
  std::unordered_set<std::string> bound_by_caller(graph.inputs().begin(), graph.inputs().end());
  bound_by_caller.insert(graph.outputs().begin(), graph.outputs().end());

  // Views: a Flatten output resolves to the block of the value it flattens.
  std::unordered_map<std::string, std::string> view_of;
  for (const auto& node : graph.nodes()) {
    if (node.op_type() == "Flatten" && node.inputs().size() == 1 && node.outputs().size() == 1 &&
        bound_by_caller.count(node.outputs()[0]) == 0) {
      view_of[node.outputs()[0]] = node.inputs()[0];
    }
  }
  auto storage_of = [&](std::string name) {
    for (auto found = view_of.find(name); found != view_of.end(); found = view_of.find(name)) name = found->second;
    return name;
  };

  // One block per planned value, in production order.
  std::vector<Block> blocks;
  std::vector<std::string> block_value;
  std::unordered_map<std::string, std::size_t> block_of;
  struct Produced {
    std::string name;
    bool view{false};
  };
  std::vector<Produced> produced;
  const int steps = static_cast<int>(graph.nodes().size());
  for (int step = 0; step < steps; ++step) {
    const Node& node = graph.nodes()[static_cast<std::size_t>(step)];
    for (const auto& name : node.outputs()) {
      if (bound_by_caller.count(name) != 0) continue;
      if (view_of.count(name) != 0) {
        produced.push_back({name, true});
        continue;
      }
      const ValueDesc* value = graph.FindValue(name);
      if (value == nullptr || value->is_constant) continue;
      if (value->tensor.ByteSize() == 0) {
        return Status::ShapeError("cannot plan memory for a dynamically sized value: " + name);
      }
      Block block;
      block.bytes = RoundUp(value->tensor.ByteSize());
      block.first = block.last = step;
      block.order = blocks.size();
      block_of[name] = blocks.size();
      blocks.push_back(block);
      block_value.push_back(name);
      produced.push_back({name, false});
    }
    for (const auto& name : node.inputs()) {
      const auto found = block_of.find(storage_of(name));
      if (found != block_of.end()) blocks[found->second].last = std::max(blocks[found->second].last, step);
    }
  }
  const std::size_t value_blocks = blocks.size();
  for (const auto& request : temporaries) {
    if (request.size_bytes == 0 || request.names.empty()) {
      return Status::ShapeError("a candidate temporary has no concrete size");
    }
    Block block;
    block.bytes = RoundUp(request.size_bytes);
    block.first = block.last = request.step;
    block.order = blocks.size();
    blocks.push_back(block);
  }
  plan->workspace_size_bytes = RoundUp(Place(&blocks));

  for (const auto& item : produced) {
    const ValueDesc* value = graph.FindValue(item.name);
    if (!item.view) {
      const Block& block = blocks[block_of.at(item.name)];
      plan->allocations.push_back(
          Allocation{item.name, value->tensor.ByteSize(), block.offset, block.reused, ""});
      continue;
    }
    const std::string& source = view_of.at(item.name);
    const auto root = block_of.find(storage_of(item.name));
    const ValueDesc* source_value = graph.FindValue(source);
    if (root == block_of.end() || source_value == nullptr) {
      return Status::Internal("Flatten view has no planned source: " + item.name);
    }
    if (value == nullptr || value->tensor.ByteSize() != source_value->tensor.ByteSize()) {
      return Status::ShapeError("Flatten view changes the byte size of " + item.name);
    }
    plan->allocations.push_back(
        Allocation{item.name, value->tensor.ByteSize(), blocks[root->second].offset, true, source});
  }
  for (std::size_t i = 0; i < temporaries.size(); ++i) {
    const Block& block = blocks[value_blocks + i];
    for (const auto& name : temporaries[i].names) {
      plan->allocations.push_back(Allocation{name, temporaries[i].size_bytes, block.offset, block.reused, ""});
    }
  }
  return Status::OK();
}

}  // namespace cutriton
