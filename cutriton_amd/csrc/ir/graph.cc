// Graph and Model: the value table, node list and host constants.
//
// Node order. TopologicalSort yields the dependency order that stays closest
// to the order in which nodes were added: among the nodes whose producers have
// all been placed, the one added first goes next (a Kahn walk over a min-heap
// of positions). A graph that is already in dependency order is left exactly as
// it is, and independent branches keep their relative order. Error kinds follow
// the reference's graph (src/ir/graph.cpp): an empty name is InvalidArgument, a
// duplicate value AlreadyExists, an undefined output NotFound, a cycle
// InvalidArgument.
#include "cutriton/ir/graph.h"

#include <algorithm>
#include <functional>
#include <queue>

#include "cutriton/core/buffer.h"

namespace cutriton {

Status Graph::AddValue(ValueDesc value) {
  if (value.name.empty()) return Status::InvalidArgument("value name must not be empty");
  auto [slot, fresh] = values_.try_emplace(value.name);
  if (!fresh) return Status::AlreadyExists("value already exists: " + value.name);
  slot->second = std::move(value);
  return Status::OK();
}

Status Graph::AddInput(std::string name, TensorDesc desc) {
  if (name.empty()) return Status::InvalidArgument("input name must not be empty");
  ValueDesc& value = values_[name];
  value.name = name;
  value.tensor = std::move(desc);
  inputs_.push_back(std::move(name));
  return Status::OK();
}

Status Graph::AddOutput(std::string name) {
  if (FindValue(name) == nullptr) return Status::NotFound("graph output is not a value: " + name);
  outputs_.push_back(std::move(name));
  return Status::OK();
}

Status Graph::AddNode(Node node) {
  if (node.name().empty()) return Status::InvalidArgument("node name must not be empty");
  if (node.op_type().empty()) return Status::InvalidArgument("node op_type must not be empty");
  for (const auto* names : {&node.outputs(), &node.inputs()}) {
    for (const auto& name : *names) CUTRITON_RETURN_IF_ERROR(EnsureValue(name));
  }
  node.set_id(static_cast<int>(nodes_.size()));
  nodes_.push_back(std::move(node));
  return Status::OK();
}

const ValueDesc* Graph::FindValue(const std::string& name) const {
  const auto found = values_.find(name);
  return found == values_.end() ? nullptr : &found->second;
}

ValueDesc* Graph::MutableValue(const std::string& name) {
  const auto found = values_.find(name);
  return found == values_.end() ? nullptr : &found->second;
}

Status Graph::SetValueDesc(const std::string& name, TensorDesc desc) {
  ValueDesc* value = MutableValue(name);
  if (value == nullptr) return Status::NotFound("value is not defined: " + name);
  value->tensor = std::move(desc);
  return Status::OK();
}

Status Graph::EnsureValue(std::string name, TensorDesc desc) {
  if (name.empty()) return Status::InvalidArgument("value name must not be empty");
  auto [slot, fresh] = values_.try_emplace(name);
  if (fresh) slot->second = ValueDesc{std::move(name), std::move(desc), false};
  return Status::OK();
}

std::unordered_map<std::string, int> Graph::BuildProducerMap() const {
  std::unordered_map<std::string, int> producer_of;
  for (const auto& node : nodes_) {
    for (const auto& name : node.outputs()) producer_of[name] = node.id();
  }
  return producer_of;
}

std::unordered_map<std::string, std::vector<int>> Graph::BuildConsumerMap() const {
  std::unordered_map<std::string, std::vector<int>> readers;
  for (const auto& node : nodes_) {
    for (const auto& name : node.inputs()) readers[name].push_back(node.id());
  }
  return readers;
}

Status Graph::TopologicalSort() {
  const std::size_t count = nodes_.size();
  const auto producer_of = BuildProducerMap();
  // Per node: the distinct other nodes it reads from (positions), and the
  // reverse edges used to release readers once a producer is placed.
  std::vector<int> unplaced_producers(count, 0);
  std::vector<std::vector<int>> readers(count);
  for (std::size_t position = 0; position < count; ++position) {
    std::vector<int> sources;
    for (const auto& name : nodes_[position].inputs()) {
      const auto found = producer_of.find(name);
      if (found != producer_of.end() && found->second != static_cast<int>(position)) {
        sources.push_back(found->second);
      }
    }
    std::sort(sources.begin(), sources.end());
    sources.erase(std::unique(sources.begin(), sources.end()), sources.end());
    unplaced_producers[position] = static_cast<int>(sources.size());
    for (const int source : sources) readers[static_cast<std::size_t>(source)].push_back(static_cast<int>(position));
  }
  std::priority_queue<int, std::vector<int>, std::greater<int>> ready;
  for (std::size_t position = 0; position < count; ++position) {
    if (unplaced_producers[position] == 0) ready.push(static_cast<int>(position));
  }
  std::vector<int> order;
  order.reserve(count);
  while (!ready.empty()) {
    const int position = ready.top();
    ready.pop();
    order.push_back(position);
    for (const int reader : readers[static_cast<std::size_t>(position)]) {
      if (--unplaced_producers[static_cast<std::size_t>(reader)] == 0) ready.push(reader);
    }
  }
  if (order.size() != count) {
    std::string stuck;  // nodes on or behind a cycle were never released
    for (std::size_t position = 0; position < count; ++position) {
      if (unplaced_producers[position] > 0) stuck += (stuck.empty() ? "" : ", ") + nodes_[position].name();
    }
    return Status::InvalidArgument("graph contains a cycle through: " + stuck);
  }
  std::vector<Node> placed;
  placed.reserve(count);
  for (const int position : order) placed.push_back(std::move(nodes_[static_cast<std::size_t>(position)]));
  nodes_ = std::move(placed);
  RenumberNodes();
  return Status::OK();
}

Status Graph::RemoveNodes(const std::vector<int>& node_ids) {
  std::vector<int> doomed = node_ids;
  std::sort(doomed.begin(), doomed.end());
  const auto survives = [&](const Node& node) { return !std::binary_search(doomed.begin(), doomed.end(), node.id()); };
  nodes_.erase(std::stable_partition(nodes_.begin(), nodes_.end(), survives), nodes_.end());
  RenumberNodes();
  return Status::OK();
}

void Graph::RenumberNodes() {
  int id = 0;
  for (auto& node : nodes_) node.set_id(id++);
}

std::vector<int64_t> GetIntListAttribute(const Node& node, const std::string& key,
                                         std::vector<int64_t> fallback) {
  return node.GetAttribute<std::vector<int64_t>>(key).value_or(std::move(fallback));
}

int64_t GetIntAttribute(const Node& node, const std::string& key, int64_t fallback) {
  return node.GetAttribute<int64_t>(key).value_or(fallback);
}

namespace {

// A model constant is host data that covers its description.
Status CheckHostConstant(const std::string& name, const Tensor& tensor) {
  if (name.empty()) return Status::InvalidArgument("constant name must not be empty");
  CUTRITON_RETURN_IF_ERROR(tensor.desc().Validate());
  const std::shared_ptr<Buffer>& buffer = tensor.buffer();
  if (buffer == nullptr || buffer->empty()) return Status::InvalidArgument("constant has no Buffer: " + name);
  const bool on_host = buffer->device_type() == DeviceType::kCPU && tensor.desc().device_type == DeviceType::kCPU;
  if (!on_host) return Status::InvalidArgument("model constants must live in host memory: " + name);
  const std::size_t end = tensor.byte_offset() + tensor.desc().ByteSize();
  if (tensor.byte_offset() > buffer->size_bytes() || end > buffer->size_bytes()) {
    return Status::InvalidArgument("constant Buffer is too small: " + name);
  }
  return Status::OK();
}

}  // namespace

Status Model::AddConstant(std::string name, Tensor tensor) {
  CUTRITON_RETURN_IF_ERROR(CheckHostConstant(name, tensor));
  ValueDesc* value = graph_.MutableValue(name);
  if (constants_.count(name) != 0 || (value != nullptr && value->is_constant)) {
    return Status::AlreadyExists("constant already exists: " + name);
  }
  // A name that nodes already read (declared before its data) becomes the
  // constant in place.
  if (value == nullptr) {
    CUTRITON_RETURN_IF_ERROR(graph_.AddValue(ValueDesc{name, tensor.desc(), true}));
  } else {
    value->tensor = tensor.desc();
    value->is_constant = true;
  }
  constants_.emplace(std::move(name), std::move(tensor));
  return Status::OK();
}

}  // namespace cutriton
