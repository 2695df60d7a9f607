// Tuning decisions: what identifies one, and where it is kept.
#pragma once

#include <optional>
#include <string>

#include "cutriton/core/status.h"
#include "cutriton/ir/graph.h"
#include "cutriton/runtime/executable_plan.h"

namespace cutriton {

// A 16-hex-digit key for the tuning decision of `op` (node `node` of
// `graph`) on device `device_id`: it changes whenever anything the choice
// depends on changes - the op and its tensors' dtypes, layouts and shapes,
// its attributes, the set of candidates and the exact code of each (pack,
// kernel, variant, generator and toolchain versions, code SHA-256), and the
// device (architecture, compute units, UUID, driver and runtime versions).
std::string TuningDecisionKey(const PlanOp& op, const Node& node, const Graph& graph, int device_id);

// One JSON file per decision, "<folder>/<key>.json":
//   {"schema_version": 1, "tuning_key": key, "candidate_id": id, "median_ms": t}
// the record format of the reference's tuning cache (src/runtime/engine.cpp:
// 297-335). Files are published by rename, so a reader never sees a partial
// record.
class TuningStore {
 public:
  explicit TuningStore(std::string folder) : folder_(std::move(folder)) {}
  // The recorded candidate id, or nothing when there is no valid record.
  std::optional<std::string> Lookup(const std::string& key) const;
  Status Record(const std::string& key, const std::string& candidate_id, double median_ms) const;

 private:
  std::string PathOf(const std::string& key) const { return folder_ + "/" + key + ".json"; }
  std::string folder_;
};

}  // namespace cutriton
