#include "runtime/tuning_store.h"

#include <cstdint>
#include <cstdio>
#include <filesystem>
#include <fstream>
#include <map>
#include <sstream>
#include <type_traits>
#include <variant>

#include "backend/json.h"
#include "cutriton_hip_runtime.h"

namespace cutriton {
namespace {

// FNV-1a over a sequence of fields. Every field is length-prefixed, so no
// two different field sequences hash the same bytes.
class Fingerprint {
 public:
  Fingerprint& Field(const std::string& text) {
    Mix(std::to_string(text.size()));
    Mix(":");
    Mix(text);
    return *this;
  }
  Fingerprint& Field(int64_t value) { return Field(std::to_string(value)); }
  std::string Hex() const {
    char out[17];
    std::snprintf(out, sizeof(out), "%016llx", static_cast<unsigned long long>(state_));
    return out;
  }

 private:
  void Mix(const std::string& bytes) {
    for (const unsigned char byte : bytes) {
      state_ ^= byte;
      state_ *= 0x100000001b3ull;  // 64-bit FNV prime
    }
  }
  std::uint64_t state_{0xcbf29ce484222325ull};  // 64-bit FNV offset basis
};

std::string AttributeText(const Attribute& attribute) {
  std::ostringstream text;
  text.precision(17);
  std::visit(
      [&](const auto& value) {
        using T = std::decay_t<decltype(value)>;
        if constexpr (std::is_same_v<T, std::vector<int64_t>> || std::is_same_v<T, std::vector<double>>) {
          text << '[';
          for (const auto item : value) text << item << ',';
          text << ']';
        } else {
          text << value;
        }
      },
      attribute);
  return std::to_string(attribute.index()) + "=" + text.str();
}

}  // namespace

std::string TuningDecisionKey(const PlanOp& op, const Node& node, const Graph& graph, int device_id) {
  Fingerprint key;
  key.Field("cutriton-tuning").Field(op.op_type).Field(device_id);
  cth_device_info info;
  if (cth_device_query(device_id, &info) == 0) {
    std::string uuid;
    for (const unsigned char byte : info.uuid) uuid += std::to_string(byte) + ".";
    key.Field(info.arch_name).Field(info.compute_units).Field(uuid).Field(info.driver_version).Field(info.runtime_version);
  }
  auto tensors = [&](const char* role, const std::vector<std::string>& names) {
    key.Field(role).Field(static_cast<int64_t>(names.size()));
    for (const auto& name : names) {
      key.Field(name);
      const ValueDesc* value = graph.FindValue(name);
      if (value == nullptr) continue;
      key.Field(static_cast<int64_t>(value->tensor.dtype)).Field(value->tensor.layout);
      for (const int64_t d : value->tensor.shape) key.Field(d);
    }
  };
  tensors("in", op.inputs);
  tensors("out", op.outputs);
  std::map<std::string, std::string> attributes;  // sorted by name
  for (const auto& [name, value] : node.attributes()) attributes[name] = AttributeText(value);
  for (const auto& [name, text] : attributes) key.Field(name).Field(text);
  for (const auto& candidate : op.candidates) {
    key.Field(candidate.candidate_id);
    for (const auto& step : candidate.steps) {
      const auto* invocation = std::get_if<KernelInvocation>(&step);
      if (invocation == nullptr) {
        key.Field("view");
        continue;
      }
      const KernelArtifact& code = invocation->artifact;
      key.Field(code.pack_name).Field(code.pack_version).Field(code.kernel_id).Field(code.kernel_version)
          .Field(code.variant_id).Field(code.abi_schema_version).Field(code.generator_version)
          .Field(code.triton_version).Field(code.sha256);
    }
  }
  return key.Hex();
}

std::optional<std::string> TuningStore::Lookup(const std::string& key) const {
  std::ifstream in(PathOf(key), std::ios::binary);
  if (!in) return std::nullopt;
  std::stringstream text;
  text << in.rdbuf();
  try {
    const json::Value record = json::Parse(text.str());
    // A record for another key (a renamed file) does not count.
    if (const json::Value* recorded = record.find("tuning_key"); recorded != nullptr && recorded->string() != key) {
      return std::nullopt;
    }
    return record.at("candidate_id").string();
  } catch (const std::exception&) {
    return std::nullopt;  // unreadable records are misses
  }
}

namespace {

std::string Quoted(const std::string& text) {
  std::string out = "\"";
  for (const char c : text) {
    if (c == '"' || c == '\\') out += '\\';
    out += c;
  }
  return out + "\"";
}

}  // namespace

Status TuningStore::Record(const std::string& key, const std::string& candidate_id, double median_ms) const {
  namespace fs = std::filesystem;
  std::error_code error;
  fs::create_directories(folder_, error);
  if (error) return Status::RuntimeError("cannot create the tuning cache folder " + folder_ + ": " + error.message());
  const fs::path target = PathOf(key);
  const fs::path staged = target.string() + ".partial";
  {
    std::ofstream out(staged, std::ios::trunc);
    out.precision(9);
    out << "{\n  \"schema_version\": 1,\n  \"tuning_key\": " << Quoted(key) << ",\n  \"candidate_id\": "
        << Quoted(candidate_id) << ",\n  \"median_ms\": " << median_ms << "\n}\n";
    if (!out.flush()) return Status::RuntimeError("cannot write the tuning record " + staged.string());
  }
  fs::rename(staged, target, error);
  if (error) {
    fs::remove(staged, error);
    return Status::RuntimeError("cannot publish the tuning record " + target.string());
  }
  return Status::OK();
}

}  // namespace cutriton
