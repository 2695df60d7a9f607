// Kernel Pack v2 loader and catalog. Schema and validation rules follow
// reference src/backend/kernel_artifact.cpp:228-532 (grid AST, argument
// sources, reserved tail, constraints, safe binary paths, SHA-256 check,
// default variant per op, repository hash). The accepted binary_format is
// "hsaco": a gfx950 AMDGPU code object loaded with hipModuleLoadData.
#include "cutriton/backend/kernel_artifact.h"

#include <fstream>
#include <initializer_list>
#include <sstream>
#include <unordered_set>

#include "backend/json.h"

namespace cutriton {
namespace {

using json::Value;

constexpr const char* kBinaryFormat = "hsaco";

int AsInt(const Value& v) { return static_cast<int>(v.number()); }

int IntOr(const Value& object, const char* key, int fallback) {
  const Value* v = object.find(key);
  return v == nullptr ? fallback : AsInt(*v);
}

double DoubleOr(const Value& object, const char* key, double fallback) {
  const Value* v = object.find(key);
  return v == nullptr ? fallback : v->number();
}

std::string ReadFile(const std::filesystem::path& path, bool* ok) {
  std::ifstream in(path, std::ios::binary);
  *ok = static_cast<bool>(in);
  std::ostringstream contents;
  if (*ok) contents << in.rdbuf();
  return contents.str();
}

void OnlyKeys(const Value& v, std::initializer_list<const char*> allowed) {
  std::unordered_set<std::string> keys(allowed.begin(), allowed.end());
  for (const auto& member : v.object()) {
    if (keys.count(member.first) == 0) {
      throw std::runtime_error("unknown grid expression field: " + member.first);
    }
  }
}

GridExpression ParseGrid(const Value& v, int depth) {
  if (depth > 8) throw std::runtime_error("grid expression is too deep");
  GridExpression e;
  const std::string kind = v.at("kind").string();
  if (kind == "literal") {
    OnlyKeys(v, {"kind", "value"});
    e.kind = GridExpressionKind::kLiteral;
    e.literal = AsInt(v.at("value"));
    if (e.literal <= 0) throw std::runtime_error("grid literal must be positive");
  } else if (kind == "input_dim" || kind == "output_dim") {
    OnlyKeys(v, {"kind", "index", "axis"});
    e.kind = kind == "input_dim" ? GridExpressionKind::kInputDim : GridExpressionKind::kOutputDim;
    e.tensor_index = AsInt(v.at("index"));
    e.axis = AsInt(v.at("axis"));
  } else if (kind == "input_numel" || kind == "output_numel") {
    OnlyKeys(v, {"kind", "index"});
    e.kind = kind == "input_numel" ? GridExpressionKind::kInputNumElements
                                   : GridExpressionKind::kOutputNumElements;
    e.tensor_index = AsInt(v.at("index"));
  } else if (kind == "meta") {
    OnlyKeys(v, {"kind", "name"});
    e.kind = GridExpressionKind::kVariantMeta;
    e.meta_name = v.at("name").string();
    if (e.meta_name.empty()) throw std::runtime_error("grid meta name is empty");
  } else if (kind == "ceil_div" || kind == "mul") {
    OnlyKeys(v, {"kind", "args"});
    const auto& args = v.at("args").array();
    if (args.size() != 2) throw std::runtime_error(kind + " grid expression needs two operands");
    e.kind = kind == "ceil_div" ? GridExpressionKind::kCeilDiv : GridExpressionKind::kMultiply;
    for (const auto& arg : args) e.operands.push_back(ParseGrid(arg, depth + 1));
  } else {
    throw std::runtime_error("unsupported grid expression kind: " + kind);
  }
  return e;
}

// ABI v1: {"op":"ceil_div","value":{"kind":"output_numel","index":i},"divisor":d}.
GridExpression ParseLegacyGrid(const Value& grid, int* divisor) {
  if (grid.at("op").string() != "ceil_div" ||
      grid.at("value").at("kind").string() != "output_numel") {
    throw std::runtime_error("unsupported ABI v1 grid expression");
  }
  *divisor = AsInt(grid.at("divisor"));
  if (*divisor <= 0) throw std::runtime_error("grid divisor must be positive");
  GridExpression numel;
  numel.kind = GridExpressionKind::kOutputNumElements;
  numel.tensor_index = IntOr(grid.at("value"), "index", 0);
  GridExpression divide;
  divide.kind = GridExpressionKind::kLiteral;
  divide.literal = *divisor;
  GridExpression root;
  root.kind = GridExpressionKind::kCeilDiv;
  root.operands = {std::move(numel), std::move(divide)};
  return root;
}

KernelArgumentSourceKind SourceKind(const std::string& name) {
  static const std::pair<const char*, KernelArgumentSourceKind> table[] = {
      {"input", KernelArgumentSourceKind::kInput},
      {"output", KernelArgumentSourceKind::kOutput},
      {"input_dim", KernelArgumentSourceKind::kInputDim},
      {"input_dim_product", KernelArgumentSourceKind::kInputDimProduct},
      {"output_dim", KernelArgumentSourceKind::kOutputDim},
      {"output_numel", KernelArgumentSourceKind::kOutputNumElements},
      {"attribute_i64", KernelArgumentSourceKind::kAttributeInt64},
      {"attribute_f64", KernelArgumentSourceKind::kAttributeFloat64},
      {"literal_i32", KernelArgumentSourceKind::kLiteralInt32},
      {"runtime_reserved", KernelArgumentSourceKind::kRuntimeReserved},
  };
  for (const auto& entry : table) {
    if (name == entry.first) return entry.second;
  }
  throw std::runtime_error("unsupported argument source: " + name);
}

KernelArgumentSpec ParseArgument(const Value& v) {
  KernelArgumentSpec argument;
  argument.name = v.at("name").string();
  argument.type = v.at("type").string();
  const Value& source = v.at("source");
  KernelArgumentSource& s = argument.source;
  s.kind = SourceKind(source.at("kind").string());
  s.index = IntOr(source, "index", 0);
  s.axis = IntOr(source, "axis", 0);
  s.begin_axis = IntOr(source, "begin_axis", 0);
  if (const Value* name = source.find("name")) s.attribute_name = name->string();
  if (const Value* alt = source.find("alternate_name")) s.alternate_attribute_name = alt->string();
  s.attribute_index = IntOr(source, "index", 0);
  s.default_int = IntOr(source, "default", 0);
  s.default_float = DoubleOr(source, "default", 0.0);
  if (const Value* layout = source.find("layout")) {
    s.layout = layout->string();
    if (s.kind != KernelArgumentSourceKind::kInput || !IsInputLayout(s.layout)) {
      throw std::runtime_error("argument " + argument.name +
                               ": only an input may request a layout, and only OHWI or NK");
    }
  }
  return argument;
}

KernelConstraint ParseConstraint(const Value& v) {
  KernelConstraint c;
  const std::string kind = v.at("kind").string();
  c.expected = AsInt(v.at("value"));
  if (kind == "attribute_i64_eq") {
    c.kind = KernelConstraintKind::kAttributeInt64Equals;
    c.attribute_name = v.at("name").string();
    c.default_value = IntOr(v, "default", 0);
  } else if (kind == "input_count_eq") {
    c.kind = KernelConstraintKind::kInputCountEquals;
  } else if (kind == "tensor_bytes_le") {
    c.kind = KernelConstraintKind::kTensorBytesAtMost;
    if (c.expected <= 0) throw std::runtime_error("tensor_bytes_le value must be positive");
  } else if (kind == "tensor_rank_eq" || kind == "dim_le") {
    c.kind = kind == "dim_le" ? KernelConstraintKind::kTensorDimAtMost : KernelConstraintKind::kTensorRankEquals;
    const std::string source = v.at("source").string();
    if (source != "input" && source != "output") {
      throw std::runtime_error(kind + " source must be input or output");
    }
    c.tensor_is_output = source == "output";
    c.tensor_index = IntOr(v, "index", 0);
    if (kind == "dim_le") {
      c.tensor_axis = static_cast<int>(AsInt(v.at("axis")));
      if (c.tensor_axis < 0) throw std::runtime_error("dim_le axis must be non-negative");
    }
  } else {
    throw std::runtime_error("unsupported kernel constraint: " + kind);
  }
  return c;
}

void CheckArgumentList(const std::vector<KernelArgumentSpec>& arguments) {
  std::unordered_set<std::string> names;
  int reserved = 0;
  for (std::size_t i = 0; i < arguments.size(); ++i) {
    if (!names.insert(arguments[i].name).second) {
      throw std::runtime_error("duplicate kernel argument name: " + arguments[i].name);
    }
    if (arguments[i].source.kind == KernelArgumentSourceKind::kRuntimeReserved) {
      ++reserved;
      if (i + 2 < arguments.size()) {
        throw std::runtime_error("runtime reserved arguments must be at the ABI tail");
      }
    }
  }
  if (reserved != 2) throw std::runtime_error("kernel ABI requires two runtime reserved arguments");
}

}  // namespace

Status ArtifactRepository::Load(const std::vector<std::string>& paths) {
  artifacts_.clear();
  by_op_type_.clear();
  repository_hash_.clear();
  if (paths.empty()) return Status::InvalidArgument("kernel artifact paths are empty");
  std::string digest_material;
  // Variants of one kernel family share a code object: read and hash each
  // file once per load.
  std::unordered_map<std::string, std::string> file_digests;
  try {
    for (const auto& item : paths) {
      const std::filesystem::path given(item);
      const std::filesystem::path manifest =
          std::filesystem::is_directory(given) ? given / "pack.json" : given;
      if (!std::filesystem::exists(manifest)) {
        return Status::NotFound("Kernel Pack not found: " + manifest.string());
      }
      const std::filesystem::path root = manifest.parent_path();
      bool readable = false;
      const std::string text = ReadFile(manifest, &readable);
      if (!readable) return Status::NotFound("Kernel Pack is unreadable: " + manifest.string());
      const Value pack = json::Parse(text);
      if (AsInt(pack.at("schema_version")) != 2) {
        return Status::InvalidArgument("Kernel Pack schema v2 is required; regenerate the pack");
      }
      const int abi = AsInt(pack.at("abi_schema_version"));
      if (abi != 1 && abi != 2) return Status::InvalidArgument("unsupported Kernel Pack ABI schema");
      const std::string pack_name = pack.at("pack_name").string();
      const int pack_version = AsInt(pack.at("pack_version"));
      const std::string generator = pack.at("generator_version").string();
      const std::string toolchain = pack.at("triton_version").string();
      digest_material += Sha256Hex(text);
      for (const Value& entry : pack.at("kernels").array()) {
        KernelArtifact a;
        a.pack_name = pack_name;
        a.pack_version = pack_version;
        a.generator_version = generator;
        a.triton_version = toolchain;
        a.abi_schema_version = abi;
        a.kernel_id = entry.at("kernel_id").string();
        a.op_type = entry.at("op_type").string();
        a.kernel_version = AsInt(entry.at("kernel_version"));
        a.variant_id = entry.at("variant_id").string();
        a.is_default = entry.at("default").boolean();
        a.symbol = entry.at("symbol").string();
        a.binary_format = entry.at("binary_format").string();
        a.sha256 = entry.at("sha256").string();
        a.dtype = entry.at("dtype").string();
        a.layout = entry.at("layout").string();
        a.min_compute_capability = AsInt(entry.at("min_compute_capability"));
        if (const Value* arch = entry.find("target_arch")) a.target_arch = arch->string();
        a.num_warps = AsInt(entry.at("num_warps"));
        a.num_stages = AsInt(entry.at("num_stages"));
        a.shared_memory_bytes = AsInt(entry.at("shared_memory_bytes"));
        if (const Value* scratch = entry.find("runtime_scratch_bytes")) {
          const double bytes = scratch->number();
          if (bytes < 0 || bytes > 1e12) throw std::runtime_error("runtime_scratch_bytes is out of range");
          a.runtime_scratch_bytes = static_cast<std::int64_t>(bytes);
        }
        if (a.num_warps <= 0 || a.num_warps > 16) {
          throw std::runtime_error("num_warps must be in 1..16 wavefronts");
        }
        if (abi == 1) {
          a.launch_grid[0] = ParseLegacyGrid(entry.at("grid"), &a.grid_divisor);
        } else {
          const auto& axes = entry.at("grid").array();
          if (axes.empty() || axes.size() > a.launch_grid.size()) {
            throw std::runtime_error("ABI v2 grid must have one to three axes");
          }
          for (std::size_t axis = 0; axis < axes.size(); ++axis) {
            a.launch_grid[axis] = ParseGrid(axes[axis], 0);
          }
          for (const auto& meta : entry.at("tuning").object()) {
            const int value = AsInt(meta.second);
            if (meta.first.empty() || value <= 0) {
              throw std::runtime_error("variant launch metadata is invalid");
            }
            a.launch_meta.emplace(meta.first, value);
          }
        }
        const std::filesystem::path relative(entry.at("binary").string());
        if (relative.is_absolute() || relative.string().find("..") != std::string::npos) {
          throw std::runtime_error("unsafe Kernel Pack binary path");
        }
        a.binary_path = root / relative;
        auto digest = file_digests.find(a.binary_path.string());
        if (digest == file_digests.end()) {
          bool found = false;
          const std::string image = ReadFile(a.binary_path, &found);
          if (!found) return Status::NotFound("kernel binary not found: " + a.binary_path.string());
          digest = file_digests.emplace(a.binary_path.string(), Sha256Hex(image)).first;
        }
        if (digest->second != a.sha256) {
          return Status::InvalidArgument("kernel binary SHA-256 mismatch: " +
                                         a.binary_path.string());
        }
        for (const Value& arg : entry.at("arguments").array()) {
          a.arguments.push_back(ParseArgument(arg));
        }
        CheckArgumentList(a.arguments);
        for (const Value& c : entry.at("constraints").array()) {
          a.constraints.push_back(ParseConstraint(c));
        }
        if (a.kernel_id.empty() || a.variant_id.empty() || a.symbol.empty() ||
            a.arguments.empty() || a.binary_format != kBinaryFormat) {
          throw std::runtime_error("incomplete kernel artifact entry (binary_format must be \"" +
                                   std::string(kBinaryFormat) + "\")");
        }
        digest_material += a.sha256;
        by_op_type_[a.op_type].push_back(a);
        artifacts_.push_back(std::move(a));
      }
    }
  } catch (const std::exception& error) {
    artifacts_.clear();
    by_op_type_.clear();
    return Status::InvalidArgument(std::string("invalid Kernel Pack: ") + error.what());
  }
  for (const auto& entry : by_op_type_) {
    bool has_default = false;
    for (const auto& a : entry.second) has_default = has_default || a.is_default;
    if (!has_default) return Status::InvalidArgument("no default kernel variant for " + entry.first);
  }
  repository_hash_ = Sha256Hex(digest_material);
  return Status::OK();
}

const std::vector<KernelArtifact>* ArtifactRepository::Find(const std::string& op_type) const {
  const auto it = by_op_type_.find(op_type);
  return it == by_op_type_.end() ? nullptr : &it->second;
}

std::vector<const KernelArtifact*> KernelCatalog::Query(const std::string& op_type,
                                                        const std::string& dtype,
                                                        const std::string& layout,
                                                        int compute_capability) const {
  std::vector<const KernelArtifact*> matches;
  if (repository_ == nullptr) return matches;
  const auto* candidates = repository_->Find(op_type);
  if (candidates == nullptr) return matches;
  for (const auto& a : *candidates) {
    const bool layout_ok = layout.empty() || a.layout.empty() || a.layout == layout;
    if (a.dtype == dtype && layout_ok && compute_capability >= a.min_compute_capability) {
      matches.push_back(&a);
    }
  }
  return matches;
}

}  // namespace cutriton
