// Minimal strict JSON reader for pack manifests and tuning records.
#pragma once

#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <variant>
#include <vector>

namespace cutriton {
namespace json {

class Value {
 public:
  using Object = std::map<std::string, Value>;
  using Array = std::vector<Value>;

  Value() : data_(nullptr) {}
  explicit Value(bool v) : data_(v) {}
  explicit Value(double v) : data_(v) {}
  explicit Value(std::string v) : data_(std::move(v)) {}
  explicit Value(Object v) : data_(std::make_shared<Object>(std::move(v))) {}
  explicit Value(Array v) : data_(std::make_shared<Array>(std::move(v))) {}

  bool is_object() const { return std::holds_alternative<std::shared_ptr<Object>>(data_); }
  bool is_array() const { return std::holds_alternative<std::shared_ptr<Array>>(data_); }
  bool is_string() const { return std::holds_alternative<std::string>(data_); }
  bool is_number() const { return std::holds_alternative<double>(data_); }
  bool is_bool() const { return std::holds_alternative<bool>(data_); }

  const Object& object() const { return *Get<std::shared_ptr<Object>>("object"); }
  const Array& array() const { return *Get<std::shared_ptr<Array>>("array"); }
  const std::string& string() const { return Get<std::string>("string"); }
  double number() const { return Get<double>("number"); }
  bool boolean() const { return Get<bool>("boolean"); }

  // Required member; throws std::runtime_error when absent.
  const Value& at(const std::string& key) const {
    const auto& members = object();
    const auto it = members.find(key);
    if (it == members.end()) throw std::runtime_error("missing JSON field: " + key);
    return it->second;
  }
  // Optional member or nullptr.
  const Value* find(const std::string& key) const {
    const auto& members = object();
    const auto it = members.find(key);
    return it == members.end() ? nullptr : &it->second;
  }

 private:
  template <typename T>
  const T& Get(const char* what) const {
    if (const T* v = std::get_if<T>(&data_)) return *v;
    throw std::runtime_error(std::string("JSON value is not a ") + what);
  }
  std::variant<std::nullptr_t, bool, double, std::string, std::shared_ptr<Object>,
               std::shared_ptr<Array>>
      data_;
};

// Parses one complete JSON document; throws std::runtime_error on any error,
// including trailing data and duplicate object keys.
Value Parse(const std::string& text);

}  // namespace json
}  // namespace cutriton
