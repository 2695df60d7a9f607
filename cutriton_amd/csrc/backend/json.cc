#include "backend/json.h"

#include <cctype>
#include <cstdlib>

namespace cutriton {
namespace json {
namespace {

class Reader {
 public:
  explicit Reader(const std::string& text) : text_(text) {}

  Value Document() {
    Value value = Any(0);
    Skip();
    if (pos_ != text_.size()) throw std::runtime_error("trailing data after JSON document");
    return value;
  }

 private:
  static constexpr int kMaxDepth = 64;

  void Skip() {
    while (pos_ < text_.size() && std::isspace(static_cast<unsigned char>(text_[pos_]))) ++pos_;
  }
  char Peek() {
    Skip();
    if (pos_ >= text_.size()) throw std::runtime_error("unexpected end of JSON");
    return text_[pos_];
  }
  void Expect(char c) {
    if (Peek() != c) throw std::runtime_error(std::string("expected '") + c + "' in JSON");
    ++pos_;
  }
  bool Literal(const char* word) {
    const std::size_t n = std::char_traits<char>::length(word);
    if (text_.compare(pos_, n, word) != 0) return false;
    pos_ += n;
    return true;
  }

  Value Any(int depth) {
    if (depth > kMaxDepth) throw std::runtime_error("JSON nesting is too deep");
    const char c = Peek();
    if (c == '{') return Value(Members(depth));
    if (c == '[') return Value(Elements(depth));
    if (c == '"') return Value(Text());
    if (c == '-' || (c >= '0' && c <= '9')) return Value(Number());
    if (Literal("true")) return Value(true);
    if (Literal("false")) return Value(false);
    if (Literal("null")) return Value();
    throw std::runtime_error("invalid JSON value");
  }

  Value::Object Members(int depth) {
    Expect('{');
    Value::Object members;
    if (Peek() == '}') {
      ++pos_;
      return members;
    }
    for (;;) {
      if (Peek() != '"') throw std::runtime_error("expected a JSON object key");
      std::string key = Text();
      Expect(':');
      if (!members.emplace(key, Any(depth + 1)).second) {
        throw std::runtime_error("duplicate JSON object key: " + key);
      }
      const char next = Peek();
      ++pos_;
      if (next == '}') return members;
      if (next != ',') throw std::runtime_error("expected ',' or '}' in JSON object");
    }
  }

  Value::Array Elements(int depth) {
    Expect('[');
    Value::Array elements;
    if (Peek() == ']') {
      ++pos_;
      return elements;
    }
    for (;;) {
      elements.push_back(Any(depth + 1));
      const char next = Peek();
      ++pos_;
      if (next == ']') return elements;
      if (next != ',') throw std::runtime_error("expected ',' or ']' in JSON array");
    }
  }

  std::string Text() {
    Expect('"');
    std::string out;
    while (pos_ < text_.size()) {
      const char c = text_[pos_++];
      if (c == '"') return out;
      if (static_cast<unsigned char>(c) < 0x20) throw std::runtime_error("control character in JSON string");
      if (c != '\\') {
        out.push_back(c);
        continue;
      }
      if (pos_ >= text_.size()) break;
      const char e = text_[pos_++];
      switch (e) {
        case '"': out.push_back('"'); break;
        case '\\': out.push_back('\\'); break;
        case '/': out.push_back('/'); break;
        case 'b': out.push_back('\b'); break;
        case 'f': out.push_back('\f'); break;
        case 'n': out.push_back('\n'); break;
        case 'r': out.push_back('\r'); break;
        case 't': out.push_back('\t'); break;
        default: throw std::runtime_error("unsupported JSON escape");
      }
    }
    throw std::runtime_error("unterminated JSON string");
  }

  double Number() {
    const std::size_t begin = pos_;
    auto digits = [&] {
      const std::size_t start = pos_;
      while (pos_ < text_.size() && std::isdigit(static_cast<unsigned char>(text_[pos_]))) ++pos_;
      return pos_ > start;
    };
    if (text_[pos_] == '-') ++pos_;
    if (!digits()) throw std::runtime_error("malformed JSON number");
    if (pos_ < text_.size() && text_[pos_] == '.') {
      ++pos_;
      if (!digits()) throw std::runtime_error("malformed JSON number");
    }
    if (pos_ < text_.size() && (text_[pos_] == 'e' || text_[pos_] == 'E')) {
      ++pos_;
      if (pos_ < text_.size() && (text_[pos_] == '+' || text_[pos_] == '-')) ++pos_;
      if (!digits()) throw std::runtime_error("malformed JSON number");
    }
    return std::strtod(text_.substr(begin, pos_ - begin).c_str(), nullptr);
  }

  const std::string& text_;
  std::size_t pos_{0};
};

}  // namespace

Value Parse(const std::string& text) { return Reader(text).Document(); }

}  // namespace json
}  // namespace cutriton
