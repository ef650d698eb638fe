// Minimal JSON value, parser and writer for the C ABI's request / config /
// response strings (RFC 8259 subset: objects, arrays, strings with escapes,
// numbers, true/false/null). Text front-end work beyond that is out of scope.

#ifndef RPG_HIP_JSON_MIN_H_
#define RPG_HIP_JSON_MIN_H_

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace rpg {

class JValue {
 public:
  enum Kind { kNull, kBool, kNumber, kString, kArray, kObject };
  JValue() = default;
  static JValue Parse(const std::string& text, std::string* err);

  Kind kind() const { return kind_; }
  bool IsNull() const { return kind_ == kNull; }
  bool IsObject() const { return kind_ == kObject; }
  bool IsArray() const { return kind_ == kArray; }
  bool IsString() const { return kind_ == kString; }
  bool IsNumber() const { return kind_ == kNumber; }
  bool IsBool() const { return kind_ == kBool; }

  // Member lookup; a null value when absent or when this is not an object.
  const JValue& Get(const std::string& key) const;
  const std::vector<JValue>& items() const { return arr_; }
  const std::string& str() const { return s_; }
  double num(double def = 0.0) const { return kind_ == kNumber ? n_ : def; }
  int64_t Int(int64_t def) const { return kind_ == kNumber ? static_cast<int64_t>(n_) : def; }
  bool Bool(bool def) const { return kind_ == kBool ? b_ : def; }

 private:
  friend class JParser;
  Kind kind_ = kNull;
  bool b_ = false;
  double n_ = 0.0;
  std::string s_;
  std::vector<JValue> arr_;
  std::map<std::string, JValue> obj_;
};

// JSON string literal (with quotes) of s, escaping control characters.
std::string JsonQuote(const std::string& s);

}  // namespace rpg

#endif  // RPG_HIP_JSON_MIN_H_
