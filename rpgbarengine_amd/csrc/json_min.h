// JSON value, parser and writer for the C ABI's request / config / response
// strings and the ChatML tool definitions (RFC 8259 plus a leading '+' on
// numbers, as the reference accepts).
//
// Behaviour the text front-end depends on (reference src/json.h:25-150,
// src/json.cc:60-483):
//   * objects keep their keys in insertion order; a repeated key replaces the
//     value in place (Python's dict after json.loads);
//   * a number remembers whether it was written as an integer (no '.', 'e' or
//     'E'), so `1` and `1.0` dump back as they came;
//   * Dump(python_sep = true) writes json.dumps(..., ensure_ascii=False)
//     style -- ", " and ": " separators, non-ASCII bytes raw, control
//     characters as \uXXXX, floats in the shortest form that reads back
//     (Python's repr), non-finite numbers as null.

#ifndef RPG_HIP_JSON_MIN_H_
#define RPG_HIP_JSON_MIN_H_

#include <cstdint>
#include <string>
#include <utility>
#include <vector>

namespace rpg {

class JValue {
 public:
  enum Kind { kNull, kBool, kNumber, kString, kArray, kObject };
  JValue() = default;
  static JValue Parse(const std::string& text, std::string* err);
  static JValue Object();
  static JValue Array();
  static JValue String(std::string s);
  static JValue Num(double v, bool int_literal);
  static JValue Integer(int64_t v) { return Num(static_cast<double>(v), true); }
  static JValue Boolean(bool b);

  Kind kind() const { return kind_; }
  bool IsNull() const { return kind_ == kNull; }
  bool IsObject() const { return kind_ == kObject; }
  bool IsArray() const { return kind_ == kArray; }
  bool IsString() const { return kind_ == kString; }
  bool IsNumber() const { return kind_ == kNumber; }
  bool IsBool() const { return kind_ == kBool; }
  bool IsIntLiteral() const { return kind_ == kNumber && int_literal_; }

  // Member lookup; a null value when absent or when this is not an object.
  const JValue& Get(const std::string& key) const;
  // Array elements (empty unless an array); object members in order.
  const std::vector<JValue>& items() const { return arr_; }
  const std::vector<std::pair<std::string, JValue>>& members() const { return obj_; }
  const std::string& str() const { return s_; }
  std::string AsStr(const std::string& def) const { return kind_ == kString ? s_ : def; }
  double num(double def = 0.0) const { return kind_ == kNumber ? n_ : def; }
  int64_t Int(int64_t def) const { return kind_ == kNumber ? static_cast<int64_t>(n_) : def; }
  bool Bool(bool def) const { return kind_ == kBool ? b_ : def; }

  // Builders: Set replaces an existing key in place, else appends.
  void Set(const std::string& key, JValue v);
  void Push(JValue v);

  // Compact (",", ":") or Python-style (", ", ": ") text.
  std::string Dump(bool python_sep = false) const;

 private:
  friend class JParser;
  Kind kind_ = kNull;
  bool b_ = false;
  bool int_literal_ = false;
  double n_ = 0.0;
  std::string s_;
  std::vector<JValue> arr_;
  std::vector<std::pair<std::string, JValue>> obj_;
};

// JSON string literal (with quotes) of s: ", \ and the control characters
// escaped, every other byte as it is.
std::string JsonQuote(const std::string& s);

}  // namespace rpg

#endif  // RPG_HIP_JSON_MIN_H_
