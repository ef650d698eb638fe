#include "json_min.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>

namespace rpg {

class JParser {
 public:
  explicit JParser(const std::string& t) : t_(t) {}
  bool Value(JValue* v, int depth) {
    if (depth > 64) return Err("nesting too deep");
    Ws();
    if (i_ >= t_.size()) return Err("unexpected end of input");
    const char c = t_[i_];
    if (c == '{') return Object(v, depth);
    if (c == '[') return Array(v, depth);
    if (c == '"') {
      v->kind_ = JValue::kString;
      return String(&v->s_);
    }
    if (Lit("true")) {
      v->kind_ = JValue::kBool;
      v->b_ = true;
      return true;
    }
    if (Lit("false")) {
      v->kind_ = JValue::kBool;
      v->b_ = false;
      return true;
    }
    if (Lit("null")) {
      v->kind_ = JValue::kNull;
      return true;
    }
    return Number(v);
  }
  bool End() {
    Ws();
    return i_ == t_.size() ? true : Err("trailing characters");
  }
  std::string err;

 private:
  bool Err(const char* m) {
    if (err.empty()) {
      char buf[128];
      std::snprintf(buf, sizeof(buf), "%s at offset %zu", m, i_);
      err = buf;
    }
    return false;
  }
  void Ws() {
    while (i_ < t_.size() && (t_[i_] == ' ' || t_[i_] == '\t' || t_[i_] == '\n' || t_[i_] == '\r')) ++i_;
  }
  bool Lit(const char* s) {
    size_t n = 0;
    while (s[n]) ++n;
    if (t_.compare(i_, n, s) == 0) {
      i_ += n;
      return true;
    }
    return false;
  }
  // sign, digits, optional fraction, optional exponent (only after a digit);
  // an integer literal has neither '.' nor an exponent
  bool Number(JValue* v) {
    const size_t start = i_;
    if (i_ < t_.size() && (t_[i_] == '-' || t_[i_] == '+')) ++i_;
    bool digits = false, is_int = true;
    while (i_ < t_.size() && t_[i_] >= '0' && t_[i_] <= '9') ++i_, digits = true;
    if (i_ < t_.size() && t_[i_] == '.') {
      ++i_;
      is_int = false;
      while (i_ < t_.size() && t_[i_] >= '0' && t_[i_] <= '9') ++i_, digits = true;
    }
    if (digits && i_ < t_.size() && (t_[i_] == 'e' || t_[i_] == 'E')) {
      ++i_;
      is_int = false;
      if (i_ < t_.size() && (t_[i_] == '-' || t_[i_] == '+')) ++i_;
      while (i_ < t_.size() && t_[i_] >= '0' && t_[i_] <= '9') ++i_;
    }
    if (!digits) {
      i_ = start;
      return Err("invalid value");
    }
    v->kind_ = JValue::kNumber;
    v->n_ = std::strtod(t_.substr(start, i_ - start).c_str(), nullptr);
    v->int_literal_ = is_int;
    return true;
  }
  static void Utf8(uint32_t cp, std::string* out) {
    if (cp < 0x80) {
      out->push_back(static_cast<char>(cp));
    } else if (cp < 0x800) {
      out->push_back(static_cast<char>(0xC0 | (cp >> 6)));
      out->push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    } else if (cp < 0x10000) {
      out->push_back(static_cast<char>(0xE0 | (cp >> 12)));
      out->push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
      out->push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    } else {
      out->push_back(static_cast<char>(0xF0 | (cp >> 18)));
      out->push_back(static_cast<char>(0x80 | ((cp >> 12) & 0x3F)));
      out->push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
      out->push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    }
  }
  bool Hex4(uint32_t* out) {
    if (i_ + 4 > t_.size()) return Err("short \\u escape");
    uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
      const char c = t_[i_++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= static_cast<uint32_t>(c - '0');
      else if (c >= 'a' && c <= 'f') v |= static_cast<uint32_t>(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= static_cast<uint32_t>(c - 'A' + 10);
      else return Err("bad \\u escape");
    }
    *out = v;
    return true;
  }
  bool String(std::string* out) {
    ++i_;  // opening quote
    while (i_ < t_.size()) {
      const char c = t_[i_++];
      if (c == '"') return true;
      if (c != '\\') {
        if (static_cast<unsigned char>(c) < 0x20) {
          --i_;
          return Err("unescaped control character in a string");
        }
        out->push_back(c);
        continue;
      }
      if (i_ >= t_.size()) break;
      const char e = t_[i_++];
      switch (e) {
        case '"': out->push_back('"'); break;
        case '\\': out->push_back('\\'); break;
        case '/': out->push_back('/'); break;
        case 'b': out->push_back('\b'); break;
        case 'f': out->push_back('\f'); break;
        case 'n': out->push_back('\n'); break;
        case 'r': out->push_back('\r'); break;
        case 't': out->push_back('\t'); break;
        case 'u': {
          // a surrogate pair joins into one code point; a lone surrogate
          // reads as U+FFFD
          uint32_t cp;
          if (!Hex4(&cp)) return false;
          if (cp >= 0xD800 && cp <= 0xDBFF) {
            if (t_.compare(i_, 2, "\\u") == 0) {
              i_ += 2;
              uint32_t lo;
              if (!Hex4(&lo)) return false;
              cp = (lo >= 0xDC00 && lo <= 0xDFFF) ? 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00) : 0xFFFDu;
            } else {
              cp = 0xFFFDu;
            }
          } else if (cp >= 0xDC00 && cp <= 0xDFFF) {
            cp = 0xFFFDu;
          }
          Utf8(cp, out);
          break;
        }
        default: return Err("bad escape");
      }
    }
    return Err("unterminated string");
  }
  bool Array(JValue* v, int depth) {
    v->kind_ = JValue::kArray;
    ++i_;
    Ws();
    if (i_ < t_.size() && t_[i_] == ']') {
      ++i_;
      return true;
    }
    for (;;) {
      JValue item;
      if (!Value(&item, depth + 1)) return false;
      v->arr_.push_back(std::move(item));
      Ws();
      if (i_ < t_.size() && t_[i_] == ',') {
        ++i_;
        continue;
      }
      if (i_ < t_.size() && t_[i_] == ']') {
        ++i_;
        return true;
      }
      return Err("expected , or ]");
    }
  }
  bool Object(JValue* v, int depth) {
    v->kind_ = JValue::kObject;
    ++i_;
    Ws();
    if (i_ < t_.size() && t_[i_] == '}') {
      ++i_;
      return true;
    }
    for (;;) {
      Ws();
      if (i_ >= t_.size() || t_[i_] != '"') return Err("expected a key");
      std::string key;
      if (!String(&key)) return false;
      Ws();
      if (i_ >= t_.size() || t_[i_] != ':') return Err("expected :");
      ++i_;
      JValue item;
      if (!Value(&item, depth + 1)) return false;
      v->Set(key, std::move(item));
      Ws();
      if (i_ < t_.size() && t_[i_] == ',') {
        ++i_;
        continue;
      }
      if (i_ < t_.size() && t_[i_] == '}') {
        ++i_;
        return true;
      }
      return Err("expected , or }");
    }
  }
  const std::string& t_;
  size_t i_ = 0;
};

JValue JValue::Parse(const std::string& text, std::string* err) {
  JParser p(text);
  JValue v;
  if (!p.Value(&v, 0) || !p.End()) {
    if (err) *err = p.err;
    return JValue();
  }
  if (err) err->clear();
  return v;
}

JValue JValue::Object() {
  JValue v;
  v.kind_ = kObject;
  return v;
}

JValue JValue::Array() {
  JValue v;
  v.kind_ = kArray;
  return v;
}

JValue JValue::String(std::string s) {
  JValue v;
  v.kind_ = kString;
  v.s_ = std::move(s);
  return v;
}

JValue JValue::Num(double d, bool int_literal) {
  JValue v;
  v.kind_ = kNumber;
  v.n_ = d;
  v.int_literal_ = int_literal;
  return v;
}

JValue JValue::Boolean(bool b) {
  JValue v;
  v.kind_ = kBool;
  v.b_ = b;
  return v;
}

const JValue& JValue::Get(const std::string& key) const {
  static const JValue kNullValue;
  if (kind_ != kObject) return kNullValue;
  for (const auto& kv : obj_)
    if (kv.first == key) return kv.second;
  return kNullValue;
}

void JValue::Set(const std::string& key, JValue v) {
  if (kind_ != kObject) {
    *this = Object();
  }
  for (auto& kv : obj_) {
    if (kv.first == key) {
      kv.second = std::move(v);
      return;
    }
  }
  obj_.emplace_back(key, std::move(v));
}

void JValue::Push(JValue v) {
  if (kind_ != kArray) *this = Array();
  arr_.push_back(std::move(v));
}

namespace {

// The shortest %.*g form that reads back to the same double (Python's
// repr), with ".0" added when it would otherwise read as an integer.
std::string ShortestDouble(double v) {
  char buf[40] = {0};
  for (int p = 1; p <= 17; ++p) {
    std::snprintf(buf, sizeof(buf), "%.*g", p, v);
    if (std::strtod(buf, nullptr) == v) break;
  }
  std::string s = buf;
  if (s.find_first_of(".eEn") == std::string::npos) s += ".0";  // 'n': inf / nan never reach here
  return s;
}

void DumpTo(const JValue& v, bool py, std::string* o) {
  switch (v.kind()) {
    case JValue::kNull: *o += "null"; return;
    case JValue::kBool: *o += v.Bool(false) ? "true" : "false"; return;
    case JValue::kString: *o += JsonQuote(v.str()); return;
    case JValue::kNumber: {
      const double d = v.num();
      if (!std::isfinite(d)) {
        *o += "null";
      } else if (v.IsIntLiteral() && std::fabs(d) < 9007199254740992.0) {
        *o += std::to_string(static_cast<long long>(d));
      } else {
        *o += ShortestDouble(d);
      }
      return;
    }
    case JValue::kArray: {
      *o += '[';
      for (size_t i = 0; i < v.items().size(); ++i) {
        if (i) *o += py ? ", " : ",";
        DumpTo(v.items()[i], py, o);
      }
      *o += ']';
      return;
    }
    case JValue::kObject: {
      *o += '{';
      for (size_t i = 0; i < v.members().size(); ++i) {
        if (i) *o += py ? ", " : ",";
        *o += JsonQuote(v.members()[i].first);
        *o += py ? ": " : ":";
        DumpTo(v.members()[i].second, py, o);
      }
      *o += '}';
      return;
    }
  }
}

}  // namespace

std::string JValue::Dump(bool python_sep) const {
  std::string o;
  DumpTo(*this, python_sep, &o);
  return o;
}

std::string JsonQuote(const std::string& s) {
  std::string o = "\"";
  for (unsigned char c : s) {
    switch (c) {
      case '"': o += "\\\""; break;
      case '\\': o += "\\\\"; break;
      case '\b': o += "\\b"; break;
      case '\f': o += "\\f"; break;
      case '\n': o += "\\n"; break;
      case '\r': o += "\\r"; break;
      case '\t': o += "\\t"; break;
      default:
        if (c < 0x20) {
          char buf[8];
          std::snprintf(buf, sizeof(buf), "\\u%04x", c);
          o += buf;
        } else {
          o.push_back(static_cast<char>(c));
        }
    }
  }
  o += "\"";
  return o;
}

}  // namespace rpg
