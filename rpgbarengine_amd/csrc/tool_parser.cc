#include "tool_parser.h"

#include <cstring>

#include "common.h"

namespace rpg {
namespace {

bool AsciiSpace(char c) { return c == ' ' || c == '\t' || c == '\r' || c == '\n' || c == '\f' || c == '\v'; }

std::string Trim(const std::string& s) {
  size_t b = 0, e = s.size();
  while (b < e && AsciiSpace(s[b])) ++b;
  while (e > b && AsciiSpace(s[e - 1])) --e;
  return s.substr(b, e - b);
}

void EraseAll(std::string* s, const char* marker) {
  const size_t n = std::strlen(marker);
  for (size_t p = s->find(marker); p != std::string::npos; p = s->find(marker, p)) s->erase(p, n);
}

void DropControlMarkers(std::string* s) {
  static const char* kRoles[] = {"system", "user", "assistant", "tool"};
  const std::string start = "<|im_start|>";
  for (size_t p = s->find(start); p != std::string::npos; p = s->find(start, p)) {
    size_t end = p + start.size();
    for (const char* r : kRoles) {
      const size_t rl = std::strlen(r);
      if (s->compare(end, rl, r) == 0 && end + rl < s->size() && (*s)[end + rl] == '\n') {
        end += rl + 1;
        break;
      }
    }
    s->erase(p, end - p);
  }
  EraseAll(s, "<|im_end|>");
  EraseAll(s, "<|endoftext|>");
}

ParsedCall ParseCall(const std::string& body) {
  ParsedCall c;
  const std::string t = Trim(body);
  std::string err;
  const JValue j = JValue::Parse(t, &err);
  if (!j.IsObject()) {
    c.arguments_raw = t;
  } else {
    c.name = j.Get("name").AsStr("");
    const JValue& a = j.Get("arguments");
    if (a.IsString()) {
      c.arguments_raw = a.str();
      std::string e2;
      JValue inner = JValue::Parse(c.arguments_raw, &e2);
      if (inner.IsObject()) c.arguments = std::move(inner);
    } else if (!a.IsNull()) {
      c.arguments_raw = a.Dump(false);
      c.arguments = a;
    }
    c.ok = !c.name.empty() && c.arguments.IsObject();
  }
  if (!c.ok) {
    if (c.name.empty())
      Log(kLogWarn, "unusable tool call: no name (arguments as written: %s)", c.arguments_raw.c_str());
    else
      Log(kLogWarn, "unusable tool call %s: arguments are not a JSON object (as written: %s)", c.name.c_str(),
          c.arguments_raw.c_str());
  }
  return c;
}

}  // namespace

ParsedReply ParseReply(const std::string& raw) {
  ParsedReply r;
  std::string w = raw;
  DropControlMarkers(&w);
  static const std::string kThinkOpen = "<think>", kThinkClose = "</think>";
  for (size_t b = w.find(kThinkOpen); b != std::string::npos; b = w.find(kThinkOpen)) {
    const size_t body = b + kThinkOpen.size();
    const size_t e = w.find(kThinkClose, body);
    if (e == std::string::npos) {
      r.reasoning += w.substr(body);
      w.erase(b);
      r.unterminated_think = true;
      break;
    }
    r.reasoning += w.substr(body, e - body);
    w.erase(b, e + kThinkClose.size() - b);
  }
  static const std::string kCallOpen = "<tool_call>", kCallClose = "</tool_call>";
  std::string text;
  size_t pos = 0;
  for (size_t b = w.find(kCallOpen, pos); b != std::string::npos; b = w.find(kCallOpen, pos)) {
    text.append(w, pos, b - pos);
    const size_t body = b + kCallOpen.size();
    const size_t e = w.find(kCallClose, body);
    if (e == std::string::npos) {
      r.calls.push_back(ParseCall(w.substr(body)));
      r.unterminated_call = true;
      pos = w.size();
      break;
    }
    r.calls.push_back(ParseCall(w.substr(body, e - body)));
    pos = e + kCallClose.size();
  }
  if (pos < w.size()) text.append(w, pos, std::string::npos);
  r.text = Trim(text);
  return r;
}

}  // namespace rpg
