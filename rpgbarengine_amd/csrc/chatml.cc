#include "chatml.h"

#include <cstdint>

namespace rpg {
namespace {

std::string TrimNewlinesRight(const std::string& s) {
  size_t e = s.size();
  while (e > 0 && s[e - 1] == '\n') --e;
  return s.substr(0, e);
}

std::string TrimNewlinesLeft(const std::string& s) {
  size_t b = 0;
  while (b < s.size() && s[b] == '\n') ++b;
  return s.substr(b);
}

bool HasPrefix(const std::string& s, const char* p) { return s.rfind(p, 0) == 0; }

bool HasSuffix(const std::string& s, const std::string& x) {
  return s.size() >= x.size() && s.compare(s.size() - x.size(), x.size(), x) == 0;
}

// Python's s.split(sep)[0] and s.split(sep)[-1]
std::string Head(const std::string& s, const std::string& sep) {
  const size_t p = s.find(sep);
  return p == std::string::npos ? s : s.substr(0, p);
}

std::string Tail(const std::string& s, const std::string& sep) {
  const size_t p = s.rfind(sep);
  return p == std::string::npos ? s : s.substr(p + sep.size());
}

// Jinja truthiness of a value
bool Truthy(const JValue& v) {
  switch (v.kind()) {
    case JValue::kNull: return false;
    case JValue::kBool: return v.Bool(false);
    case JValue::kNumber: return v.num() != 0.0;
    case JValue::kString: return !v.str().empty();
    case JValue::kArray: return !v.items().empty();
    case JValue::kObject: return !v.members().empty();
  }
  return false;
}

bool IsToolResponse(const std::string& c) { return HasPrefix(c, "<tool_response>") && HasSuffix(c, "</tool_response>"); }

}  // namespace

std::vector<ChatMessage> ParseChatMessages(const JValue& messages) {
  std::vector<ChatMessage> out;
  for (const JValue& m : messages.items()) {
    ChatMessage cm;
    cm.role = m.Get("role").AsStr("");
    cm.content = m.Get("content").AsStr("");
    const JValue& rc = m.Get("reasoning_content");
    if (rc.IsString()) {
      cm.has_reasoning = true;
      cm.reasoning = rc.str();
    }
    for (const JValue& tc : m.Get("tool_calls").items()) {
      const JValue& fn = tc.Get("function");
      const JValue& src = fn.IsObject() ? fn : tc;
      ChatToolCall call;
      call.name = src.Get("name").AsStr("");
      const JValue& a = src.Get("arguments");
      call.arguments = a.IsString() ? a.str() : a.Dump(true);
      cm.tool_calls.push_back(std::move(call));
    }
    out.push_back(std::move(cm));
  }
  return out;
}

JValue ParseChatTools(const JValue& tools) { return tools.IsArray() ? tools : JValue::Array(); }

std::string RenderChatml(const std::vector<ChatMessage>& msgs, const JValue& tools, bool add_generation_prompt,
                         bool enable_thinking) {
  std::string o;
  const bool system_first = !msgs.empty() && msgs[0].role == "system";
  if (Truthy(tools)) {
    o += "<|im_start|>system\n";
    if (system_first) o += msgs[0].content + "\n\n";
    o += "# Tools\n\nYou may call one or more functions to assist with the user query.\n\n"
         "You are provided with function signatures within <tools></tools> XML tags:\n<tools>";
    for (const JValue& t : tools.items()) o += "\n" + t.Dump(true);
    o += "\n</tools>\n\nFor each function call, return a json object with function name and arguments within "
         "<tool_call></tool_call> XML tags:\n<tool_call>\n{\"name\": <function-name>, \"arguments\": "
         "<args-json-object>}\n</tool_call><|im_end|>\n";
  } else if (system_first) {
    o += "<|im_start|>system\n" + msgs[0].content + "<|im_end|>\n";
  }
  // the last real user query (default: the last message)
  const int64_t n = static_cast<int64_t>(msgs.size());
  int64_t last_query = n - 1;
  for (int64_t i = n - 1; i >= 0; --i) {
    const ChatMessage& m = msgs[static_cast<size_t>(i)];
    if (m.role == "user" && !IsToolResponse(m.content)) {
      last_query = i;
      break;
    }
  }
  for (int64_t i = 0; i < n; ++i) {
    const ChatMessage& m = msgs[static_cast<size_t>(i)];
    if (m.role == "user" || (m.role == "system" && i != 0)) {
      o += "<|im_start|>" + m.role + "\n" + m.content + "<|im_end|>\n";
    } else if (m.role == "assistant") {
      std::string content = m.content, reasoning;
      if (m.has_reasoning) {
        reasoning = m.reasoning;
      } else if (content.find("</think>") != std::string::npos) {
        reasoning = TrimNewlinesLeft(Tail(TrimNewlinesRight(Head(content, "</think>")), "<think>"));
        content = TrimNewlinesLeft(Tail(content, "</think>"));
      }
      o += "<|im_start|>assistant\n";
      if (i > last_query && (i == n - 1 || !reasoning.empty())) {
        o += "<think>\n" + TrimNewlinesLeft(TrimNewlinesRight(reasoning)) + "\n</think>\n\n" +
             TrimNewlinesLeft(content);
      } else {
        o += content;
      }
      for (size_t k = 0; k < m.tool_calls.size(); ++k) {
        if (k > 0 || !content.empty()) o += "\n";
        o += "<tool_call>\n{\"name\": \"" + m.tool_calls[k].name + "\", \"arguments\": " + m.tool_calls[k].arguments +
             "}\n</tool_call>";
      }
      o += "<|im_end|>\n";
    } else if (m.role == "tool") {
      if (i == 0 || msgs[static_cast<size_t>(i - 1)].role != "tool") o += "<|im_start|>user";
      o += "\n<tool_response>\n" + m.content + "\n</tool_response>";
      if (i == n - 1 || msgs[static_cast<size_t>(i + 1)].role != "tool") o += "<|im_end|>\n";
    }
  }
  if (add_generation_prompt) {
    o += "<|im_start|>assistant\n";
    if (!enable_thinking) o += "<think>\n\n</think>\n\n";
  }
  return o;
}

}  // namespace rpg
