// include/rpg_text.h: the text front-end (tokenizer, ChatML, reply parse) as
// C functions, on the host CPU. The same code runs inside
// rpg_engine_generate (engine_abi.cc).

#include "rpg_text.h"

#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "chatml.h"
#include "common.h"
#include "gguf.h"
#include "json_min.h"
#include "tokenizer.h"
#include "tool_parser.h"
#include "unicode.h"

namespace {

std::mutex g_mu;
std::map<int32_t, std::shared_ptr<rpg::Tokenizer>> g_toks;
int32_t g_next = 1;

std::shared_ptr<rpg::Tokenizer> Require(int32_t h) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_toks.find(h);
  RPG_CHECK(it != g_toks.end(), "invalid tokenizer handle %d", h);
  return it->second;
}

char* DupBytes(const std::string& s) {
  char* b = new char[s.size() + 1];
  std::memcpy(b, s.data(), s.size());
  b[s.size()] = '\0';
  return b;
}

template <typename F, typename R>
R Guard(F f, R fail) {
  try {
    rpg::SetLastError("");
    return f();
  } catch (const std::exception& e) {
    rpg::SetLastError(e.what());
  } catch (...) {
    rpg::SetLastError("unknown exception");
  }
  return fail;
}

std::string Bytes(const char* p, int64_t len) {
  RPG_CHECK(p != nullptr || len == 0, "null text");
  RPG_CHECK(len >= 0, "negative length");
  return std::string(p ? p : "", static_cast<size_t>(len));
}

}  // namespace

extern "C" {

int32_t rpg_text_tokenizer_load(const char* gguf_path) {
  return Guard([&]() -> int32_t {
    RPG_CHECK(gguf_path != nullptr && *gguf_path, "empty GGUF path");
    std::unique_ptr<rpg::GgufFile> g(rpg::GgufFile::Open(gguf_path));
    auto t = std::make_shared<rpg::Tokenizer>(rpg::Tokenizer::FromGguf(*g));
    std::lock_guard<std::mutex> lk(g_mu);
    const int32_t h = g_next++;
    g_toks[h] = t;
    return h;
  }, int32_t(-1));
}

void rpg_text_tokenizer_free(int32_t tok) {
  std::lock_guard<std::mutex> lk(g_mu);
  g_toks.erase(tok);
}

int32_t rpg_text_vocab_size(int32_t tok) {
  return Guard([&]() -> int32_t { return static_cast<int32_t>(Require(tok)->size()); }, int32_t(-1));
}

int64_t rpg_text_encode(int32_t tok, const char* text, int64_t len, int32_t parse_special, int32_t* out, int64_t cap) {
  return Guard([&]() -> int64_t {
    const std::vector<int32_t> ids = Require(tok)->Encode(Bytes(text, len), parse_special != 0);
    const int64_t n = static_cast<int64_t>(ids.size());
    if (out != nullptr && cap > 0) std::memcpy(out, ids.data(), sizeof(int32_t) * static_cast<size_t>(std::min(n, cap)));
    return n;
  }, int64_t(-1));
}

char* rpg_text_decode(int32_t tok, const int32_t* ids, int64_t n, int32_t skip_special, int64_t* out_len) {
  return Guard([&]() -> char* {
    RPG_CHECK(n >= 0 && (ids != nullptr || n == 0), "bad id array");
    const std::string s = Require(tok)->Decode(std::vector<int32_t>(ids, ids + n), skip_special != 0);
    if (out_len) *out_len = static_cast<int64_t>(s.size());
    return DupBytes(s);
  }, static_cast<char*>(nullptr));
}

int64_t rpg_text_split(int32_t tok, const char* text, int64_t len, int64_t* piece_lens, int64_t cap) {
  return Guard([&]() -> int64_t {
    const std::vector<std::string> pieces = Require(tok)->Split(Bytes(text, len));
    const int64_t n = static_cast<int64_t>(pieces.size());
    for (int64_t i = 0; piece_lens != nullptr && i < std::min(n, cap); ++i)
      piece_lens[i] = static_cast<int64_t>(pieces[static_cast<size_t>(i)].size());
    return n;
  }, int64_t(-1));
}

char* rpg_text_render_chatml(const char* request_json) {
  return Guard([&]() -> char* {
    RPG_CHECK(request_json != nullptr, "null request");
    std::string err;
    const rpg::JValue req = rpg::JValue::Parse(request_json, &err);
    RPG_CHECK(err.empty(), "request_json failed to parse: %s", err.c_str());
    RPG_CHECK(req.IsObject(), "request_json must be a JSON object");
    return DupBytes(rpg::RenderChatml(rpg::ParseChatMessages(req.Get("messages")),
                                      rpg::ParseChatTools(req.Get("tools")), true,
                                      req.Get("enable_thinking").Bool(true)));
  }, static_cast<char*>(nullptr));
}

char* rpg_text_parse_reply(const char* text, int64_t len) {
  return Guard([&]() -> char* {
    const rpg::ParsedReply r = rpg::ParseReply(Bytes(text, len));
    rpg::JValue o = rpg::JValue::Object();
    o.Set("text", rpg::JValue::String(r.text));
    o.Set("reasoning", rpg::JValue::String(r.reasoning));
    rpg::JValue calls = rpg::JValue::Array();
    for (const rpg::ParsedCall& c : r.calls) {
      rpg::JValue one = rpg::JValue::Object();
      one.Set("name", rpg::JValue::String(c.name));
      one.Set("arguments_raw", rpg::JValue::String(c.arguments_raw));
      one.Set("arguments", c.arguments);
      one.Set("ok", rpg::JValue::Boolean(c.ok));
      calls.Push(std::move(one));
    }
    o.Set("tool_calls", std::move(calls));
    o.Set("unterminated_think", rpg::JValue::Boolean(r.unterminated_think));
    o.Set("unterminated_tool_call", rpg::JValue::Boolean(r.unterminated_call));
    return DupBytes(o.Dump(false));
  }, static_cast<char*>(nullptr));
}

int32_t rpg_text_char_classes(uint32_t first, int64_t n, uint8_t* out) {
  return Guard([&]() -> int32_t {
    RPG_CHECK(n >= 0 && (out != nullptr || n == 0), "bad output buffer");
    for (int64_t i = 0; i < n; ++i) {
      const uint32_t cp = first + static_cast<uint32_t>(i);
      out[i] = static_cast<uint8_t>((rpg::uni::IsLetter(cp) ? 1 : 0) | (rpg::uni::IsNumber(cp) ? 2 : 0) |
                                    (rpg::uni::IsSpace(cp) ? 4 : 0));
    }
    return 0;
  }, int32_t(-1));
}

char* rpg_text_json_redump(const char* json, int32_t python) {
  return Guard([&]() -> char* {
    RPG_CHECK(json != nullptr, "null JSON");
    std::string err;
    const rpg::JValue v = rpg::JValue::Parse(json, &err);
    RPG_CHECK(err.empty(), "JSON failed to parse: %s", err.c_str());
    return DupBytes(v.Dump(python != 0));
  }, static_cast<char*>(nullptr));
}

}  // extern "C"
