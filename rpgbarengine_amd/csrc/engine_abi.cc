// The 10-function C ABI of include/rpg_engine.h over the GPU token loop.
//
// Behaviour follows reference src/engine.cc:195-549: handle registry with a
// lock held only for lookup, exceptions translated to -1 / NULL + last error,
// session defaults (max_tokens 256, temperature 0 = greedy, seed 0), engine-
// pinned top_k = 0 / top_p = 0.95, temperature clamped to [0, 2], longest-
// common-prefix reuse of the cached ids (a full hit backs off one position),
// capacity check before the cache is touched, cache reset on a failed prefill
// (and on a failed generation), stop ids = eos + <|im_end|> + request/session
// stop strings that are one token. A request's "messages" (+ "tools", "enable_thinking") render as
// Qwen3 ChatML and tokenize with the model's BBPE vocabulary
// (reference src/engine.cc:366-378); the reply decodes with its special
// tokens and parses into text and tool calls (src/engine.cc:472-515). A
// request may instead carry "input_ids" (token ids, no rendering); its
// response adds "output_ids".

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "chatml.h"
#include "common.h"
#include "json_min.h"
#include "model.h"
#include "rpg_engine.h"
#include "session.h"
#include "tokenizer.h"
#include "tool_parser.h"

namespace {

using rpg::JValue;

constexpr const char* kVersion = "0.4.1";  // interface version of the reference library it replaces
constexpr int32_t kDefaultMaxTokens = 256;
constexpr int64_t kSeqMargin = 4;
constexpr int32_t kTopK = 0;
constexpr float kTopP = 0.95f;
constexpr float kMaxTemperature = 2.0f;

struct ModelEntry {
  std::shared_ptr<rpg::DeviceModel> model;
  int32_t max_pos = 0;
  int32_t default_max_seq = 0;
  std::vector<int32_t> sessions;
  std::unique_ptr<rpg::Tokenizer> tok;  // null when the GGUF holds no BBPE vocabulary
};

struct SessionEntry {
  int32_t model = -1;
  std::shared_ptr<rpg::DeviceModel> model_ref;
  std::unique_ptr<rpg::Session> s;
  std::vector<int32_t> cached_ids;
  int32_t max_tokens = kDefaultMaxTokens;
  std::vector<std::string> stop;
  float temperature = 0.0f;
  uint64_t seed = 0;
};

std::mutex g_mu;
std::map<int32_t, std::shared_ptr<ModelEntry>> g_models;
std::map<int32_t, std::shared_ptr<SessionEntry>> g_sessions;
int32_t g_next_model = 1, g_next_session = 1;

JValue ParseOrEmpty(const char* text, const char* what) {
  if (text == nullptr || *text == '\0') return JValue::Parse("{}", nullptr);
  std::string err;
  JValue v = JValue::Parse(text, &err);
  RPG_CHECK(err.empty(), "%s is not valid JSON: %s", what, err.c_str());
  RPG_CHECK(v.IsObject(), "%s must be a JSON object", what);
  return v;
}

int32_t AsI32(const JValue& v, int32_t def) { return v.IsNumber() ? static_cast<int32_t>(v.num()) : def; }
float AsF32(const JValue& v, float def) { return v.IsNumber() ? static_cast<float>(v.num()) : def; }

std::shared_ptr<ModelEntry> ModelLocked(int32_t h) {
  auto it = g_models.find(h);
  RPG_CHECK(it != g_models.end(), "invalid model handle %d (possibly unloaded)", h);
  return it->second;
}

std::shared_ptr<SessionEntry> SessionLocked(int32_t h) {
  auto it = g_sessions.find(h);
  RPG_CHECK(it != g_sessions.end(), "invalid session handle %d (possibly destroyed)", h);
  return it->second;
}

char* Dup(const std::string& s) {
  char* b = new char[s.size() + 1];
  std::memcpy(b, s.data(), s.size());
  b[s.size()] = '\0';
  return b;
}

int32_t IdOf(const ModelEntry& m, const std::string& s) { return m.tok ? m.tok->IdOf(s) : -1; }

// A stop string is a vocabulary entry or text that encodes to one token;
// longer ones need text-level matching, the host's job (reference
// src/engine.cc:142-166).
void AppendStop(const ModelEntry& m, const std::string& s, std::vector<int32_t>* out) {
  if (s.empty() || !m.tok) return;
  const int32_t id = m.tok->IdOf(s);
  if (id >= 0) {
    out->push_back(id);
    return;
  }
  const std::vector<int32_t> ids = m.tok->Encode(s, false);
  if (ids.size() == 1) {
    out->push_back(ids[0]);
    return;
  }
  rpg::Log(rpg::kLogWarn, "stop string \"%s\" encodes to %zu tokens, not one; ignored", s.c_str(), ids.size());
}

bool Contains(const std::vector<int32_t>& v, int32_t id) { return std::find(v.begin(), v.end(), id) != v.end(); }

}  // namespace

#define ABI_CATCH(ret)                     \
  catch (const std::exception& e) {        \
    rpg::SetLastError(e.what());           \
    return ret;                            \
  }                                        \
  catch (...) {                            \
    rpg::SetLastError("unknown exception"); \
    return ret;                            \
  }

extern "C" {

const char* rpg_engine_version(void) { return kVersion; }

const char* rpg_engine_last_error(void) { return rpg::LastError(); }

int32_t rpg_engine_load_model(const char* model_path, const char* config_json) {
  try {
    rpg::SetLastError("");
    RPG_CHECK(model_path != nullptr && *model_path != '\0', "model_path is empty");
    const JValue cfg = ParseOrEmpty(config_json, "config_json");
    const int32_t max_pos = AsI32(cfg.Get("max_pos"), 4096);
    int32_t max_seq = AsI32(cfg.Get("max_seq"), 0);
    RPG_CHECK(max_pos > 0, "config_json.max_pos must be positive (got %d)", max_pos);
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
      (void)hipGetLastError();
      rpg::Throw("no GPU is visible: this engine needs an MI355X (gfx950)");
    }
    auto e = std::make_shared<ModelEntry>();
    e->model.reset(rpg::DeviceModel::Load(model_path, max_pos).release());
    const rpg::ModelConfig& c = e->model->config();
    int32_t eff = max_pos;
    if (c.context_length > 0 && c.context_length < eff) eff = c.context_length;
    if (max_seq <= 0) max_seq = eff;
    if (max_seq > eff) {
      rpg::Log(rpg::kLogWarn, "config_json.max_seq=%d exceeds the %d available positions; clamped", max_seq, eff);
      max_seq = eff;
    }
    e->max_pos = eff;
    e->default_max_seq = max_seq;
    try {
      e->tok.reset(new rpg::Tokenizer(rpg::Tokenizer::FromGguf(e->model->gguf())));
    } catch (const std::exception& ex) {
      rpg::Log(rpg::kLogWarn, "no tokenizer (%s): requests must carry input_ids", ex.what());
    }
    std::lock_guard<std::mutex> lk(g_mu);
    RPG_CHECK(g_next_model > 0, "model handles exhausted");
    const int32_t h = g_next_model++;
    g_models[h] = e;
    return h;
  }
  ABI_CATCH(-1)
}

void rpg_engine_unload_model(int32_t model) {
  try {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_models.find(model);
    if (it == g_models.end()) return;
    for (int32_t s : it->second->sessions) g_sessions.erase(s);
    g_models.erase(it);
  } catch (...) {
  }
}

int32_t rpg_engine_session_create(int32_t model, const char* session_json) {
  try {
    rpg::SetLastError("");
    const JValue cfg = ParseOrEmpty(session_json, "session_json");
    std::shared_ptr<ModelEntry> m;
    {
      std::lock_guard<std::mutex> lk(g_mu);
      m = ModelLocked(model);
    }
    const int32_t max_seq = AsI32(cfg.Get("max_seq"), m->default_max_seq);
    RPG_CHECK(max_seq > 0 && max_seq <= m->max_pos, "session_json.max_seq=%d must be in (0, %d]", max_seq,
              m->max_pos);
    auto s = std::make_shared<SessionEntry>();
    s->model = model;
    s->model_ref = m->model;
    s->max_tokens = AsI32(cfg.Get("max_tokens"), kDefaultMaxTokens);
    RPG_CHECK(s->max_tokens > 0, "session_json.max_tokens must be positive (got %d)", s->max_tokens);
    if (s->max_tokens >= max_seq) {
      rpg::Log(rpg::kLogWarn, "session_json.max_tokens=%d too large for max_seq=%d; clamped to %d", s->max_tokens,
               max_seq, max_seq - 1);
      s->max_tokens = max_seq - 1;
    }
    for (const JValue& v : cfg.Get("stop").items())
      if (v.IsString()) s->stop.push_back(v.str());
    s->temperature = AsF32(cfg.Get("temperature"), 0.0f);
    if (s->temperature < 0.0f) s->temperature = 0.0f;
    if (s->temperature > kMaxTemperature) s->temperature = kMaxTemperature;
    s->seed = static_cast<uint64_t>(cfg.Get("seed").Int(0));
    s->s.reset(new rpg::Session(*m->model, max_seq));
    std::lock_guard<std::mutex> lk(g_mu);
    RPG_CHECK(g_models.count(model), "model %d was unloaded during session creation", model);
    RPG_CHECK(g_next_session > 0, "session handles exhausted");
    const int32_t h = g_next_session++;
    m->sessions.push_back(h);
    g_sessions[h] = s;
    return h;
  }
  ABI_CATCH(-1)
}

void rpg_engine_session_destroy(int32_t session) {
  try {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_sessions.find(session);
    if (it == g_sessions.end()) return;
    auto mit = g_models.find(it->second->model);
    if (mit != g_models.end()) {
      auto& v = mit->second->sessions;
      for (size_t i = 0; i < v.size(); ++i) {
        if (v[i] == session) {
          v.erase(v.begin() + static_cast<long>(i));
          break;
        }
      }
    }
    g_sessions.erase(it);
  } catch (...) {
  }
}

int32_t rpg_engine_session_reset(int32_t session) {
  try {
    rpg::SetLastError("");
    std::shared_ptr<SessionEntry> s;
    {
      std::lock_guard<std::mutex> lk(g_mu);
      s = SessionLocked(session);
    }
    s->s->Reset();
    s->cached_ids.clear();
    return RPG_ENGINE_OK;
  }
  ABI_CATCH(-1)
}

char* rpg_engine_generate(int32_t session, const char* request_json) {
  try {
    rpg::SetLastError("");
    std::shared_ptr<SessionEntry> s;
    std::shared_ptr<ModelEntry> m;
    {
      std::lock_guard<std::mutex> lk(g_mu);
      s = SessionLocked(session);
      m = ModelLocked(s->model);
    }
    const rpg::ModelConfig& c = m->model->config();
    RPG_CHECK(request_json != nullptr && *request_json != '\0', "request_json is empty");
    std::string perr;
    const JValue req = JValue::Parse(request_json, &perr);
    RPG_CHECK(perr.empty(), "request_json failed to parse: %s", perr.c_str());
    RPG_CHECK(req.IsObject(), "request_json must be a JSON object");

    // ---- prompt ids: ChatML render + BBPE, or the caller's token ids
    std::vector<int32_t> ids;
    const JValue& in = req.Get("input_ids");
    const bool token_path = in.IsArray() && req.Get("messages").IsNull();
    if (token_path) {
      for (const JValue& v : in.items()) {
        RPG_CHECK(v.IsNumber(), "input_ids must hold integers");
        ids.push_back(static_cast<int32_t>(v.num()));
      }
      if (c.add_bos && c.bos_id >= 0 && (ids.empty() || ids[0] != c.bos_id)) ids.insert(ids.begin(), c.bos_id);
    } else {
      const std::vector<rpg::ChatMessage> msgs = rpg::ParseChatMessages(req.Get("messages"));
      RPG_CHECK(!msgs.empty(), "messages is empty: at least one message is required");
      RPG_CHECK(m->tok != nullptr, "the model has no BBPE vocabulary: pass \"input_ids\" instead of messages");
      const std::string prompt = rpg::RenderChatml(msgs, rpg::ParseChatTools(req.Get("tools")), true,
                                                   req.Get("enable_thinking").Bool(true));
      ids = m->tok->Encode(prompt, true);
      if (c.add_bos && c.bos_id >= 0) ids.insert(ids.begin(), c.bos_id);
    }
    const int64_t total = static_cast<int64_t>(ids.size());
    RPG_CHECK(total > 0, "the prompt is empty");

    // ---- longest common prefix with the cached ids
    int64_t lcp = 0;
    const int64_t cached = static_cast<int64_t>(s->cached_ids.size());
    RPG_CHECK(cached == s->s->len(), "internal state mismatch: cached_ids=%lld, kv.len=%lld", (long long)cached,
              (long long)s->s->len());
    while (lcp < cached && lcp < total && s->cached_ids[static_cast<size_t>(lcp)] == ids[static_cast<size_t>(lcp)])
      ++lcp;
    if (lcp == total) lcp = total - 1;  // forward at least one position
    const int64_t rows = total - lcp;

    int32_t max_tokens = AsI32(req.Get("max_tokens"), s->max_tokens);
    if (max_tokens <= 0) max_tokens = s->max_tokens;
    float temperature = AsF32(req.Get("temperature"), s->temperature);
    if (temperature < 0.0f) temperature = 0.0f;
    if (temperature > kMaxTemperature) {
      rpg::Log(rpg::kLogWarn, "temperature %.3f above %.1f; clamped", temperature, kMaxTemperature);
      temperature = kMaxTemperature;
    }
    const uint64_t seed = static_cast<uint64_t>(req.Get("seed").Int(static_cast<int64_t>(s->seed)));
    RPG_CHECK(total + max_tokens + kSeqMargin <= s->s->max_seq(),
              "sequence too long: prompt %lld + generate %d + margin %lld exceeds the session capacity %lld "
              "(raise session_json.max_seq or call session_reset)",
              (long long)total, max_tokens, (long long)kSeqMargin, (long long)s->s->max_seq());

    // ---- prefill
    s->s->SetLen(lcp);
    try {
      s->s->Prefill(ids.data() + lcp, rows, nullptr, nullptr);
      RPG_CHECK(s->s->len() == total, "after prefill kv.len=%lld, expected %lld", (long long)s->s->len(),
                (long long)total);
      s->cached_ids = ids;
    } catch (...) {
      s->s->Reset();
      s->cached_ids.clear();
      throw;
    }

    // ---- stop ids
    std::vector<int32_t> stop_ids;
    if (c.eos_id >= 0) stop_ids.push_back(c.eos_id);
    const int32_t im_end = IdOf(*m, "<|im_end|>");
    if (im_end >= 0 && (stop_ids.empty() || stop_ids[0] != im_end)) stop_ids.push_back(im_end);
    for (const JValue& v : req.Get("stop").items())
      if (v.IsString()) AppendStop(*m, v.str(), &stop_ids);
    for (const std::string& sp : s->stop) AppendStop(*m, sp, &stop_ids);

    // ---- generate
    rpg::SampleParams sp;
    sp.temperature = temperature;
    sp.top_k = kTopK;
    sp.top_p = kTopP;
    sp.seed = seed;
    // A generation that fails part way leaves the cache longer than the
    // cached ids: start the session over rather than leave that mismatch for
    // the next call to trip on.
    std::vector<int32_t> gen;
    try {
      gen = s->s->Generate(nullptr, max_tokens, sp, stop_ids, nullptr);
    } catch (...) {
      s->s->Reset();
      s->cached_ids.clear();
      throw;
    }
    s->cached_ids.insert(s->cached_ids.end(), gen.begin(), gen.end());

    // ---- decode (special tokens kept: <tool_call> is one) and parse
    const rpg::ParsedReply parsed = rpg::ParseReply(m->tok ? m->tok->Decode(gen, false) : std::string());
    std::string finish;
    if (!parsed.calls.empty())
      finish = "tool_calls";
    else if (parsed.unterminated_call || parsed.unterminated_think)
      finish = "length";
    else if (static_cast<int32_t>(gen.size()) >= max_tokens && (gen.empty() || !Contains(stop_ids, gen.back())))
      finish = "length";
    else
      finish = "stop";
    JValue resp = JValue::Object();
    resp.Set("text", JValue::String(parsed.text));
    JValue calls = JValue::Array();
    for (const rpg::ParsedCall& pc : parsed.calls) {
      JValue one = JValue::Object();
      one.Set("name", JValue::String(pc.name));
      one.Set("arguments", pc.ok ? pc.arguments : JValue());
      calls.Push(std::move(one));
    }
    resp.Set("tool_calls", std::move(calls));
    resp.Set("finish_reason", JValue::String(finish));
    JValue usage = JValue::Object();
    usage.Set("prompt_tokens", JValue::Integer(total));
    usage.Set("completion_tokens", JValue::Integer(static_cast<int64_t>(gen.size())));
    resp.Set("usage", std::move(usage));
    if (token_path) {
      JValue out = JValue::Array();
      for (int32_t id : gen) out.Push(JValue::Integer(id));
      resp.Set("output_ids", std::move(out));
    }
    return Dup(resp.Dump(false));
  }
  ABI_CATCH(nullptr)
}

void rpg_engine_free(char* buf) { delete[] buf; }

char* rpg_engine_model_info(int32_t model) {
  try {
    rpg::SetLastError("");
    std::shared_ptr<ModelEntry> m;
    size_t n_sessions = 0;
    {
      std::lock_guard<std::mutex> lk(g_mu);
      m = ModelLocked(model);
      n_sessions = m->sessions.size();
    }
    const rpg::ModelConfig& c = m->model->config();
    // the reference's keys, order and number forms (reference
    // src/engine.cc:519-547; rope_theta as the shortest round-trip double,
    // src/json.cc:317-332)
    JValue o = JValue::Object();
    o.Set("arch", JValue::String(c.arch));
    o.Set("name", JValue::String(c.name));
    o.Set("n_layers", JValue::Integer(c.n_layers));
    o.Set("hidden", JValue::Integer(c.hidden));
    o.Set("n_heads", JValue::Integer(c.n_heads));
    o.Set("n_kv_heads", JValue::Integer(c.n_kv_heads));
    o.Set("head_dim", JValue::Integer(c.head_dim));
    o.Set("intermediate", JValue::Integer(c.intermediate));
    o.Set("vocab", JValue::Integer(c.vocab));
    o.Set("context_length", JValue::Integer(c.context_length));
    o.Set("rope_theta", JValue::Num(static_cast<double>(c.rope_theta), false));
    o.Set("tied_embeddings", JValue::Boolean(c.tied_embeddings));
    o.Set("path", JValue::String(m->model->gguf().path()));
    o.Set("max_pos", JValue::Integer(m->max_pos));
    o.Set("default_max_seq", JValue::Integer(m->default_max_seq));
    o.Set("weight_bytes", JValue::Integer(m->model->weight_bytes()));
    o.Set("sessions", JValue::Integer(static_cast<int64_t>(n_sessions)));
    const std::string text = o.Dump(false);
    return Dup(text);
  }
  ABI_CATCH(nullptr)
}

}  // extern "C"
