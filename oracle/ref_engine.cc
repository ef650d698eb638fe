// ref_engine -- drives the *reference* library's C ABI (include/rpg_engine.h,
// src/engine.cc) through a scripted conversation and records its answers.
// Test infrastructure: compiled by oracle/Makefile (target `ref`) against the
// reference sources where they lie; nothing in the product links it.
//
//   ref_engine SCRIPT OUT
// SCRIPT: records (u32 length + bytes): the GGUF path, config_json,
// session_json, then one request_json per call to rpg_engine_generate (the
// record "!reset" calls rpg_engine_session_reset instead). OUT: one record per
// call: the response, or "\x01" + rpg_engine_last_error() on failure. The
// record "!info" calls rpg_engine_model_info on the model instead.

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "rpg_engine.h"

namespace {

std::vector<std::string> ReadRecords(const char* path) {
  std::vector<std::string> out;
  std::FILE* f = std::fopen(path, "rb");
  if (!f) return out;
  for (;;) {
    uint32_t n;
    if (std::fread(&n, 4, 1, f) != 1) break;
    std::string s(n, '\0');
    if (n && std::fread(&s[0], 1, n, f) != n) break;
    out.push_back(std::move(s));
  }
  std::fclose(f);
  return out;
}

void Put(std::FILE* f, const std::string& s) {
  const uint32_t n = static_cast<uint32_t>(s.size());
  std::fwrite(&n, 4, 1, f);
  std::fwrite(s.data(), 1, s.size(), f);
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 3) {
    std::fprintf(stderr, "usage: ref_engine SCRIPT OUT\n");
    return 2;
  }
  const std::vector<std::string> rec = ReadRecords(argv[1]);
  if (rec.size() < 3) {
    std::fprintf(stderr, "script needs a model path, config_json and session_json\n");
    return 2;
  }
  const int32_t model = rpg_engine_load_model(rec[0].c_str(), rec[1].c_str());
  if (model < 0) {
    std::fprintf(stderr, "load_model: %s\n", rpg_engine_last_error());
    return 1;
  }
  const int32_t session = rpg_engine_session_create(model, rec[2].c_str());
  if (session < 0) {
    std::fprintf(stderr, "session_create: %s\n", rpg_engine_last_error());
    return 1;
  }
  std::FILE* out = std::fopen(argv[2], "wb");
  if (!out) return 1;
  for (size_t i = 3; i < rec.size(); ++i) {
    if (rec[i] == "!info") {
      char* r = rpg_engine_model_info(model);
      if (r == nullptr) {
        Put(out, std::string("\x01") + rpg_engine_last_error());
      } else {
        Put(out, r);
        rpg_engine_free(r);
      }
      continue;
    }
    if (rec[i] == "!reset") {
      Put(out, rpg_engine_session_reset(session) == RPG_ENGINE_OK ? std::string("ok")
                                                                  : std::string("\x01") + rpg_engine_last_error());
      continue;
    }
    char* r = rpg_engine_generate(session, rec[i].c_str());
    if (r == nullptr) {
      Put(out, std::string("\x01") + rpg_engine_last_error());
    } else {
      Put(out, r);
      rpg_engine_free(r);
    }
  }
  std::fclose(out);
  rpg_engine_session_destroy(session);
  rpg_engine_unload_model(model);
  return 0;
}
