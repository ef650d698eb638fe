// ref_golden -- drives the *reference* engine's own internal API and writes
// its answers as raw little-endian files (float32 / int32).
//
// This is test infrastructure: it is compiled (by oracle/Makefile, target
// `ref`) against the reference sources where they lie and linked with the
// reference's own objects, with the reference's own flags (-O2 -std=c++20,
// -mavx2 -mfma on src/matmul_avx2.cc only, reference CMakeLists.txt:18,44-49).
// Its outputs pin the CPU restatement in oracle/cpu_ref and serve as the
// "reference" CPU baseline in bench.py. Nothing in the product links it.
//
// Subcommands (all paths are files of raw values):
//   dequant  TYPE N IN OUT                      DequantizeRow (src/quant.cc:416)
//   dot      TYPE K ROWS W A OUT_DISPATCH OUT_SCALAR
//                                              DotRowQuant / DotRowQuantRef per row
//                                              (src/matmul.cc:73-108)
//   matmul   TYPE ROWS COLS W X N THREADS OUT   QuantMatrix::MatMulBatch (src/model.cc:39-69)
//   kernels  OP N IN OUT [args]                 rmsnorm|softmax|silu|rope|argmax (src/kernels.h)
//   sample   N LOGITS T TOPK TOPP U OUT_PROBS   FilterToProbs + SampleToken (src/sampler.cc)
//   uniform  SEED COUNTER COUNT OUT             CounterUniform (src/sampler.cc:16-34)
//   model    GGUF [options]                     Model::Load + ForwardFull + Generate
//            --ids FILE --n N                  prompt ids (int32)
//            --threads T --max-seq S
//            --logits-out FILE                  all-row logits of the prefill ([n, vocab])
//            --last-logits-out FILE             last-row logits of the prefill ([vocab])
//            --nocache-logits-out FILE          ForwardFull without KV cache ([n, vocab])
//            --gen N --temp T --top-k K --top-p P --seed S --gen-out FILE
//            --step-logits-out FILE             logits after each generated token ([gen, vocab])
//            --time                             print prefill/decode timings as JSON
//   unicode  OUT                                one byte per code point 0..0x10FFFF: bit 0 letter,
//                                              bit 1 number, bit 2 space (src/unicode.h)
//   text     GGUF IN OUT                        per text of IN: Encode with and without special
//                                              tokens, PreTokenize, Decode of the first with and
//                                              without specials (src/tokenizer.cc:132-372)
//   chatml   IN OUT                             per request JSON of IN: RenderChatml of its
//                                              messages / tools / enable_thinking
//                                              (src/chat_template.cc)
//   reply    IN OUT                             per text of IN: ParseModelOutput as JSON
//                                              (src/tool_parser.cc)
//   json     IN OUT                             per JSON text of IN: Dump and DumpPython
// IN / OUT of the text modes: records of u32 length + bytes; an OUT record of
// int32 ids is u32 count + ids.

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "chat_template.h"
#include "common.h"
#include "gguf.h"
#include "json.h"
#include "kernels.h"
#include "kv_cache.h"
#include "matmul.h"
#include "model.h"
#include "quant.h"
#include "qwen3.h"
#include "sampler.h"
#include "threads.h"
#include "tokenizer.h"
#include "tool_parser.h"
#include "unicode.h"

namespace {

template <typename T>
std::vector<T> ReadRaw(const std::string& path) {
  std::FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) rpg::Throw("cannot open %s", path.c_str());
  std::fseek(f, 0, SEEK_END);
  const long n = std::ftell(f);
  std::fseek(f, 0, SEEK_SET);
  std::vector<T> v(static_cast<size_t>(n) / sizeof(T));
  if (!v.empty() && std::fread(v.data(), sizeof(T), v.size(), f) != v.size())
    rpg::Throw("short read %s", path.c_str());
  std::fclose(f);
  return v;
}

template <typename T>
void WriteRaw(const std::string& path, const T* p, size_t n) {
  std::FILE* f = std::fopen(path.c_str(), "wb");
  if (!f) rpg::Throw("cannot write %s", path.c_str());
  if (n && std::fwrite(p, sizeof(T), n, f) != n) rpg::Throw("short write %s", path.c_str());
  std::fclose(f);
}

int CmdDequant(int argc, char** argv) {
  if (argc < 6) return 2;
  const uint32_t type = static_cast<uint32_t>(std::atoi(argv[2]));
  const int64_t n = std::atoll(argv[3]);
  const std::vector<uint8_t> in = ReadRaw<uint8_t>(argv[4]);
  std::vector<float> out(static_cast<size_t>(n));
  rpg::DequantizeRow(type, in.data(), n, out.data());
  WriteRaw(argv[5], out.data(), out.size());
  return 0;
}

int CmdDot(int argc, char** argv) {
  if (argc < 9) return 2;
  const uint32_t type = static_cast<uint32_t>(std::atoi(argv[2]));
  const int64_t k = std::atoll(argv[3]);
  const int64_t rows = std::atoll(argv[4]);
  const std::vector<uint8_t> w = ReadRaw<uint8_t>(argv[5]);
  const std::vector<float> a = ReadRaw<float>(argv[6]);
  const int64_t rb = rpg::TypeRowBytes(type, k);
  std::vector<float> o1(static_cast<size_t>(rows)), o2(static_cast<size_t>(rows));
  for (int64_t r = 0; r < rows; ++r) {
    o1[r] = rpg::DotRowQuant(type, a.data(), w.data() + r * rb, k);
    o2[r] = rpg::DotRowQuantRef(type, a.data(), w.data() + r * rb, k);
  }
  WriteRaw(argv[7], o1.data(), o1.size());
  WriteRaw(argv[8], o2.data(), o2.size());
  std::printf("kernel=%s\n", rpg::ActiveKernelName());
  return 0;
}

int CmdMatmul(int argc, char** argv) {
  if (argc < 10) return 2;
  const uint32_t type = static_cast<uint32_t>(std::atoi(argv[2]));
  const int64_t rows = std::atoll(argv[3]);
  const int64_t cols = std::atoll(argv[4]);
  const std::vector<uint8_t> w = ReadRaw<uint8_t>(argv[5]);
  const std::vector<float> x = ReadRaw<float>(argv[6]);
  const int64_t n = std::atoll(argv[7]);
  const int threads = std::atoi(argv[8]);
  rpg::QuantMatrix m(w.data(), type, rows, cols);
  rpg::ThreadPool pool(threads > 0 ? threads : 1);
  std::vector<float> out(static_cast<size_t>(n * rows), 0.0f);
  m.MatMulBatch(x.data(), n, out.data(), &pool);
  WriteRaw(argv[9], out.data(), out.size());
  return 0;
}

int CmdKernels(int argc, char** argv) {
  if (argc < 6) return 2;
  const std::string op = argv[2];
  const int64_t n = std::atoll(argv[3]);
  std::vector<float> in = ReadRaw<float>(argv[4]);
  std::vector<float> out(in.size(), 0.0f);
  if (op == "rmsnorm") {
    // in = [x (n) | w (n)], argv[6] = eps
    const float eps = std::strtof(argv[6], nullptr);
    rpg::RmsNorm(in.data(), in.data() + n, n, eps, out.data());
    out.resize(static_cast<size_t>(n));
  } else if (op == "softmax") {
    out = in;
    rpg::SoftmaxInPlace(out.data(), n);
  } else if (op == "silu") {
    out = in;
    rpg::SiluInPlace(out.data(), n);
  } else if (op == "rope") {
    // in = [x (heads*hd) | cos (hd/2) | sin (hd/2)], argv[6] = heads, argv[7] = head_dim
    const int heads = std::atoi(argv[6]);
    const int hd = std::atoi(argv[7]);
    out.assign(in.begin(), in.begin() + static_cast<int64_t>(heads) * hd);
    const float* c = in.data() + static_cast<int64_t>(heads) * hd;
    rpg::RopeInPlace(out.data(), heads, hd, c, c + hd / 2);
  } else if (op == "argmax") {
    const int32_t a = rpg::ArgMax(in.data(), n);
    WriteRaw(argv[5], &a, 1);
    return 0;
  } else if (op == "dot") {
    // in = [a (n) | b (n)]
    const float d = rpg::Dot(in.data(), in.data() + n, n);
    WriteRaw(argv[5], &d, 1);
    return 0;
  } else {
    return 2;
  }
  WriteRaw(argv[5], out.data(), out.size());
  return 0;
}

int CmdSample(int argc, char** argv) {
  if (argc < 9) return 2;
  const int64_t n = std::atoll(argv[2]);
  const std::vector<float> logits = ReadRaw<float>(argv[3]);
  rpg::SampleOptions opt;
  opt.temperature = std::strtof(argv[4], nullptr);
  opt.top_k = std::atoi(argv[5]);
  opt.top_p = std::strtof(argv[6], nullptr);
  const float u = std::strtof(argv[7], nullptr);
  std::vector<float> probs;
  rpg::FilterToProbs(logits.data(), n, opt, &probs);
  WriteRaw(argv[8], probs.data(), probs.size());
  const int32_t tok = rpg::SampleToken(logits.data(), n, opt, u);
  std::printf("%d\n", tok);
  return 0;
}

int CmdUniform(int argc, char** argv) {
  if (argc < 6) return 2;
  const uint64_t seed = std::strtoull(argv[2], nullptr, 10);
  const uint64_t c0 = std::strtoull(argv[3], nullptr, 10);
  const int64_t cnt = std::atoll(argv[4]);
  std::vector<float> u(static_cast<size_t>(cnt));
  for (int64_t i = 0; i < cnt; ++i) u[i] = rpg::CounterUniform(seed, c0 + static_cast<uint64_t>(i));
  WriteRaw(argv[5], u.data(), u.size());
  return 0;
}

int CmdModel(int argc, char** argv) {
  if (argc < 3) return 2;
  const std::string path = argv[2];
  std::string ids_path, logits_out, last_out, nocache_out, gen_out, step_out;
  int64_t n = -1, max_seq = 0;
  int threads = 0, gen = 0, top_k = 0;
  float temp = 0.0f, top_p = 1.0f;
  uint64_t seed = 0;
  bool timing = false;
  for (int i = 3; i < argc; ++i) {
    const std::string a = argv[i];
    auto next = [&]() -> const char* {
      if (i + 1 >= argc) rpg::Throw("missing value after %s", a.c_str());
      return argv[++i];
    };
    if (a == "--ids") ids_path = next();
    else if (a == "--n") n = std::atoll(next());
    else if (a == "--threads") threads = std::atoi(next());
    else if (a == "--max-seq") max_seq = std::atoll(next());
    else if (a == "--logits-out") logits_out = next();
    else if (a == "--last-logits-out") last_out = next();
    else if (a == "--nocache-logits-out") nocache_out = next();
    else if (a == "--gen") gen = std::atoi(next());
    else if (a == "--temp") temp = std::strtof(next(), nullptr);
    else if (a == "--top-k") top_k = std::atoi(next());
    else if (a == "--top-p") top_p = std::strtof(next(), nullptr);
    else if (a == "--seed") seed = std::strtoull(next(), nullptr, 10);
    else if (a == "--gen-out") gen_out = next();
    else if (a == "--step-logits-out") step_out = next();
    else if (a == "--time") timing = true;
    else rpg::Throw("unknown option %s", a.c_str());
  }
  std::vector<int32_t> ids = ReadRaw<int32_t>(ids_path);
  if (n >= 0 && n < static_cast<int64_t>(ids.size())) ids.resize(static_cast<size_t>(n));
  const int64_t seq = static_cast<int64_t>(ids.size());
  rpg::Model model = rpg::Model::Load(path, threads, 4096);
  const rpg::ModelConfig& c = model.config();
  if (max_seq <= 0) max_seq = seq + gen + 8;
  rpg::ForwardScratch scratch;

  if (!nocache_out.empty()) {
    std::vector<float> plain;
    rpg::ForwardFull(model, ids.data(), seq, &scratch, &plain);
    WriteRaw(nocache_out, plain.data(), plain.size());
  }

  rpg::KvCache kv(c, max_seq);
  std::vector<float> logits;
  // page the weights in before timing (reference tools/prefill_prof.cc:286-296)
  if (timing) {
    rpg::KvCache warm(c, 2);
    std::vector<float> wl;
    rpg::ForwardFull(model, ids.data(), 1, &scratch, &wl, rpg::ForwardOptions(), &warm);
  }
  const auto t0 = std::chrono::steady_clock::now();
  rpg::ForwardFull(model, ids.data(), seq, &scratch, &logits, rpg::ForwardOptions(), &kv);
  const auto t1 = std::chrono::steady_clock::now();
  if (!logits_out.empty()) WriteRaw(logits_out, logits.data(), logits.size());
  const float* last = logits.data() + (seq - 1) * c.vocab;
  if (!last_out.empty()) WriteRaw(last_out, last, static_cast<size_t>(c.vocab));

  double decode_ms = 0.0;
  std::vector<int32_t> out;
  if (gen > 0) {
    rpg::GenerateOptions g;
    g.max_tokens = gen;
    g.sample.temperature = temp;
    g.sample.top_k = top_k;
    g.sample.top_p = top_p;
    g.seed = seed;
    if (!step_out.empty()) {
      // Generate's own loop, restated with the per-step logits kept: one
      // forward per returned token (src/qwen3.cc:317-354).
      std::vector<float> cur(last, last + c.vocab);
      std::vector<float> all;
      const bool greedy = !(g.sample.temperature > 0.0f);
      for (int i = 0; i < gen; ++i) {
        int32_t next;
        if (greedy) {
          next = rpg::ArgMax(cur.data(), c.vocab);
        } else {
          const float u = rpg::CounterUniform(seed, static_cast<uint64_t>(kv.len()));
          next = rpg::SampleToken(cur.data(), c.vocab, g.sample, u);
        }
        out.push_back(next);
        rpg::ForwardStep(model, next, kv.len(), &kv, &scratch, &cur);
        all.insert(all.end(), cur.begin(), cur.end());
      }
      WriteRaw(step_out, all.data(), all.size());
    } else {
      const auto t2 = std::chrono::steady_clock::now();
      rpg::Generate(model, &kv, &scratch, last, g, &out);
      const auto t3 = std::chrono::steady_clock::now();
      decode_ms = std::chrono::duration<double, std::milli>(t3 - t2).count();
    }
    if (!gen_out.empty()) WriteRaw(gen_out, out.data(), out.size());
  }
  if (timing) {
    const double prefill_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    std::printf("{\"prefill_tokens\": %lld, \"prefill_ms\": %.3f, \"decode_tokens\": %zu, "
                "\"decode_ms\": %.3f, \"threads\": %d}\n",
                static_cast<long long>(seq), prefill_ms, out.size(), decode_ms, model.pool().size());
  }
  return 0;
}

std::vector<std::string> ReadRecords(const std::string& path) {
  const std::vector<uint8_t> raw = ReadRaw<uint8_t>(path);
  std::vector<std::string> out;
  size_t i = 0;
  while (i + 4 <= raw.size()) {
    uint32_t n;
    std::memcpy(&n, raw.data() + i, 4);
    i += 4;
    if (i + n > raw.size()) rpg::Throw("truncated record in %s", path.c_str());
    out.emplace_back(reinterpret_cast<const char*>(raw.data() + i), n);
    i += n;
  }
  return out;
}

struct RecordWriter {
  std::FILE* f;
  explicit RecordWriter(const std::string& path) : f(std::fopen(path.c_str(), "wb")) {
    if (!f) rpg::Throw("cannot open %s", path.c_str());
  }
  ~RecordWriter() { std::fclose(f); }
  void Bytes(const std::string& s) {
    const uint32_t n = static_cast<uint32_t>(s.size());
    std::fwrite(&n, 4, 1, f);
    std::fwrite(s.data(), 1, s.size(), f);
  }
  void Ids(const std::vector<int32_t>& v) {
    const uint32_t n = static_cast<uint32_t>(v.size());
    std::fwrite(&n, 4, 1, f);
    if (n) std::fwrite(v.data(), 4, v.size(), f);
  }
};

int CmdUnicode(int argc, char** argv) {
  if (argc != 3) return 2;
  std::vector<uint8_t> cls(0x110000);
  for (uint32_t cp = 0; cp < 0x110000; ++cp)
    cls[cp] = static_cast<uint8_t>((rpg::IsUnicodeLetter(cp) ? 1 : 0) | (rpg::IsUnicodeNumber(cp) ? 2 : 0) |
                                   (rpg::IsUnicodeSpace(cp) ? 4 : 0));
  WriteRaw(argv[2], cls.data(), cls.size());
  return 0;
}

int CmdText(int argc, char** argv) {
  if (argc != 5) return 2;
  const rpg::GgufFile g = rpg::GgufFile::Open(argv[2]);
  const rpg::Tokenizer tok = rpg::Tokenizer::FromGguf(g);
  RecordWriter w(argv[4]);
  for (const std::string& t : ReadRecords(argv[3])) {
    const std::vector<int32_t> ids = tok.Encode(t, true);
    w.Ids(ids);
    w.Ids(tok.Encode(t, false));
    std::vector<int32_t> lens;
    for (const std::string& p : tok.PreTokenize(t)) lens.push_back(static_cast<int32_t>(p.size()));
    w.Ids(lens);
    w.Bytes(tok.Decode(ids, false));
    w.Bytes(tok.Decode(ids, true));
  }
  return 0;
}

int CmdChatml(int argc, char** argv) {
  if (argc != 4) return 2;
  RecordWriter w(argv[3]);
  for (const std::string& t : ReadRecords(argv[2])) {
    std::string err;
    const rpg::Json req = rpg::Json::Parse(t, &err);
    if (!err.empty()) rpg::Throw("bad request JSON: %s", err.c_str());
    rpg::ChatTemplateOptions opt;
    opt.add_generation_prompt = true;
    opt.enable_thinking = req.Get("enable_thinking").AsBool(true);
    w.Bytes(rpg::RenderChatml(rpg::ParseMessages(req.Get("messages")), rpg::ParseTools(req.Get("tools")), opt));
  }
  return 0;
}

int CmdReply(int argc, char** argv) {
  if (argc != 4) return 2;
  RecordWriter w(argv[3]);
  for (const std::string& t : ReadRecords(argv[2])) {
    const rpg::ParsedOutput p = rpg::ParseModelOutput(t);
    rpg::Json o = rpg::Json::Object();
    o.Set("text", p.text);
    o.Set("reasoning", p.reasoning);
    rpg::Json calls = rpg::Json::Array();
    for (const rpg::ParsedToolCall& c : p.tool_calls) {
      rpg::Json one = rpg::Json::Object();
      one.Set("name", c.name);
      one.Set("arguments_raw", c.arguments_raw);
      one.Set("arguments", c.arguments);
      one.Set("ok", c.ok);
      calls.PushBack(std::move(one));
    }
    o.Set("tool_calls", std::move(calls));
    o.Set("unterminated_think", p.unterminated_think);
    o.Set("unterminated_tool_call", p.unterminated_tool_call);
    w.Bytes(o.Dump(false));
  }
  return 0;
}

int CmdJson(int argc, char** argv) {
  if (argc != 4) return 2;
  RecordWriter w(argv[3]);
  for (const std::string& t : ReadRecords(argv[2])) {
    std::string err;
    const rpg::Json j = rpg::Json::Parse(t, &err);
    w.Bytes(err.empty() ? j.Dump(false) : std::string("\x01") + "error");
    w.Bytes(err.empty() ? j.DumpPython() : std::string("\x01") + "error");
  }
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    std::fprintf(stderr, "usage: ref_golden dequant|dot|matmul|kernels|sample|uniform|model ...\n");
    return 2;
  }
  try {
    const std::string cmd = argv[1];
    int rc = 2;
    if (cmd == "dequant") rc = CmdDequant(argc, argv);
    else if (cmd == "dot") rc = CmdDot(argc, argv);
    else if (cmd == "matmul") rc = CmdMatmul(argc, argv);
    else if (cmd == "kernels") rc = CmdKernels(argc, argv);
    else if (cmd == "sample") rc = CmdSample(argc, argv);
    else if (cmd == "uniform") rc = CmdUniform(argc, argv);
    else if (cmd == "model") rc = CmdModel(argc, argv);
    else if (cmd == "unicode") rc = CmdUnicode(argc, argv);
    else if (cmd == "text") rc = CmdText(argc, argv);
    else if (cmd == "chatml") rc = CmdChatml(argc, argv);
    else if (cmd == "reply") rc = CmdReply(argc, argv);
    else if (cmd == "json") rc = CmdJson(argc, argv);
    if (rc == 2) std::fprintf(stderr, "bad arguments for %s\n", cmd.c_str());
    return rc;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 1;
  }
}
