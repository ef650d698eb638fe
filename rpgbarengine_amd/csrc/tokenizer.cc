#include "tokenizer.h"

#include <algorithm>
#include <climits>

#include "common.h"
#include "gguf.h"
#include "unicode.h"

namespace rpg {
namespace {

struct Cps {
  std::vector<uint32_t> cp;
  std::vector<size_t> off;  // byte offset of each code point; off[n] = size
};

Cps DecodeCps(const std::string& s) {
  Cps c;
  size_t i = 0;
  while (i < s.size()) {
    const uni::Decoded d = uni::DecodeUtf8(s.data() + i, s.size() - i);
    c.cp.push_back(d.cp);
    c.off.push_back(i);
    i += static_cast<size_t>(d.len);
  }
  c.off.push_back(s.size());
  return c;
}

inline bool Newline(uint32_t c) { return c == '\r' || c == '\n'; }

// The pre-tokenizer pattern at code point p: the length (in code points) of
// the match of its first alternative that matches, with each alternative's
// own greedy / backtracking preference.
size_t MatchAt(const std::vector<uint32_t>& cp, size_t p) {
  const size_t m = cp.size();
  const uint32_t c = cp[p];
  auto letter = [&](size_t i) { return uni::IsLetter(cp[i]); };
  auto number = [&](size_t i) { return uni::IsNumber(cp[i]); };
  auto space = [&](size_t i) { return uni::IsSpace(cp[i]); };
  auto ascii_lower = [](uint32_t x) { return (x >= 'A' && x <= 'Z') ? x + 32 : x; };

  // 'S 'T 'RE 'VE 'M 'LL 'D in either case
  if (c == '\'' && p + 1 < m) {
    const uint32_t a = ascii_lower(cp[p + 1]);
    if (a == 's' || a == 't' || a == 'm' || a == 'd') return 2;
    if (p + 2 < m) {
      const uint32_t b = ascii_lower(cp[p + 2]);
      if ((a == 'r' || a == 'v') && b == 'e') return 3;
      if (a == 'l' && b == 'l') return 3;
    }
  }
  // [^\r\n\p{L}\p{N}]?\p{L}+ : the optional prefix is taken when c can be
  // one; giving it back cannot help (then c itself would have to be a letter)
  {
    const size_t q = (!Newline(c) && !letter(p) && !number(p)) ? p + 1 : p;
    size_t r = q;
    while (r < m && letter(r)) ++r;
    if (r > q) return r - p;
  }
  // \p{N}
  if (number(p)) return 1;
  //  ?[^\s\p{L}\p{N}]+[\r\n]*
  {
    const size_t q = c == ' ' ? p + 1 : p;
    size_t r = q;
    while (r < m && !space(r) && !letter(r) && !number(r)) ++r;
    if (r > q) {
      while (r < m && Newline(cp[r])) ++r;
      return r - p;
    }
  }
  // whitespace run [p, e)
  size_t e = p;
  while (e < m && space(e)) ++e;
  // \s*[\r\n]+ : \s* gives back down to the run's last line break
  for (size_t k = e; k > p; --k)
    if (Newline(cp[k - 1])) return k - p;
  // \s+(?!\S) : the whole run at the end of the text, else all but its last
  if (e == m) return e - p;
  if (e - p >= 2) return e - 1 - p;
  // \s+
  return std::max<size_t>(e - p, 1);
}

}  // namespace

Tokenizer Tokenizer::FromGguf(const GgufFile& g) {
  Tokenizer t;
  const std::vector<std::string>* toks = g.StrArray("tokenizer.ggml.tokens");
  RPG_CHECK(toks != nullptr && !toks->empty(), "the GGUF holds no tokenizer.ggml.tokens");
  const std::vector<std::string>* merges = g.StrArray("tokenizer.ggml.merges");
  RPG_CHECK(merges != nullptr && !merges->empty(), "the GGUF holds no tokenizer.ggml.merges (BBPE needs them)");
  t.tokens_ = *toks;
  t.ids_.reserve(t.tokens_.size() * 2);
  for (size_t i = 0; i < t.tokens_.size(); ++i) t.ids_.emplace(t.tokens_[i], static_cast<int32_t>(i));
  t.types_.assign(t.tokens_.size(), 1);
  if (const std::vector<double>* ty = g.NumArray("tokenizer.ggml.token_type")) {
    RPG_CHECK(ty->size() == t.tokens_.size(), "tokenizer.ggml.token_type has %zu entries for %zu tokens", ty->size(),
              t.tokens_.size());
    for (size_t i = 0; i < ty->size(); ++i) t.types_[i] = static_cast<uint8_t>((*ty)[i]);
  }
  t.ranks_.reserve(merges->size() * 2);
  for (size_t i = 0; i < merges->size(); ++i) {
    const std::string& m = (*merges)[i];
    const size_t sp = m.find(' ');
    RPG_CHECK(sp != std::string::npos, "merge %zu has no space: %s", i, m.c_str());
    t.ranks_.emplace(m.substr(0, sp) + '\x1F' + m.substr(sp + 1), static_cast<int32_t>(i));
  }
  for (size_t i = 0; i < t.tokens_.size(); ++i)
    if (t.types_[i] == 3 || t.types_[i] == 4) t.specials_.emplace_back(t.tokens_[i], static_cast<int32_t>(i));
  std::stable_sort(t.specials_.begin(), t.specials_.end(),
                   [](const std::pair<std::string, int32_t>& a, const std::pair<std::string, int32_t>& b) {
                     return a.first.size() > b.first.size();
                   });
  t.bos_ = static_cast<int32_t>(g.Int("tokenizer.ggml.bos_token_id", -1));
  t.eos_ = static_cast<int32_t>(g.Int("tokenizer.ggml.eos_token_id", -1));
  t.pad_ = static_cast<int32_t>(g.Int("tokenizer.ggml.padding_token_id", -1));
  t.unk_ = static_cast<int32_t>(g.Int("tokenizer.ggml.unknown_token_id", -1));
  return t;
}

int32_t Tokenizer::IdOf(const std::string& token) const {
  auto it = ids_.find(token);
  return it == ids_.end() ? -1 : it->second;
}

bool Tokenizer::IsSpecial(int32_t id) const {
  return id >= 0 && static_cast<size_t>(id) < types_.size() && (types_[id] == 3 || types_[id] == 4);
}

int32_t Tokenizer::Rank(const std::string& a, const std::string& b) const {
  std::string key;
  key.reserve(a.size() + b.size() + 1);
  key += a;
  key += '\x1F';
  key += b;
  auto it = ranks_.find(key);
  return it == ranks_.end() ? -1 : it->second;
}

std::vector<std::string> Tokenizer::Split(const std::string& text) const {
  std::vector<std::string> pieces;
  const Cps c = DecodeCps(text);
  for (size_t p = 0; p < c.cp.size();) {
    const size_t end = p + MatchAt(c.cp, p);
    pieces.push_back(text.substr(c.off[p], c.off[end] - c.off[p]));
    p = end;
  }
  return pieces;
}

void Tokenizer::EncodePiece(const std::string& piece, std::vector<int32_t>* out) const {
  if (piece.empty()) return;
  // one symbol per byte, spelled as its GPT-2 character
  std::vector<std::string> sym;
  sym.reserve(piece.size());
  for (unsigned char b : piece) {
    std::string s;
    uni::AppendUtf8(uni::ByteToCp(b), &s);
    sym.push_back(std::move(s));
  }
  // rank[i]: merge rank of (sym[i], sym[i + 1]), -1 when none; each round
  // merges the lowest-ranked pair, the leftmost of equals
  std::vector<int32_t> rank(sym.size() > 1 ? sym.size() - 1 : 0);
  for (size_t i = 0; i + 1 < sym.size(); ++i) rank[i] = Rank(sym[i], sym[i + 1]);
  for (;;) {
    size_t best = SIZE_MAX;
    int32_t best_rank = INT32_MAX;
    for (size_t i = 0; i < rank.size(); ++i)
      if (rank[i] >= 0 && rank[i] < best_rank) best_rank = rank[i], best = i;
    if (best == SIZE_MAX) break;
    sym[best] += sym[best + 1];
    sym.erase(sym.begin() + static_cast<long>(best) + 1);
    rank.erase(rank.begin() + static_cast<long>(best));
    if (best > 0) rank[best - 1] = Rank(sym[best - 1], sym[best]);
    if (best < rank.size()) rank[best] = Rank(sym[best], sym[best + 1]);
  }
  for (const std::string& s : sym) {
    const int32_t id = IdOf(s);
    if (id >= 0) {
      out->push_back(id);
      continue;
    }
    // not in the vocabulary: its bytes one token each
    const Cps c = DecodeCps(s);
    for (uint32_t cp : c.cp) {
      const int b = uni::CpToByte(cp);
      RPG_CHECK(b >= 0, "symbol %s is neither a token nor byte characters", s.c_str());
      std::string one;
      uni::AppendUtf8(uni::ByteToCp(static_cast<uint8_t>(b)), &one);
      const int32_t bid = IdOf(one);
      RPG_CHECK(bid >= 0, "byte 0x%02X has no token in the vocabulary", b);
      out->push_back(bid);
    }
  }
}

void Tokenizer::EncodeText(const std::string& text, std::vector<int32_t>* out) const {
  for (const std::string& piece : Split(text)) EncodePiece(piece, out);
}

std::vector<int32_t> Tokenizer::Encode(const std::string& text, bool parse_special) const {
  std::vector<int32_t> out;
  if (!parse_special) {
    EncodeText(text, &out);
    return out;
  }
  size_t plain = 0, i = 0;
  while (i < text.size()) {
    const std::pair<std::string, int32_t>* hit = nullptr;
    for (const auto& sp : specials_) {
      if (sp.first.size() <= text.size() - i && text.compare(i, sp.first.size(), sp.first) == 0) {
        hit = &sp;
        break;
      }
    }
    if (hit == nullptr) {
      ++i;
      continue;
    }
    if (i > plain) EncodeText(text.substr(plain, i - plain), &out);
    out.push_back(hit->second);
    i += hit->first.size();
    plain = i;
  }
  if (plain < text.size()) EncodeText(text.substr(plain), &out);
  return out;
}

std::string Tokenizer::Decode(const std::vector<int32_t>& ids, bool skip_special) const {
  std::string out;
  for (int32_t id : ids) {
    if (id < 0 || static_cast<size_t>(id) >= tokens_.size()) continue;
    if (skip_special && IsSpecial(id)) continue;
    const Cps c = DecodeCps(tokens_[static_cast<size_t>(id)]);
    for (uint32_t cp : c.cp) {
      const int b = uni::CpToByte(cp);
      if (b >= 0)
        out.push_back(static_cast<char>(b));
      else
        uni::AppendUtf8(cp, &out);
    }
  }
  return out;
}

}  // namespace rpg
