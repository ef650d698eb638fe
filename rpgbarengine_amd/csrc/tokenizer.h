// Byte-level BPE tokenizer of Qwen models, read from the GGUF metadata
// (tokenizer.ggml.tokens / .merges / .token_type and the bos / eos / pad /
// unk ids). Behaviour of the reference tokenizer (reference
// src/tokenizer.h:1-94, src/tokenizer.cc:132-374):
//   * special tokens -- token_type 3 (control) and 4 (user-defined) -- match
//     as whole strings before any BPE, longest first, when parse_special;
//   * the text between them is split by the Qwen2 pre-tokenizer pattern
//       (?:'[sS]|'[tT]|'[rR][eE]|'[vV][eE]|'[mM]|'[lL][lL]|'[dD])
//       |[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*
//       |\s*[\r\n]+|\s+(?!\S)|\s+
//     with leftmost-first alternation (no Unicode normalisation);
//   * each piece's bytes map to GPT-2 byte characters and merge pair by
//     pair, the lowest-ranked adjacent pair first (the leftmost on ties),
//     one merge at a time; a merged symbol missing from the vocabulary falls
//     back to its single-byte tokens;
//   * decoding maps byte characters back to bytes and passes other code
//     points through as UTF-8.
// CPU code: the text front-end runs on the host around the GPU token loop.

#ifndef RPG_HIP_TOKENIZER_H_
#define RPG_HIP_TOKENIZER_H_

#include <cstdint>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace rpg {

class GgufFile;

class Tokenizer {
 public:
  // Throws when the GGUF holds no token list or no merges.
  static Tokenizer FromGguf(const GgufFile& g);

  std::vector<int32_t> Encode(const std::string& text, bool parse_special) const;
  std::string Decode(const std::vector<int32_t>& ids, bool skip_special) const;
  // The pre-tokenizer's pieces of a text without special tokens.
  std::vector<std::string> Split(const std::string& text) const;

  int32_t IdOf(const std::string& token) const;  // -1 when absent
  bool IsSpecial(int32_t id) const;
  size_t size() const { return tokens_.size(); }
  int32_t bos() const { return bos_; }
  int32_t eos() const { return eos_; }

 private:
  void EncodePiece(const std::string& piece, std::vector<int32_t>* out) const;
  void EncodeText(const std::string& text, std::vector<int32_t>* out) const;
  int32_t Rank(const std::string& a, const std::string& b) const;

  std::vector<std::string> tokens_;
  std::vector<uint8_t> types_;
  std::unordered_map<std::string, int32_t> ids_;     // the first id of a token string wins
  std::unordered_map<std::string, int32_t> ranks_;   // "left\x1Fright" -> merge rank (the first wins)
  std::vector<std::pair<std::string, int32_t>> specials_;  // longest first
  int32_t bos_ = -1, eos_ = -1, pad_ = -1, unk_ = -1;
};

}  // namespace rpg

#endif  // RPG_HIP_TOKENIZER_H_
