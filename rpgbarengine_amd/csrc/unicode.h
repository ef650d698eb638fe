// UTF-8, the GPT-2 byte <-> code point map and the code-point classes of
// the BBPE pre-tokenizer (reference src/unicode.h:1-164).
//
// Decoding is lenient in the reference's way: a byte that does not start a
// well-formed sequence (bad lead byte, truncated or broken continuation,
// overlong form, surrogate) reads as U+FFFD and consumes one byte; four-byte
// leads F0..F7 are taken as they come (no cap at U+10FFFF).

#ifndef RPG_HIP_UNICODE_H_
#define RPG_HIP_UNICODE_H_

#include <cstddef>
#include <cstdint>
#include <string>

#include "unicode_tables.h"

namespace rpg {
namespace uni {

template <size_t N>
inline bool InTable(const CodeRange (&t)[N], uint32_t cp) {
  size_t lo = 0, hi = N;
  while (lo < hi) {
    const size_t mid = (lo + hi) / 2;
    if (cp < t[mid].lo)
      hi = mid;
    else if (cp > t[mid].hi)
      lo = mid + 1;
    else
      return true;
  }
  return false;
}

inline bool IsLetter(uint32_t cp) { return InTable(kLetter, cp); }
inline bool IsNumber(uint32_t cp) { return InTable(kNumber, cp); }
inline bool IsSpace(uint32_t cp) { return InTable(kSpace, cp); }

struct Decoded {
  uint32_t cp;
  int len;  // bytes consumed (1..4), 0 only at the end of input
};

inline Decoded DecodeUtf8(const char* s, size_t n) {
  if (n == 0) return {0, 0};
  const uint8_t* p = reinterpret_cast<const uint8_t*>(s);
  const uint32_t b = p[0];
  if (b < 0x80) return {b, 1};
  int len;
  uint32_t cp;
  if ((b & 0xE0) == 0xC0) {
    len = 2;
    cp = b & 0x1F;
  } else if ((b & 0xF0) == 0xE0) {
    len = 3;
    cp = b & 0x0F;
  } else if ((b & 0xF8) == 0xF0) {
    len = 4;
    cp = b & 0x07;
  } else {
    return {0xFFFD, 1};
  }
  if (n < static_cast<size_t>(len)) return {0xFFFD, 1};
  for (int i = 1; i < len; ++i) {
    if ((p[i] & 0xC0) != 0x80) return {0xFFFD, 1};
    cp = (cp << 6) | (p[i] & 0x3F);
  }
  static const uint32_t kMin[5] = {0, 0, 0x80, 0x800, 0x10000};
  if (cp < kMin[len] || (cp >= 0xD800 && cp <= 0xDFFF)) return {0xFFFD, 1};
  return {cp, len};
}

inline void AppendUtf8(uint32_t cp, std::string* out) {
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

// GPT-2's bytes_to_unicode: the printable Latin-1 bytes ('!'..'~',
// U+00A1..U+00AC, U+00AE..U+00FF) stand for themselves; the other 68 bytes
// (0x00..0x20, 0x7F..0xA0, 0xAD), in byte order, take U+0100..U+0143.
inline bool ByteIsPrintable(uint32_t b) { return (b >= 0x21 && b <= 0x7E) || (b >= 0xA1 && b <= 0xAC) || b >= 0xAE; }

inline uint32_t ByteToCp(uint8_t b) {
  if (ByteIsPrintable(b)) return b;
  if (b <= 0x20) return 0x100 + b;
  if (b < 0xAD) return 0x100 + 0x21 + (b - 0x7F);
  return 0x143;  // 0xAD
}

// The byte a code point of the map stands for, or -1.
inline int CpToByte(uint32_t cp) {
  if (cp < 0x100) return ByteIsPrintable(cp) ? static_cast<int>(cp) : -1;
  if (cp > 0x143) return -1;
  const uint32_t k = cp - 0x100;
  if (k <= 0x20) return static_cast<int>(k);
  if (k < 0x43) return static_cast<int>(0x7F + (k - 0x21));
  return 0xAD;
}

}  // namespace uni
}  // namespace rpg

#endif  // RPG_HIP_UNICODE_H_
