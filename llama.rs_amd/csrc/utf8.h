// utf8.h — UTF-8 decoding as Rust's str / String::from_utf8_lossy define it
// (host code shared by the GGUF reader and the tokenizer).
#pragma once
#include <cstdint>
#include <string>
#include <vector>

namespace rlh {

// Length of the valid UTF-8 sequence starting at s[i] (1-4), or 0 when the
// bytes at i do not start one. *bad receives the length of the maximal
// prefix that could still have started a valid sequence (at least 1): the
// bytes one U+FFFD replaces (the Unicode "maximal subpart" rule that
// from_utf8_lossy follows).
inline int utf8_seq(const uint8_t* s, size_t n, size_t i, int* bad) {
  const uint8_t b = s[i];
  *bad = 1;
  if (b < 0x80) return 1;
  int need;
  uint8_t lo = 0x80, hi = 0xBF;
  if (b >= 0xC2 && b <= 0xDF) {
    need = 1;
  } else if (b >= 0xE0 && b <= 0xEF) {
    need = 2;
    if (b == 0xE0) lo = 0xA0;
    if (b == 0xED) hi = 0x9F;
  } else if (b >= 0xF0 && b <= 0xF4) {
    need = 3;
    if (b == 0xF0) lo = 0x90;
    if (b == 0xF4) hi = 0x8F;
  } else {
    return 0;
  }
  for (int k = 1; k <= need; k++) {
    if (i + k >= n) return 0;
    const uint8_t c = s[i + k];
    const uint8_t l = k == 1 ? lo : 0x80, h = k == 1 ? hi : 0xBF;
    if (c < l || c > h) return 0;
    *bad = k + 1;
  }
  return need + 1;
}

inline uint32_t utf8_cp(const uint8_t* s, int len) {
  if (len == 1) return s[0];
  if (len == 2) return ((s[0] & 0x1Fu) << 6) | (s[1] & 0x3Fu);
  if (len == 3) return ((s[0] & 0x0Fu) << 12) | ((s[1] & 0x3Fu) << 6) | (s[2] & 0x3Fu);
  return ((s[0] & 0x07u) << 18) | ((s[1] & 0x3Fu) << 12) | ((s[2] & 0x3Fu) << 6) | (s[3] & 0x3Fu);
}

inline void utf8_put(std::string& out, uint32_t cp) {
  if (cp < 0x80) {
    out += (char)cp;
  } else if (cp < 0x800) {
    out += (char)(0xC0 | (cp >> 6));
    out += (char)(0x80 | (cp & 0x3F));
  } else if (cp < 0x10000) {
    out += (char)(0xE0 | (cp >> 12));
    out += (char)(0x80 | ((cp >> 6) & 0x3F));
    out += (char)(0x80 | (cp & 0x3F));
  } else {
    out += (char)(0xF0 | (cp >> 18));
    out += (char)(0x80 | ((cp >> 12) & 0x3F));
    out += (char)(0x80 | ((cp >> 6) & 0x3F));
    out += (char)(0x80 | (cp & 0x3F));
  }
}

// String::from_utf8_lossy: valid sequences copied, each maximal invalid
// subpart replaced by U+FFFD.
inline std::string utf8_lossy(const uint8_t* s, size_t n) {
  std::string out;
  out.reserve(n);
  size_t i = 0;
  while (i < n) {
    int bad;
    const int len = utf8_seq(s, n, i, &bad);
    if (len) {
      out.append((const char*)s + i, (size_t)len);
      i += (size_t)len;
    } else {
      out += "\xEF\xBF\xBD";
      i += (size_t)bad;
    }
  }
  return out;
}

// Decodes valid UTF-8 into (byte offset, code point) pairs; false on
// invalid input (a Rust &str is always valid).
inline bool utf8_chars(const uint8_t* s, size_t n, std::vector<std::pair<size_t, uint32_t>>* out) {
  out->clear();
  size_t i = 0;
  while (i < n) {
    int bad;
    const int len = utf8_seq(s, n, i, &bad);
    if (!len) return false;
    out->emplace_back(i, utf8_cp(s + i, len));
    i += (size_t)len;
  }
  return true;
}

}  // namespace rlh
