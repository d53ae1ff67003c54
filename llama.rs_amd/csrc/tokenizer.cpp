// tokenizer.cpp — byte-level BPE tokenizer (GPT-2 / Qwen2 flavour) built from
// GGUF vocabulary data, and the Qwen3 chat templates (host C++, part of
// librlh). Restates src/tokenizer.rs:
//   bytes_to_unicode (7-32), Tokenizer::new (56-112), pretokenize (142-246,
//   the Qwen2 pattern written out by hand), match_contraction (248-268),
//   bpe (270-297: repeatedly merge the lowest-rank adjacent pair, leftmost
//   first), encode with verbatim special tokens (299-327), decode and
//   token_bytes (124-140, 336-359, lossy UTF-8), format_qwen_chat /
//   format_qwen_multiturn (386-430); Model::read_tokenizer (model.rs:295-330).
// Character classes are Rust's char::is_alphabetic / is_numeric /
// is_whitespace (tokenizer.rs:45-53) from generated Unicode tables.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/rlh.h"
#include "sampler.h"
#include "unicode_tables.h"
#include "utf8.h"

namespace {

using rlh::set_error;

template <size_t N>
bool in_table(const uint32_t (&t)[N][2], uint32_t cp) {
  size_t lo = 0, hi = N;
  while (lo < hi) {
    const size_t mid = (lo + hi) / 2;
    if (cp < t[mid][0]) hi = mid;
    else if (cp > t[mid][1]) lo = mid + 1;
    else return true;
  }
  return false;
}
bool is_letter(uint32_t c) { return in_table(kAlphabetic, c); }
bool is_number(uint32_t c) { return in_table(kNumeric, c); }
bool is_space(uint32_t c) { return in_table(kWhiteSpace, c); }

// bytes_to_unicode (tokenizer.rs:7-32): byte -> code point of its character.
void bytes_to_unicode(uint32_t table[256]) {
  bool direct[256] = {};
  for (uint32_t b = 0x21; b <= 0x7e; b++) direct[b] = true;
  for (uint32_t b = 0xa1; b <= 0xac; b++) direct[b] = true;
  for (uint32_t b = 0xae; b <= 0xff; b++) direct[b] = true;
  uint32_t n = 0;
  for (uint32_t b = 0; b < 256; b++) table[b] = direct[b] ? b : 256 + n++;
}

struct PairHash {
  size_t operator()(uint64_t k) const { return std::hash<uint64_t>()(k); }
};

}  // namespace

struct rlh_tokenizer {
  std::vector<std::string> id_to_token;
  std::unordered_map<uint64_t, std::pair<uint32_t, uint32_t>, PairHash> merges;  // (l, r) -> (rank, merged)
  uint32_t byte_to_id[256] = {};
  std::unordered_map<uint32_t, uint8_t> char_to_byte;
  std::vector<std::pair<std::string, uint32_t>> specials;  // longest first
  uint32_t bos = 1, eos = 2;

  // pretokenize (tokenizer.rs:142-246): byte ranges of the pieces.
  void pretokenize(const std::string& text, std::vector<std::pair<size_t, size_t>>* pieces) const {
    std::vector<std::pair<size_t, uint32_t>> ch;
    rlh::utf8_chars((const uint8_t*)text.data(), text.size(), &ch);
    const size_t n = ch.size();
    pieces->clear();
    size_t i = 0;
    auto C = [&](size_t k) { return ch[k].second; };
    while (i < n) {
      const uint32_t c = C(i);
      size_t end = 0;
      if (c == '\'') end = match_contraction(ch, i);  // alt1: 's 't 'm 'd 're 've 'll (any case)
      if (end == 0) {  // alt2: [^\r\n\p{L}\p{N}]?\p{L}+
        if (is_letter(c)) {
          size_t j = i + 1;
          while (j < n && is_letter(C(j))) j++;
          end = j;
        } else if (c != '\r' && c != '\n' && !is_number(c) && i + 1 < n && is_letter(C(i + 1))) {
          size_t j = i + 1;
          while (j < n && is_letter(C(j))) j++;
          end = j;
        }
      }
      if (end == 0 && is_number(c)) end = i + 1;  // alt3: \p{N}
      if (end == 0) {  // alt4: ' ?[^\s\p{L}\p{N}]+[\r\n]*', before the whitespace alternatives
        size_t j = i;
        if (C(j) == ' ' && i + 1 < n) j++;
        const size_t mid = j;
        while (j < n && !is_space(C(j)) && !is_letter(C(j)) && !is_number(C(j))) j++;
        if (j > mid) {
          while (j < n && (C(j) == '\r' || C(j) == '\n')) j++;
          end = j;
        }
      }
      if (end == 0 && is_space(c)) {  // alt5: \s*[\r\n]+
        size_t j = i;
        while (j < n && is_space(C(j)) && C(j) != '\r' && C(j) != '\n') j++;
        size_t k = j;
        while (k < n && (C(k) == '\r' || C(k) == '\n')) k++;
        if (k > j) {
          end = k;
        } else {  // alt6: \s+(?!\S), alt7: \s+
          size_t run = i;
          while (run < n && is_space(C(run))) run++;
          const size_t len = run - i;
          if (run == n) end = run;
          else if (len >= 2) end = run - 1;  // the last space starts the next piece
          else end = run;
        }
      }
      if (end <= i) end = i + 1;
      const size_t b0 = ch[i].first, b1 = end >= n ? text.size() : ch[end].first;
      pieces->emplace_back(b0, b1);
      i = end;
    }
  }

  static size_t match_contraction(const std::vector<std::pair<size_t, uint32_t>>& ch, size_t i) {
    const size_t n = ch.size();
    if (i + 1 >= n) return 0;
    const uint32_t c1 = ch[i + 1].second;
    switch (c1) {
      case 's': case 'S': case 't': case 'T': case 'm': case 'M': case 'd': case 'D': return i + 2;
      case 'r': case 'R': case 'v': case 'V': case 'l': case 'L':
        if (i + 2 < n) {
          const uint32_t c2 = ch[i + 2].second;
          if (c2 == 'e' || c2 == 'E' || c2 == 'l' || c2 == 'L') return i + 3;
        }
        return 0;
      default: return 0;
    }
  }

  // bpe (tokenizer.rs:270-297)
  void bpe(const uint8_t* bytes, size_t len, std::vector<uint32_t>* out) const {
    std::vector<uint32_t> syms(len);
    for (size_t k = 0; k < len; k++) syms[k] = byte_to_id[bytes[k]];
    while (syms.size() >= 2) {
      bool found = false;
      size_t bi = 0;
      uint32_t br = 0, bm = 0;
      for (size_t k = 0; k + 1 < syms.size(); k++) {
        auto it = merges.find(((uint64_t)syms[k] << 32) | syms[k + 1]);
        if (it != merges.end() && (!found || it->second.first < br)) {
          found = true;
          bi = k;
          br = it->second.first;
          bm = it->second.second;
        }
      }
      if (!found) break;
      syms[bi] = bm;
      syms.erase(syms.begin() + (ptrdiff_t)bi + 1);
    }
    out->insert(out->end(), syms.begin(), syms.end());
  }

  void encode_normal(const std::string& text, std::vector<uint32_t>* ids) const {
    std::vector<std::pair<size_t, size_t>> pieces;
    pretokenize(text, &pieces);
    for (auto& p : pieces) bpe((const uint8_t*)text.data() + p.first, p.second - p.first, ids);
  }

  // encode (tokenizer.rs:299-327): the earliest special token occurrence
  // (the longest one first at equal starts) splits the text.
  void encode(const std::string& text, std::vector<uint32_t>* ids) const {
    size_t pos = 0;
    while (pos < text.size()) {
      bool found = false;
      size_t fs = 0, fe = 0;
      uint32_t fid = 0;
      for (auto& sp : specials) {
        if (sp.first.empty()) continue;  // an empty special would match everywhere
        const size_t rel = text.find(sp.first, pos);
        if (rel != std::string::npos && (!found || rel < fs)) {
          found = true;
          fs = rel;
          fe = rel + sp.first.size();
          fid = sp.second;
        }
      }
      if (!found) {
        encode_normal(text.substr(pos), ids);
        break;
      }
      if (fs > pos) encode_normal(text.substr(pos, fs - pos), ids);
      ids->push_back(fid);
      pos = fe;
    }
  }

  void token_bytes(uint32_t id, std::string* out) const {
    if (id >= id_to_token.size()) return;
    const std::string& s = id_to_token[id];
    std::vector<std::pair<size_t, uint32_t>> ch;
    rlh::utf8_chars((const uint8_t*)s.data(), s.size(), &ch);  // vocab strings are valid UTF-8
    for (size_t k = 0; k < ch.size(); k++) {
      auto it = char_to_byte.find(ch[k].second);
      if (it != char_to_byte.end()) {
        *out += (char)it->second;
      } else {
        const size_t b1 = k + 1 < ch.size() ? ch[k + 1].first : s.size();
        out->append(s, ch[k].first, b1 - ch[k].first);
      }
    }
  }
};

namespace {

int copy_out(const std::string& s, char* out, uint64_t cap, uint64_t* len) {
  if (len) *len = s.size();
  if (out && cap) {
    const size_t k = std::min<size_t>(s.size(), (size_t)cap);
    std::memcpy(out, s.data(), k);
    if (k < cap) out[k] = 0;
  }
  if (s.size() > cap) return set_error(RLH_EINVAL, "output buffer too small (*len holds the size needed)");
  return RLH_OK;
}

bool valid_utf8(const char* s, uint64_t n) {
  std::vector<std::pair<size_t, uint32_t>> ch;
  return rlh::utf8_chars((const uint8_t*)s, (size_t)n, &ch);
}

}  // namespace

extern "C" {

int rlh_tokenizer_create(const char* const* tokens, uint64_t n_tokens, const uint32_t* token_types, uint64_t n_types,
                         const char* const* merges, uint64_t n_merges, uint32_t bos_id, uint32_t eos_id,
                         rlh_tokenizer** out) {
  if (!out || (n_tokens && !tokens) || (n_types && !token_types) || (n_merges && !merges))
    return set_error(RLH_EINVAL, "null argument");
  *out = nullptr;
  rlh_tokenizer* t = new rlh_tokenizer();
  t->bos = bos_id;
  t->eos = eos_id;
  std::unordered_map<std::string, uint32_t> to_id;
  to_id.reserve((size_t)n_tokens);
  for (uint64_t i = 0; i < n_tokens; i++) {
    if (!tokens[i]) {
      delete t;
      return set_error(RLH_EINVAL, "null token string");
    }
    t->id_to_token.emplace_back(rlh::utf8_lossy((const uint8_t*)tokens[i], std::strlen(tokens[i])));
    to_id.emplace(t->id_to_token.back(), (uint32_t)i);  // the first occurrence keeps its id
  }
  uint32_t b2u[256];
  bytes_to_unicode(b2u);
  for (uint32_t b = 0; b < 256; b++) {
    t->char_to_byte[b2u[b]] = (uint8_t)b;
    std::string s;
    rlh::utf8_put(s, b2u[b]);
    auto it = to_id.find(s);
    if (it != to_id.end()) t->byte_to_id[b] = it->second;
  }
  for (uint64_t r = 0; r < n_merges; r++) {
    if (!merges[r]) continue;
    const std::string m = rlh::utf8_lossy((const uint8_t*)merges[r], std::strlen(merges[r]));
    const size_t sp = m.find(' ');  // split_once(' ')
    if (sp == std::string::npos) continue;
    const std::string l = m.substr(0, sp), rr = m.substr(sp + 1);
    auto li = to_id.find(l), ri = to_id.find(rr), mi = to_id.find(l + rr);
    if (li == to_id.end() || ri == to_id.end() || mi == to_id.end()) continue;
    t->merges[((uint64_t)li->second << 32) | ri->second] = {(uint32_t)r, mi->second};  // a later rank replaces
  }
  for (uint64_t i = 0; i < n_tokens; i++) {
    const uint32_t ty = i < n_types ? token_types[i] : 1u;
    if (ty == 3 || ty == 4) t->specials.emplace_back(t->id_to_token[i], (uint32_t)i);
  }
  std::stable_sort(t->specials.begin(), t->specials.end(),
                   [](const auto& a, const auto& b) { return a.first.size() > b.first.size(); });
  *out = t;
  return RLH_OK;
}

int rlh_tokenizer_from_gguf(const rlh_gguf* g, rlh_tokenizer** out) {
  if (!g || !out) return set_error(RLH_EINVAL, "null argument");
  *out = nullptr;
  const char* kTok = "tokenizer.ggml.tokens";
  uint32_t ty = 0, et = 0;
  uint64_t n = 0;
  if (rlh_gguf_meta_type(g, kTok, &ty, &et, &n) || ty != 9 || et != 8)
    return set_error(RLH_EFORMAT, "missing metadata key: tokenizer.ggml.tokens");
  std::vector<const char*> toks(n);
  for (uint64_t i = 0; i < n; i++)
    if (rlh_gguf_meta_arr_str(g, kTok, i, &toks[i], nullptr)) return set_error(RLH_EFORMAT, "bad token string");
  // token types: each element's as_u32, 1 when absent (model.rs:302-307)
  std::vector<uint32_t> types;
  uint64_t nt = 0;
  if (!rlh_gguf_meta_type(g, "tokenizer.ggml.token_type", &ty, &et, &nt) && ty == 9) {
    types.assign(nt, 1u);
    for (uint64_t i = 0; i < nt; i++) {
      uint64_t u = 0;
      int64_t s = 0;
      if (!rlh_gguf_meta_arr_scalar(g, "tokenizer.ggml.token_type", i, &u, &s, nullptr)) {
        const bool sig = et == 1 || et == 3 || et == 5 || et == 11;
        if (et <= 5 || et == 10 || et == 11) types[i] = sig ? (uint32_t)(uint64_t)s : (uint32_t)u;
      }
    }
  } else {
    types.assign(n, 1u);
  }
  // merges: a string array, else none (model.rs:309-312)
  std::vector<const char*> mg;
  uint64_t nm = 0;
  if (!rlh_gguf_meta_type(g, "tokenizer.ggml.merges", &ty, &et, &nm) && ty == 9 && et == 8) {
    mg.resize(nm);
    for (uint64_t i = 0; i < nm; i++)
      if (rlh_gguf_meta_arr_str(g, "tokenizer.ggml.merges", i, &mg[i], nullptr)) mg.clear();
  }
  uint32_t bos = 1, eos = 2;  // model.rs:320-325
  if (rlh_gguf_meta_u32(g, "tokenizer.ggml.bos_token_id", &bos)) bos = 1;
  if (rlh_gguf_meta_u32(g, "tokenizer.ggml.eos_token_id", &eos)) eos = 2;
  return rlh_tokenizer_create(toks.data(), n, types.data(), types.size(), mg.data(), mg.size(), bos, eos, out);
}

void rlh_tokenizer_destroy(rlh_tokenizer* t) { delete t; }
uint64_t rlh_tokenizer_vocab_size(const rlh_tokenizer* t) { return t ? t->id_to_token.size() : 0; }
uint32_t rlh_tokenizer_bos(const rlh_tokenizer* t) { return t ? t->bos : 0; }
uint32_t rlh_tokenizer_eos(const rlh_tokenizer* t) { return t ? t->eos : 0; }

int rlh_tokenizer_encode(const rlh_tokenizer* t, const char* text, uint64_t len, uint32_t* ids, uint64_t cap,
                         uint64_t* n_ids) {
  if (!t || (!text && len) || !n_ids || (!ids && cap)) return set_error(RLH_EINVAL, "null argument");
  if (!valid_utf8(text, len)) return set_error(RLH_EINVAL, "text is not valid UTF-8");
  std::vector<uint32_t> v;
  t->encode(std::string(text ? text : "", (size_t)len), &v);
  *n_ids = v.size();
  if (ids) std::memcpy(ids, v.data(), std::min<size_t>(v.size(), (size_t)cap) * 4);
  if (v.size() > cap) return set_error(RLH_EINVAL, "ids buffer too small (*n_ids holds the count needed)");
  return RLH_OK;
}

int rlh_tokenizer_pretokenize(const rlh_tokenizer* t, const char* text, uint64_t len, uint64_t* bounds, uint64_t cap,
                              uint64_t* n_pieces) {
  if (!t || (!text && len) || !n_pieces || (!bounds && cap)) return set_error(RLH_EINVAL, "null argument");
  if (!valid_utf8(text, len)) return set_error(RLH_EINVAL, "text is not valid UTF-8");
  std::vector<std::pair<size_t, size_t>> p;
  t->pretokenize(std::string(text ? text : "", (size_t)len), &p);
  *n_pieces = p.size();
  for (size_t k = 0; k < p.size() && 2 * k + 1 < cap; k++) {
    bounds[2 * k] = p[k].first;
    bounds[2 * k + 1] = p[k].second;
  }
  if (2 * p.size() > cap) return set_error(RLH_EINVAL, "bounds buffer too small (2 entries per piece)");
  return RLH_OK;
}

int rlh_tokenizer_decode(const rlh_tokenizer* t, const uint32_t* ids, uint64_t n, char* out, uint64_t cap,
                         uint64_t* len) {
  if (!t || (!ids && n) || !len) return set_error(RLH_EINVAL, "null argument");
  std::string bytes;
  for (uint64_t k = 0; k < n; k++) t->token_bytes(ids[k], &bytes);  // unknown ids are skipped
  return copy_out(rlh::utf8_lossy((const uint8_t*)bytes.data(), bytes.size()), out, cap, len);
}

int rlh_tokenizer_token_bytes(const rlh_tokenizer* t, uint32_t id, char* out, uint64_t cap, uint64_t* len) {
  if (!t || !len) return set_error(RLH_EINVAL, "null argument");
  std::string bytes;
  t->token_bytes(id, &bytes);
  return copy_out(bytes, out, cap, len);
}

// format_qwen_chat / format_qwen_multiturn (tokenizer.rs:386-430)
int rlh_format_qwen_chat(const char* const* roles, const char* const* contents, uint64_t n_turns, const char* prompt,
                         const char* system, int no_think, char* out, uint64_t cap, uint64_t* len) {
  if (!prompt || !len || (n_turns && (!roles || !contents))) return set_error(RLH_EINVAL, "null argument");
  std::string s;
  if (system) {
    s += "<|im_start|>system\n";
    s += system;
    s += "<|im_end|>\n";
  }
  for (uint64_t k = 0; k < n_turns; k++) {
    if (!roles[k] || !contents[k]) return set_error(RLH_EINVAL, "null turn");
    s += "<|im_start|>";
    s += roles[k];
    s += "\n";
    s += contents[k];
    s += "<|im_end|>\n";
  }
  s += "<|im_start|>user\n";
  s += prompt;
  s += "<|im_end|>\n<|im_start|>assistant\n";
  if (no_think) s += "<think>\n\n</think>\n\n";
  return copy_out(s, out, cap, len);
}

}  // extern "C"
