// Byte-level BPE tokenizer of the Qwen2.5 family and the chat template: the
// text side of the decode path (the reference's QwenTokenizer,
// include/tokenizer.h:18-41, src/tokenizer.cpp), with no PCRE2 or JSON
// library (neither is part of this image):
//   * the ranks file is the exporter's qwen25_bpe_ranks.json
//     (export_weights.py:328-365): {"vocab": {token: id}, "added_tokens":
//     {"id": token}, ...}, read by a small JSON reader below;
//   * the Qwen2 pre-tokenizer pattern (src/tokenizer.cpp:86, compiled there
//     with PCRE2_UTF | PCRE2_UCP) runs as a hand-written scanner over code
//     points, its seven alternatives tried in order with the backtracking
//     PCRE2 would do; the Unicode classes come from cq_unicode_tables.inc;
//   * byte-level BPE as in src/tokenizer.cpp:107-143: the bytes of a chunk
//     map to the GPT-2 byte alphabet, then the adjacent pair whose
//     concatenation has the lowest vocabulary id merges (its first
//     occurrence), until no pair is in the vocabulary;
//   * special tokens split the text first, the earliest occurrence winning
//     and the longest token at equal positions (src/tokenizer.cpp:170-201).
// Deliberate differences: bytes that are not valid UTF-8 are kept as
// single-byte "other" characters (PCRE2 would stop matching there and the
// reference drops the rest of the text); the class tables are Unicode 13.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <fstream>
#include <limits>
#include <memory>
#include <sstream>
#include <string>
#include <unordered_map>
#include <vector>

#include "cq_common.h"

struct cq_tokenizer {
  std::unordered_map<std::string, int32_t> encoder;   // byte-alphabet token -> id
  std::unordered_map<int32_t, std::string> decoder;
  std::vector<std::pair<std::string, int32_t>> specials;   // longest first
  std::string byte_token[256];                              // byte -> its one-character token
  std::unordered_map<uint32_t, uint8_t> byte_of_cp;         // alphabet code point -> byte
};

namespace cq {
namespace {

struct CodeRange {
  uint32_t lo, hi;
};
#include "cq_unicode_tables.inc"

template <size_t N>
bool in_ranges(const CodeRange (&r)[N], uint32_t cp) {
  size_t lo = 0, hi = N;
  while (lo < hi) {
    const size_t mid = (lo + hi) / 2;
    if (cp < r[mid].lo) hi = mid;
    else if (cp > r[mid].hi) lo = mid + 1;
    else return true;
  }
  return false;
}

void put_utf8(uint32_t cp, std::string& out) {
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

// One decoded character: code point (kInvalid for a byte that does not
// start a valid UTF-8 sequence) and its byte offset.
constexpr uint32_t kInvalid = 0xFFFFFFFFu;
struct Char {
  uint32_t cp;
  size_t off;
};

std::vector<Char> decode_utf8(const char* s, size_t n) {
  std::vector<Char> out;
  out.reserve(n);
  size_t i = 0;
  while (i < n) {
    const uint8_t b = (uint8_t)s[i];
    int len = 0;
    uint32_t cp = 0, min = 0;
    if (b < 0x80) { len = 1; cp = b; }
    else if ((b & 0xE0) == 0xC0) { len = 2; cp = b & 0x1F; min = 0x80; }
    else if ((b & 0xF0) == 0xE0) { len = 3; cp = b & 0x0F; min = 0x800; }
    else if ((b & 0xF8) == 0xF0) { len = 4; cp = b & 0x07; min = 0x10000; }
    bool ok = len > 0 && i + len <= n;
    for (int k = 1; ok && k < len; ++k) {
      const uint8_t c = (uint8_t)s[i + k];
      if ((c & 0xC0) != 0x80) ok = false;
      else cp = (cp << 6) | (c & 0x3F);
    }
    if (ok && len > 1 && (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF))) ok = false;
    if (!ok) {
      out.push_back({kInvalid, i});
      i += 1;
    } else {
      out.push_back({cp, i});
      i += len;
    }
  }
  return out;
}

// ------------------------------------------------------- pre-tokenizer
// (?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}|
//  ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+
struct Scanner {
  const std::vector<Char>& c;
  size_t n;
  explicit Scanner(const std::vector<Char>& chars) : c(chars), n(chars.size()) {}
  bool letter(size_t i) const { return i < n && c[i].cp != kInvalid && in_ranges(kLetterRanges, c[i].cp); }
  bool number(size_t i) const { return i < n && c[i].cp != kInvalid && in_ranges(kNumberRanges, c[i].cp); }
  bool space(size_t i) const { return i < n && c[i].cp != kInvalid && in_ranges(kSpaceRanges, c[i].cp); }
  bool crlf(size_t i) const { return i < n && (c[i].cp == '\r' || c[i].cp == '\n'); }
  bool is(size_t i, char lower) const {
    if (i >= n) return false;
    const uint32_t cp = c[i].cp;
    if (cp == (uint32_t)lower || cp == (uint32_t)(lower - 32)) return true;
    return lower == 's' && cp == 0x17F;   // caseless UTF matching folds LONG S to s
  }

  // end (exclusive) of the token starting at i
  size_t next(size_t i) const {
    // 1. contractions, case-insensitive
    if (c[i].cp == '\'') {
      if (is(i + 1, 's') || is(i + 1, 't') || is(i + 1, 'm') || is(i + 1, 'd')) return i + 2;
      if ((is(i + 1, 'r') && is(i + 2, 'e')) || (is(i + 1, 'v') && is(i + 2, 'e')) ||
          (is(i + 1, 'l') && is(i + 2, 'l')))
        return i + 3;
    }
    // 2. an optional non-letter, non-number, non-CR/LF character, then letters
    {
      size_t j = i;
      if (!crlf(i) && !letter(i) && !number(i) && letter(i + 1)) j = i + 1;
      if (letter(j)) {
        while (letter(j)) ++j;
        return j;
      }
    }
    // 3. one number
    if (number(i)) return i + 1;
    // 4. an optional space, symbols, then CR/LF
    {
      size_t j = i + (c[i].cp == ' ' ? 1 : 0);
      size_t k = j;
      while (k < n && !space(k) && !letter(k) && !number(k)) ++k;
      if (k > j) {
        while (crlf(k)) ++k;
        return k;
      }
    }
    if (space(i)) {
      size_t e = i;
      while (space(e)) ++e;
      // 5. whitespace up to and including its last CR/LF
      for (size_t q = e; q > i; --q)
        if (crlf(q - 1)) return q;
      // 6. whitespace not followed by a non-space: all of it at the end of
      // the text, else all but its last character
      if (e == n) return e;
      if (e - 1 > i) return e - 1;
      // 7. the single whitespace character
      return e;
    }
    return i + 1;   // unreachable for valid classes; keeps the scan moving
  }
};

// -------------------------------------------------------------- JSON
// Just enough JSON for the ranks file: objects, strings (all escapes,
// surrogate pairs), integers; anything else is skipped.
struct Json {
  const std::string& s;
  size_t p = 0;
  std::string err;
  explicit Json(const std::string& text) : s(text) {}
  void ws() {
    while (p < s.size() && (s[p] == ' ' || s[p] == '\n' || s[p] == '\r' || s[p] == '\t')) ++p;
  }
  bool fail(const std::string& m) {
    if (err.empty()) err = m + " at byte " + std::to_string(p);
    return false;
  }
  bool expect(char ch) {
    ws();
    if (p >= s.size() || s[p] != ch) return fail(std::string("expected '") + ch + "'");
    ++p;
    return true;
  }
  bool hex4(uint32_t* v) {
    if (p + 4 > s.size()) return fail("short \\u escape");
    uint32_t x = 0;
    for (int k = 0; k < 4; ++k) {
      const char h = s[p++];
      x <<= 4;
      if (h >= '0' && h <= '9') x |= h - '0';
      else if (h >= 'a' && h <= 'f') x |= h - 'a' + 10;
      else if (h >= 'A' && h <= 'F') x |= h - 'A' + 10;
      else return fail("bad \\u escape");
    }
    *v = x;
    return true;
  }
  bool str(std::string* out) {
    ws();
    if (p >= s.size() || s[p] != '"') return fail("expected a string");
    ++p;
    out->clear();
    while (p < s.size() && s[p] != '"') {
      const char ch = s[p++];
      if (ch != '\\') {
        *out += ch;
        continue;
      }
      if (p >= s.size()) return fail("bad escape");
      const char e = s[p++];
      switch (e) {
        case '"': *out += '"'; break;
        case '\\': *out += '\\'; break;
        case '/': *out += '/'; break;
        case 'b': *out += '\b'; break;
        case 'f': *out += '\f'; break;
        case 'n': *out += '\n'; break;
        case 'r': *out += '\r'; break;
        case 't': *out += '\t'; break;
        case 'u': {
          uint32_t cp;
          if (!hex4(&cp)) return false;
          if (cp >= 0xD800 && cp <= 0xDBFF && p + 6 <= s.size() && s[p] == '\\' && s[p + 1] == 'u') {
            p += 2;
            uint32_t lo;
            if (!hex4(&lo)) return false;
            if (lo >= 0xDC00 && lo <= 0xDFFF) cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
            else return fail("unpaired surrogate");
          } else if (cp >= 0xD800 && cp <= 0xDFFF) {
            return fail("unpaired surrogate");   // a lone half of a pair is not text (RFC 8259 section 8.2)
          }
          put_utf8(cp, *out);
          break;
        }
        default: return fail("bad escape");
      }
    }
    if (p >= s.size()) return fail("unterminated string");
    ++p;
    return true;
  }
  bool integer(long long* v) {
    ws();
    size_t q = p;
    if (q < s.size() && s[q] == '-') ++q;
    if (q >= s.size() || s[q] < '0' || s[q] > '9') return fail("expected an integer");
    while (q < s.size() && s[q] >= '0' && s[q] <= '9') ++q;
    *v = std::stoll(s.substr(p, q - p));
    p = q;
    return true;
  }
  bool skip() {   // any value
    ws();
    if (p >= s.size()) return fail("unexpected end");
    const char ch = s[p];
    if (ch == '"') {
      std::string t;
      return str(&t);
    }
    if (ch == '{' || ch == '[') {
      const char close = ch == '{' ? '}' : ']';
      ++p;
      ws();
      if (p < s.size() && s[p] == close) {
        ++p;
        return true;
      }
      while (true) {
        if (ch == '{') {
          std::string k;
          if (!str(&k) || !expect(':')) return false;
        }
        if (!skip()) return false;
        ws();
        if (p < s.size() && s[p] == ',') {
          ++p;
          continue;
        }
        return expect(close);
      }
    }
    while (p < s.size() && s[p] != ',' && s[p] != '}' && s[p] != ']' && s[p] != ' ' && s[p] != '\n' &&
           s[p] != '\r' && s[p] != '\t')
      ++p;
    return true;
  }
  // object: calls member(key) with the position at the value; member must consume it
  template <typename F>
  bool object(F member) {
    if (!expect('{')) return false;
    ws();
    if (p < s.size() && s[p] == '}') {
      ++p;
      return true;
    }
    while (true) {
      std::string k;
      if (!str(&k) || !expect(':')) return false;
      if (!member(k)) return false;
      ws();
      if (p < s.size() && s[p] == ',') {
        ++p;
        continue;
      }
      return expect('}');
    }
  }
};

// GPT-2 byte alphabet: printable bytes map to themselves, the rest to 256+n
// in byte order (src/tokenizer.cpp:10-41).
void build_byte_alphabet(cq_tokenizer& t) {
  int n = 0;
  for (int b = 0; b < 256; ++b) {
    const bool printable = (b >= '!' && b <= '~') || (b >= 0xA1 && b <= 0xAC) || (b >= 0xAE && b <= 0xFF);
    const uint32_t cp = printable ? (uint32_t)b : (uint32_t)(256 + n++);
    std::string s;
    put_utf8(cp, s);
    t.byte_token[b] = s;
    t.byte_of_cp[cp] = (uint8_t)b;
  }
}

void bpe(const cq_tokenizer& t, const char* s, size_t n, std::vector<int32_t>& out) {
  std::vector<std::string> parts;
  parts.reserve(n);
  for (size_t i = 0; i < n; ++i) parts.push_back(t.byte_token[(uint8_t)s[i]]);
  while (parts.size() >= 2) {
    int32_t best = std::numeric_limits<int32_t>::max();
    size_t at = 0;
    for (size_t i = 0; i + 1 < parts.size(); ++i) {
      auto it = t.encoder.find(parts[i] + parts[i + 1]);
      if (it != t.encoder.end() && it->second < best) {
        best = it->second;
        at = i;
      }
    }
    if (best == std::numeric_limits<int32_t>::max()) break;
    parts[at] += parts[at + 1];
    parts.erase(parts.begin() + at + 1);
  }
  for (const std::string& p : parts) {
    auto it = t.encoder.find(p);
    out.push_back(it == t.encoder.end() ? 0 : it->second);   // every byte token is in a byte-level vocabulary
  }
}

void encode_plain(const cq_tokenizer& t, const char* s, size_t n, std::vector<int32_t>& out) {
  const std::vector<Char> chars = decode_utf8(s, n);
  const Scanner sc(chars);
  size_t i = 0;
  while (i < chars.size()) {
    const size_t e = sc.next(i);
    const size_t b0 = chars[i].off, b1 = e < chars.size() ? chars[e].off : n;
    bpe(t, s + b0, b1 - b0, out);
    i = e;
  }
}

void encode(const cq_tokenizer& t, const char* s, size_t n, std::vector<int32_t>& out) {
  const std::string text(s, n);
  size_t pos = 0;
  while (pos < n) {
    size_t best = std::string::npos;
    const std::pair<std::string, int32_t>* hit = nullptr;
    for (const auto& sp : t.specials) {   // longest first: strict < keeps the longest at a tie
      const size_t f = text.find(sp.first, pos);
      if (f != std::string::npos && f < best) {
        best = f;
        hit = &sp;
      }
    }
    if (!hit) {
      encode_plain(t, s + pos, n - pos, out);
      break;
    }
    if (best > pos) encode_plain(t, s + pos, best - pos, out);
    out.push_back(hit->second);
    pos = best + hit->first.size();
  }
}

// src/tokenizer.cpp:210-236: the decoder is the vocabulary only -- an id
// that is not in it (Qwen's added tokens such as <|im_end|> are not in
// vocab.json) decodes to nothing; a vocabulary entry whose text is one of
// the added tokens decodes to that text literally; any other entry maps its
// byte-alphabet characters back to bytes.
void decode_one(const cq_tokenizer& t, int32_t id, std::string& out) {
  auto it = t.decoder.find(id);
  if (it == t.decoder.end()) return;
  const std::string& tok = it->second;
  for (const auto& sp : t.specials)
    if (sp.first == tok) {
      out += tok;
      return;
    }
  for (const Char& ch : decode_utf8(tok.data(), tok.size())) {
    auto b = ch.cp == kInvalid ? t.byte_of_cp.end() : t.byte_of_cp.find(ch.cp);
    if (b != t.byte_of_cp.end()) {
      out += (char)b->second;
    } else if (ch.cp == kInvalid) {   // not in the byte alphabet: the token's own bytes
      out += tok[ch.off];
    } else {
      put_utf8(ch.cp, out);
    }
  }
}

}  // namespace
}  // namespace cq

using namespace cq;

extern "C" int cq_tokenizer_load(const char* ranks_json_path, cq_tokenizer** out) {
  if (!ranks_json_path || !out) return fail(CQ_EINVAL, "tokenizer_load: null argument");
  *out = nullptr;
  std::ifstream f(ranks_json_path, std::ios::binary);
  if (!f) return fail(CQ_EIO, std::string("tokenizer_load: cannot open ") + ranks_json_path);
  std::stringstream ss;
  ss << f.rdbuf();
  const std::string text = ss.str();
  std::unique_ptr<cq_tokenizer> t(new cq_tokenizer);
  Json js(text);
  bool have_vocab = false;
  const bool ok = js.object([&](const std::string& key) {
    if (key == "vocab") {
      have_vocab = true;
      return js.object([&](const std::string& tok) {
        long long id;
        if (!js.integer(&id)) return false;
        if (id < 0 || id > std::numeric_limits<int32_t>::max()) return js.fail("token id out of range");
        t->encoder[tok] = (int32_t)id;
        t->decoder[(int32_t)id] = tok;
        return true;
      });
    }
    if (key == "added_tokens") {
      return js.object([&](const std::string& id_text) {
        std::string tok;
        if (!js.str(&tok)) return false;
        char* end = nullptr;
        const long id = std::strtol(id_text.c_str(), &end, 10);
        if (id_text.empty() || *end || id < 0) return js.fail("bad added-token id '" + id_text + "'");
        t->specials.emplace_back(tok, (int32_t)id);
        return true;
      });
    }
    return js.skip();
  });
  if (!ok) return fail(CQ_EFORMAT, "tokenizer_load: " + js.err);
  if (!have_vocab || t->encoder.empty()) return fail(CQ_EFORMAT, "tokenizer_load: no \"vocab\" object");
  std::stable_sort(t->specials.begin(), t->specials.end(),
                   [](const auto& a, const auto& b) { return a.first.size() > b.first.size(); });
  build_byte_alphabet(*t);
  *out = t.release();
  return CQ_OK;
}

extern "C" int cq_tokenizer_free(cq_tokenizer* t) {
  delete t;
  return CQ_OK;
}

extern "C" int cq_tokenizer_encode(cq_tokenizer* t, const char* text, size_t len, int32_t* ids, int32_t cap,
                                   int32_t* n_out) {
  if (!t || (!text && len) || !n_out) return fail(CQ_EINVAL, "tokenizer_encode: null argument");
  std::vector<int32_t> v;
  encode(*t, text, len, v);
  *n_out = (int32_t)v.size();
  if ((int64_t)v.size() > cap) return fail(CQ_ERANGE, "tokenizer_encode: output holds " + std::to_string(cap) +
                                                         " ids, the text needs " + std::to_string(v.size()));
  if (!v.empty()) std::memcpy(ids, v.data(), v.size() * sizeof(int32_t));
  return CQ_OK;
}

extern "C" int cq_tokenizer_decode(cq_tokenizer* t, const int32_t* ids, int32_t n, char* buf, size_t cap,
                                   size_t* len_out) {
  if (!t || (!ids && n) || !len_out || n < 0) return fail(CQ_EINVAL, "tokenizer_decode: bad argument");
  std::string s;
  for (int32_t i = 0; i < n; ++i) decode_one(*t, ids[i], s);
  *len_out = s.size();
  if (s.size() > cap) return fail(CQ_ERANGE, "tokenizer_decode: buffer too small");
  if (!s.empty()) std::memcpy(buf, s.data(), s.size());
  return CQ_OK;
}

extern "C" int32_t cq_tokenizer_token_id(cq_tokenizer* t, const char* token) {
  if (!t || !token) return -1;
  auto it = t->encoder.find(token);
  if (it != t->encoder.end()) return it->second;
  for (const auto& sp : t->specials)
    if (sp.first == token) return sp.second;
  return -1;
}

extern "C" int32_t cq_tokenizer_vocab_size(cq_tokenizer* t) {
  if (!t) return -1;
  int32_t m = -1;
  for (const auto& kv : t->decoder) m = std::max(m, kv.first);
  for (const auto& sp : t->specials) m = std::max(m, sp.second);   // added tokens count too
  return m + 1;
}

extern "C" int cq_chat_template(const char* const* roles, const char* const* contents, int32_t n_messages,
                                int32_t add_generation_prompt, char* buf, size_t cap, size_t* len_out) {
  if ((n_messages && (!roles || !contents)) || !len_out || n_messages < 0)
    return fail(CQ_EINVAL, "chat_template: bad argument");
  std::string s;
  for (int32_t i = 0; i < n_messages; ++i) {
    if (!roles[i] || !contents[i]) return fail(CQ_EINVAL, "chat_template: null message");
    s += "<|im_start|>";
    s += roles[i];
    s += "\n";
    s += contents[i];
    s += "<|im_end|>\n";
  }
  if (add_generation_prompt) s += "<|im_start|>assistant\n";
  *len_out = s.size();
  if (s.size() > cap) return fail(CQ_ERANGE, "chat_template: buffer too small");
  if (!s.empty()) std::memcpy(buf, s.data(), s.size());
  return CQ_OK;
}
