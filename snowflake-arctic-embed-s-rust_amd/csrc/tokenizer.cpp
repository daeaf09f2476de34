// tokenizer.cpp -- BERT WordPiece tokenizer, behaviour of src/tokenizer.rs.
#include "tokenizer.hpp"

#include <algorithm>
#include <cstdio>
#include <thread>

#include "../../include/arctic_embed.h"

namespace ae {

namespace {

#include "unicode_lower.inc"

const char* kQueryPrefix = "Represent this sentence for searching relevant passages: ";  // src/tokenizer.rs:23

// lenient UTF-8 decoder: invalid sequences decode to U+FFFD (dropped by the normalizer)
std::u32string decode_utf8(const std::string& s) {
  std::u32string out;
  out.reserve(s.size());
  size_t i = 0;
  const size_t n = s.size();
  while (i < n) {
    const unsigned char c = (unsigned char)s[i];
    uint32_t cp;
    int len;
    if (c < 0x80) { cp = c; len = 1; }
    else if ((c >> 5) == 0x6) { cp = c & 0x1F; len = 2; }
    else if ((c >> 4) == 0xE) { cp = c & 0x0F; len = 3; }
    else if ((c >> 3) == 0x1E) { cp = c & 0x07; len = 4; }
    else { out.push_back(0xFFFD); i++; continue; }
    if (i + len > n) { out.push_back(0xFFFD); i++; continue; }
    bool ok = true;
    for (int k = 1; k < len; k++) {
      const unsigned char cc = (unsigned char)s[i + k];
      if ((cc >> 6) != 0x2) { ok = false; break; }
      cp = (cp << 6) | (cc & 0x3F);
    }
    if (!ok || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF) || (len == 2 && cp < 0x80) ||
        (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000)) {
      out.push_back(0xFFFD);
      i++;
      continue;
    }
    out.push_back(cp);
    i += len;
  }
  return out;
}

void append_utf8(std::string& out, uint32_t cp) {
  if (cp < 0x80) {
    out.push_back(char(cp));
  } else if (cp < 0x800) {
    out.push_back(char(0xC0 | (cp >> 6)));
    out.push_back(char(0x80 | (cp & 0x3F)));
  } else if (cp < 0x10000) {
    out.push_back(char(0xE0 | (cp >> 12)));
    out.push_back(char(0x80 | ((cp >> 6) & 0x3F)));
    out.push_back(char(0x80 | (cp & 0x3F)));
  } else {
    out.push_back(char(0xF0 | (cp >> 18)));
    out.push_back(char(0x80 | ((cp >> 12) & 0x3F)));
    out.push_back(char(0x80 | ((cp >> 6) & 0x3F)));
    out.push_back(char(0x80 | (cp & 0x3F)));
  }
}

// char::is_whitespace (Unicode White_Space)
bool is_unicode_whitespace(uint32_t c) {
  return (c >= 0x9 && c <= 0xD) || c == 0x20 || c == 0x85 || c == 0xA0 || c == 0x1680 || (c >= 0x2000 && c <= 0x200A) ||
         c == 0x2028 || c == 0x2029 || c == 0x202F || c == 0x205F || c == 0x3000;
}
bool is_bert_whitespace(uint32_t c) { return c == ' ' || c == '\t' || c == '\n' || c == '\r' || is_unicode_whitespace(c); }
// char::is_control (general category Cc) minus \t \n \r (src/tokenizer.rs:217-223)
bool is_bert_control(uint32_t c) {
  if (c == '\t' || c == '\n' || c == '\r') return false;
  return c <= 0x1F || (c >= 0x7F && c <= 0x9F);
}
bool is_chinese_char(uint32_t cp) {  // src/tokenizer.rs:225-236
  return (cp >= 0x4E00 && cp <= 0x9FFF) || (cp >= 0x3400 && cp <= 0x4DBF) || (cp >= 0x20000 && cp <= 0x2A6DF) ||
         (cp >= 0x2A700 && cp <= 0x2B73F) || (cp >= 0x2B740 && cp <= 0x2B81F) || (cp >= 0x2B820 && cp <= 0x2CEAF) ||
         (cp >= 0xF900 && cp <= 0xFAFF) || (cp >= 0x2F800 && cp <= 0x2FA1F);
}
bool is_bert_punctuation(uint32_t cp) {  // src/tokenizer.rs:238-286
  if ((cp >= 33 && cp <= 47) || (cp >= 58 && cp <= 64) || (cp >= 91 && cp <= 96) || (cp >= 123 && cp <= 126))
    return true;
  if ((cp >= 0x2000 && cp <= 0x206F) || (cp >= 0x3000 && cp <= 0x303F) || (cp >= 0xFE30 && cp <= 0xFE6F) ||
      (cp >= 0xFF01 && cp <= 0xFF0F) || (cp >= 0xFF1A && cp <= 0xFF20) || (cp >= 0xFF3B && cp <= 0xFF40) ||
      (cp >= 0xFF5B && cp <= 0xFF65))
    return true;
  switch (cp) {
    case 0xA1: case 0xA7: case 0xAB: case 0xB6: case 0xB7: case 0xBB: case 0xBF:
      return true;
    default:
      return false;  // the remaining listed characters all lie in U+2000..U+206F
  }
}
bool is_combining_mark(uint32_t cp) {  // src/tokenizer.rs:288-296
  return (cp >= 0x0300 && cp <= 0x036F) || (cp >= 0x1AB0 && cp <= 0x1AFF) || (cp >= 0x1DC0 && cp <= 0x1DFF) ||
         (cp >= 0x20D0 && cp <= 0x20FF) || (cp >= 0xFE20 && cp <= 0xFE2F);
}
// precomposed Latin-1 / Latin Extended-A letters -> NFD base (src/tokenizer.rs:298-327)
uint32_t strip_latin_accent(uint32_t c) {
  auto in = [&](uint32_t a, uint32_t b) { return c >= a && c <= b; };
  if (in(0xC0, 0xC5) || in(0xE0, 0xE5) || in(0x100, 0x104)) return 'a';
  if (c == 0xC7 || c == 0xE7 || in(0x106, 0x10C)) return 'c';
  if (c == 0x10E || c == 0x10F) return 'd';
  if (in(0xC8, 0xCB) || in(0xE8, 0xEB) || in(0x112, 0x11A)) return 'e';
  if (in(0x11C, 0x122)) return 'g';
  if (c == 0x124 || c == 0x125) return 'h';
  if (in(0xCC, 0xCF) || in(0xEC, 0xEF) || in(0x128, 0x12E)) return 'i';
  if (c == 0x134 || c == 0x135) return 'j';
  if (c == 0x136 || c == 0x137) return 'k';
  if (in(0x139, 0x13E)) return 'l';
  if (c == 0xD1 || c == 0xF1 || in(0x143, 0x147)) return 'n';
  if (in(0xD2, 0xD6) || in(0xF2, 0xF6) || in(0x14C, 0x150)) return 'o';
  if (in(0x154, 0x158)) return 'r';
  if (in(0x15A, 0x160) || in(0x15B, 0x161)) return 's';
  if (in(0x162, 0x164)) return 't';
  if (in(0xD9, 0xDC) || in(0xF9, 0xFC) || in(0x168, 0x172)) return 'u';
  if (c == 0x174 || c == 0x175) return 'w';
  if (c == 0xDD || c == 0xFD || c == 0xFF || c == 0x176 || c == 0x177 || c == 0x178) return 'y';
  if (in(0x179, 0x17E)) return 'z';
  return c;
}

// char::to_lowercase
void to_lower(uint32_t c, uint32_t out[3], int& n) {
  n = 1;
  out[0] = c;
  if (c < 0x80) {
    if (c >= 'A' && c <= 'Z') out[0] = c + 32;
    return;
  }
  const size_t ns = sizeof(kLowerSingle) / sizeof(kLowerSingle[0]);
  size_t lo = 0, hi = ns;
  while (lo < hi) {
    size_t mid = (lo + hi) / 2;
    if (kLowerSingle[mid][0] < c) lo = mid + 1; else hi = mid;
  }
  if (lo < ns && kLowerSingle[lo][0] == c) {
    out[0] = kLowerSingle[lo][1];
    return;
  }
  for (const auto& m : kLowerMulti) {
    if (m[0] == c) {
      n = 0;
      for (int k = 1; k < 4 && m[k]; k++) out[n++] = m[k];
      return;
    }
  }
}

}  // namespace

int Tokenizer::load_vocab_file(const std::string& path, std::string& err) {
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) {
    err = "cannot open " + path;
    return AE_ERR_NOT_FOUND;
  }
  std::string text;
  char buf[65536];
  size_t got;
  while ((got = std::fread(buf, 1, sizeof(buf), f)) > 0) text.append(buf, got);
  std::fclose(f);
  load_vocab_str(text);
  return AE_OK;
}

void Tokenizer::load_vocab_str(const std::string& text) {
  root_.clear();
  sub_.clear();
  id_to_token_.clear();
  size_t pos = 0, idx = 0;
  while (pos < text.size()) {  // str::lines: split on '\n'; a '\r' before it is dropped
    size_t nl = text.find('\n', pos);
    size_t end = nl == std::string::npos ? text.size() : nl;
    std::string line = text.substr(pos, end - pos);
    if (nl != std::string::npos && !line.empty() && line.back() == '\r') line.pop_back();
    const uint16_t id = uint16_t(idx);
    if (line.size() > 2 && line[0] == '#' && line[1] == '#') sub_[line.substr(2)] = id;
    root_[line] = id;
    id_to_token_.push_back(line);
    idx++;
    if (nl == std::string::npos) break;
    pos = nl + 1;
  }
  query_prefix_ids_.clear();
  encode_raw(kQueryPrefix, query_prefix_ids_);
}

void Tokenizer::encode(const std::string& text, bool is_query, std::vector<uint16_t>& out) const {
  out.clear();
  out.push_back(kCls);
  if (is_query) out.insert(out.end(), query_prefix_ids_.begin(), query_prefix_ids_.end());
  encode_raw(text, out);
  if (out.size() >= kMaxSeqLen) out.resize(kMaxSeqLen - 1);
  out.push_back(kSep);
}

void Tokenizer::encode_raw(const std::string& text, std::vector<uint16_t>& out) const {
  // BertNormalizer (src/tokenizer.rs:105-130)
  std::u32string norm;
  norm.reserve(text.size() + 16);
  for (uint32_t ch : decode_utf8(text)) {
    if (ch == 0 || ch == 0xFFFD || is_bert_control(ch)) continue;
    if (is_bert_whitespace(ch)) {
      norm.push_back(' ');
      continue;
    }
    if (is_chinese_char(ch)) {
      norm.push_back(' ');
      norm.push_back(ch);
      norm.push_back(' ');
      continue;
    }
    if (is_combining_mark(ch)) continue;
    uint32_t lc[3];
    int nl;
    to_lower(strip_latin_accent(ch), lc, nl);
    for (int k = 0; k < nl; k++)
      if (!is_combining_mark(lc[k])) norm.push_back(lc[k]);
  }
  // BertPreTokenizer + WordPiece (src/tokenizer.rs:132-154)
  std::string word;
  bool in_word = false;
  auto flush = [&]() {
    if (in_word) wordpiece(word, out);
    word.clear();
    in_word = false;
  };
  for (uint32_t ch : norm) {
    if (ch == ' ') {
      flush();
    } else if (is_bert_punctuation(ch)) {
      flush();
      std::string p;
      append_utf8(p, ch);
      wordpiece(p, out);
    } else {
      append_utf8(word, ch);
      in_word = true;
    }
  }
  flush();
}

void Tokenizer::wordpiece(const std::string& word, std::vector<uint16_t>& out) const {  // :157-208
  if (word.empty()) return;
  auto it = root_.find(word);
  if (it != root_.end()) {
    out.push_back(it->second);
    return;
  }
  size_t chars = 0;
  for (unsigned char c : word)
    if ((c & 0xC0) != 0x80) chars++;
  if (chars > kMaxWordChars) {
    out.push_back(kUnk);
    return;
  }
  const size_t start_out = out.size();
  size_t start = 0;
  const size_t len = word.size();
  while (start < len) {
    size_t end = len;
    bool found = false;
    uint16_t id = 0;
    while (end > start) {
      const std::string slice = word.substr(start, end - start);
      const auto& table = start == 0 ? root_ : sub_;
      auto m = table.find(slice);
      if (m != table.end()) {
        id = m->second;
        found = true;
        break;
      }
      end--;  // back to the previous UTF-8 boundary
      while (end > start && (((unsigned char)word[end]) & 0xC0) == 0x80) end--;
    }
    if (!found) {
      out.resize(start_out);
      out.push_back(kUnk);
      return;
    }
    out.push_back(id);
    start = end;
  }
}

void Tokenizer::encode_batch(const char* const* texts, size_t n, bool is_query, int num_threads,
                             std::vector<std::vector<uint16_t>>& out) const {
  out.assign(n, {});
  const size_t threads = std::max<size_t>(1, std::min<size_t>(size_t(num_threads < 1 ? 1 : num_threads), n));
  if (threads == 1) {
    for (size_t i = 0; i < n; i++) encode(texts[i] ? texts[i] : "", is_query, out[i]);
    return;
  }
  std::vector<std::thread> pool;
  for (size_t t = 0; t < threads; t++)
    pool.emplace_back([&, t]() {
      for (size_t i = t; i < n; i += threads) encode(texts[i] ? texts[i] : "", is_query, out[i]);
    });
  for (auto& th : pool) th.join();
}

}  // namespace ae
