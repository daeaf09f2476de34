// tokenizer.hpp -- BERT WordPiece tokenizer (host side of the text API).
//
// Restates the reference's BertTokenizer (src/tokenizer.rs): vocab.txt loading
// with separate root / "##" subword tables, BertNormalizer (control removal,
// whitespace folding, CJK isolation, Latin accent stripping, lowercase),
// whitespace + punctuation pre-tokenization, greedy longest-match WordPiece,
// `[CLS] (+ query prefix) ... [SEP]` framing truncated to 512 ids.
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace ae {

class Tokenizer {
 public:
  static constexpr uint16_t kUnk = 100, kCls = 101, kSep = 102;  // src/tokenizer.rs:15-21
  static constexpr size_t kMaxSeqLen = 512;
  static constexpr size_t kMaxWordChars = 100;

  int load_vocab_file(const std::string& path, std::string& err);  // from_vocab_file, :34-37
  void load_vocab_str(const std::string& text);                    // from_vocab_str, :39-66
  size_t vocab_size() const { return id_to_token_.size(); }
  // encode_into (src/tokenizer.rs:91-102)
  void encode(const std::string& text, bool is_query, std::vector<uint16_t>& out) const;
  void encode_batch(const char* const* texts, size_t n, bool is_query, int num_threads,
                    std::vector<std::vector<uint16_t>>& out) const;

 private:
  void encode_raw(const std::string& text, std::vector<uint16_t>& out) const;
  void wordpiece(const std::string& word, std::vector<uint16_t>& out) const;
  std::unordered_map<std::string, uint16_t> root_, sub_;
  std::vector<std::string> id_to_token_;
  std::vector<uint16_t> query_prefix_ids_;
};

}  // namespace ae
