// Host-side driver for the AddressSanitizer / UndefinedBehaviorSanitizer build of
// the product's .ae8 loader (csrc/ae8.cpp), its WordPiece tokenizer
// (csrc/tokenizer.cpp) and the CPU oracle (oracle/oracle.c, oracle/x86.c).
// Built by tests/sanitize/Makefile with g++/gcc only (no GPU code); run by
// tests/test_sanitize.py, which compares what it prints with the unsanitized
// libraries' results.
//
//   driver loader <dir>                 synthetic pack write/load, truncations, bad magic
//   driver tokenize <vocab> <in> <out>  texts in, ids out (length-prefixed records)
//   driver oracle <pack> <in> <out>     every oracle driver over one packed batch
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <string>
#include <vector>

#include "../../include/arctic_embed.h"
#include "../../oracle/oracle.h"
#include "../../snowflake-arctic-embed-s-rust_amd/csrc/ae8.hpp"
#include "../../snowflake-arctic-embed-s-rust_amd/csrc/tokenizer.hpp"

namespace {

int fails = 0;
void check(bool ok, const char* what, long detail = 0) {
  if (!ok) {
    std::fprintf(stderr, "FAIL %s (%ld)\n", what, detail);
    ++fails;
  }
}

std::vector<char> read_all(const std::string& p) {
  std::ifstream f(p, std::ios::binary);
  return std::vector<char>((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
}
void write_all(const std::string& p, const void* d, size_t n) {
  std::ofstream f(p, std::ios::binary);
  f.write(static_cast<const char*>(d), static_cast<std::streamsize>(n));
}

// The product loader and the oracle loader must agree on every outcome.
int or_code_to_ae(int c) {
  switch (c) {
    case OR_OK: return AE_OK;
    case OR_ERR_IO: return AE_ERR_NOT_FOUND;
    case OR_ERR_INVALID_DATA: return AE_ERR_INVALID_DATA;
    case OR_ERR_EOF: return AE_ERR_EOF;
    default: return AE_ERR_INVALID_ARG;
  }
}

int load_both(const std::string& path, size_t* size_ae, size_t* size_or) {
  ae::ModelRaw m;
  std::string err;
  int a = ae::load_ae8(path, m, err);
  if (a == AE_OK) {
    a = ae::validate_model(m, err);
    if (size_ae) *size_ae = m.size_bytes();
  }
  or_model* om = nullptr;
  int o = or_code_to_ae(or_load_ae8(path.c_str(), &om));
  if (om) {
    if (size_or) *size_or = or_size_bytes(om);
    or_free(om);
  }
  check(a == o || (o == AE_OK && a == AE_ERR_INVALID_DATA), "loaders disagree", a * 100 + o);
  return a;
}

int run_loader(const std::string& dir) {
  const std::string pack = dir + "/model.ae8";
  std::string err;
  check(ae::write_synthetic_ae8(pack, 0xAE85EED, err) == AE_OK, "write_synthetic_ae8");
  size_t sa = 0, so = 0;
  check(load_both(pack, &sa, &so) == AE_OK, "load synthetic");
  check(sa == so && sa > 0, "size_bytes agree", static_cast<long>(sa) - static_cast<long>(so));
  check(load_both(dir + "/missing.ae8", nullptr, nullptr) == AE_ERR_NOT_FOUND, "missing file");

  std::vector<char> data = read_all(pack);
  std::vector<char> bad = data;
  bad[6] = '9';
  write_all(dir + "/bad.ae8", bad.data(), bad.size());
  check(load_both(dir + "/bad.ae8", nullptr, nullptr) == AE_ERR_INVALID_DATA, "bad magic");

  // every cut inside the header and the first tensor headers, then a stride over the rest
  std::vector<size_t> cuts;
  for (size_t c = 0; c < 160 && c < data.size(); ++c) cuts.push_back(c);
  for (size_t c = 160; c < data.size(); c += data.size() / 97 + 1) cuts.push_back(c);
  cuts.push_back(data.size() - 1);
  const std::string tp = dir + "/trunc.ae8";
  for (size_t c : cuts) {
    write_all(tp, data.data(), c);
    check(load_both(tp, nullptr, nullptr) == AE_ERR_EOF, "truncated pack", static_cast<long>(c));
  }
  // trailing bytes are ignored, as in the reference
  std::vector<char> longer = data;
  longer.insert(longer.end(), 13, '\x7f');
  write_all(tp, longer.data(), longer.size());
  check(load_both(tp, nullptr, nullptr) == AE_OK, "trailing bytes");
  std::printf("loader: %zu cuts, size_bytes %zu\n", cuts.size(), sa);
  return fails ? 1 : 0;
}

// records: u8 is_query, u32 n_bytes, bytes
int run_tokenize(const std::string& vocab, const std::string& in, const std::string& out) {
  ae::Tokenizer tok;
  std::string err;
  if (tok.load_vocab_file(vocab, err) != AE_OK) {
    std::fprintf(stderr, "vocab: %s\n", err.c_str());
    return 2;
  }
  std::vector<char> d = read_all(in);
  std::vector<std::string> texts;
  std::vector<int> query;
  for (size_t at = 0; at + 5 <= d.size();) {
    uint32_t n;
    std::memcpy(&n, &d[at + 1], 4);
    query.push_back(d[at]);
    texts.emplace_back(&d[at + 5], n);
    at += 5 + n;
  }
  std::vector<uint16_t> flat;
  std::vector<uint32_t> offs{0};
  for (size_t i = 0; i < texts.size(); ++i) {
    std::vector<uint16_t> ids;
    tok.encode(texts[i], query[i] != 0, ids);
    flat.insert(flat.end(), ids.begin(), ids.end());
    offs.push_back(static_cast<uint32_t>(flat.size()));
  }
  // the threaded batch path returns the same ids
  std::vector<const char*> ptrs;
  for (auto& t : texts) ptrs.push_back(t.c_str());
  for (int q = 0; q < 2; ++q) {
    std::vector<std::vector<uint16_t>> batch;
    tok.encode_batch(ptrs.data(), ptrs.size(), q != 0, 4, batch);
    check(batch.size() == texts.size(), "encode_batch size");
    for (size_t i = 0; i < texts.size() && i < batch.size(); ++i) {
      if (query[i] != q || texts[i].find('\0') != std::string::npos) continue;
      check(std::vector<uint16_t>(flat.begin() + offs[i], flat.begin() + offs[i + 1]) == batch[i],
            "encode_batch ids", static_cast<long>(i));
    }
  }
  std::ofstream f(out, std::ios::binary);
  uint32_t n = static_cast<uint32_t>(texts.size());
  f.write(reinterpret_cast<const char*>(&n), 4);
  f.write(reinterpret_cast<const char*>(offs.data()), offs.size() * 4);
  f.write(reinterpret_cast<const char*>(flat.data()), flat.size() * 2);
  std::printf("tokenize: %u texts, %zu ids\n", n, flat.size());
  return fails ? 1 : 0;
}

// in: u32 b, u32 offsets[b+1], u16 ids[offsets[b]]
// out: forward_cls of sequence 0, then [b,384] for ragged, batch (1 and 4 threads),
//      x86 backend batch, ArmSme-attention batch; then the attention kernels on
//      seeded qkv rows
int run_oracle(const std::string& pack, const std::string& in, const std::string& out) {
  or_model* m = nullptr;
  if (or_load_ae8(pack.c_str(), &m) != OR_OK) return 2;
  std::vector<char> d = read_all(in);
  uint32_t b;
  std::memcpy(&b, d.data(), 4);
  std::vector<uint32_t> offs(b + 1);
  std::memcpy(offs.data(), &d[4], 4 * (b + 1));
  std::vector<uint16_t> ids(offs[b]);
  std::memcpy(ids.data(), &d[4 + 4 * (b + 1)], 2 * ids.size());

  const size_t H = OR_HIDDEN;
  std::vector<float> res;
  std::vector<float> v(H * b);
  check(or_forward_cls(m, ids.data(), offs[1], v.data()) == OR_OK, "forward_cls");
  res.insert(res.end(), v.begin(), v.begin() + H);
  check(or_forward_ragged_cls(m, ids.data(), offs.data(), static_cast<int>(b), v.data()) == OR_OK, "ragged");
  res.insert(res.end(), v.begin(), v.end());
  for (int th : {1, 4}) {
    check(or_embed_batch_tokens(m, ids.data(), offs.data(), b, th, v.data()) == OR_OK, "embed_batch");
    res.insert(res.end(), v.begin(), v.end());
  }
  int x86 = or_x86_backend();
  check(or_x86_prepare(m) == OR_OK, "x86_prepare");
  check(or_x86_embed_batch_tokens(m, ids.data(), offs.data(), b, 2, v.data()) == OR_OK, "x86 batch");
  res.insert(res.end(), v.begin(), v.end());
  check(or_embed_tokens_sme(m, ids.data(), offs.data(), static_cast<int>(b), v.data()) == OR_OK, "sme batch");
  res.insert(res.end(), v.begin(), v.end());

  // attention over a ragged packed batch: exact per head, and the quantized form
  const int cu[4] = {0, 1, 19, 52};
  const int T = cu[3];
  std::vector<float> qkv(static_cast<size_t>(T) * 1152), ctx(static_cast<size_t>(T) * H, 0.f);
  uint64_t s = 0x9E3779B97F4A7C15ull;
  for (auto& x : qkv) {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    x = static_cast<float>(static_cast<int32_t>(s >> 40) - (1 << 23)) * (1.0f / (1 << 22));
  }
  for (int seg = 0; seg < 3; ++seg)
    for (int h = 0; h < OR_HEADS; ++h)
      or_attention_head(&qkv[static_cast<size_t>(cu[seg]) * 1152], cu[seg + 1] - cu[seg], 1152, h * 32,
                        384 + h * 32, 768 + h * 32, &ctx[static_cast<size_t>(cu[seg]) * H + h * 32], 384);
  res.insert(res.end(), ctx.begin(), ctx.end());
  or_attention_sme(qkv.data(), T, cu, 3, ctx.data());
  res.insert(res.end(), ctx.begin(), ctx.end());
  or_free(m);
  write_all(out, res.data(), res.size() * 4);
  std::printf("oracle: %u sequences, %zu ids, x86 backend %d\n", b, ids.size(), x86);
  return fails ? 1 : 0;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc >= 3 && !std::strcmp(argv[1], "loader")) return run_loader(argv[2]);
  if (argc >= 5 && !std::strcmp(argv[1], "tokenize")) return run_tokenize(argv[2], argv[3], argv[4]);
  if (argc >= 5 && !std::strcmp(argv[1], "oracle")) return run_oracle(argv[2], argv[3], argv[4]);
  std::fprintf(stderr, "usage: driver loader <dir> | tokenize <vocab> <in> <out> | oracle <pack> <in> <out>\n");
  return 2;
}
