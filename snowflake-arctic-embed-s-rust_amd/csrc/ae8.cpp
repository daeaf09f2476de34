// ae8.cpp -- `.ae8` reader (src/quantize.rs:76-208) and seeded synthetic writer.
#include "ae8.hpp"

#include <cmath>
#include <cstdio>
#include <cstring>

#include "../../include/arctic_embed.h"

namespace ae {

namespace {

struct Reader {
  const uint8_t* p;
  size_t left;
  int u64(uint64_t& v) {
    if (left < 8) return AE_ERR_EOF;
    v = 0;
    for (int i = 0; i < 8; i++) v |= uint64_t(p[i]) << (8 * i);
    p += 8;
    left -= 8;
    return AE_OK;
  }
  int i8v(std::vector<int8_t>& out) {  // read_i8_vec (src/quantize.rs:168-176)
    uint64_t n;
    if (int rc = u64(n)) return rc;
    if (n > left) return AE_ERR_EOF;
    out.assign(reinterpret_cast<const int8_t*>(p), reinterpret_cast<const int8_t*>(p) + n);
    p += n;
    left -= n;
    return AE_OK;
  }
  int f32v(std::vector<float>& out) {  // read_f32_vec (src/quantize.rs:178-189)
    uint64_t n;
    if (int rc = u64(n)) return rc;
    if (n > left / 4) return AE_ERR_EOF;
    out.resize(n);
    for (uint64_t i = 0; i < n; i++) {
      uint32_t u = uint32_t(p[4 * i]) | (uint32_t(p[4 * i + 1]) << 8) | (uint32_t(p[4 * i + 2]) << 16) |
                   (uint32_t(p[4 * i + 3]) << 24);
      std::memcpy(&out[i], &u, 4);
    }
    p += n * 4;
    left -= n * 4;
    return AE_OK;
  }
  int linear(LinearRaw& l) {  // read_linear (src/quantize.rs:191-208)
    if (int rc = u64(l.n_out)) return rc;
    if (int rc = u64(l.k_in)) return rc;
    if (int rc = i8v(l.w_q)) return rc;
    if (int rc = f32v(l.w_scale)) return rc;
    if (int rc = f32v(l.bias)) return rc;
    return f32v(l.inv_smooth);
  }
  int byte(uint8_t& b) {
    if (left < 1) return AE_ERR_EOF;
    b = *p++;
    left--;
    return AE_OK;
  }
};

const uint8_t kMagic[8] = {'A', 'R', 'C', 'T', 'I', 'C', '8', 0x01};  // src/quantize.rs:20

size_t linear_bytes(const LinearRaw& l) {
  return l.w_q.size() + (l.w_scale.size() + l.bias.size() + l.inv_smooth.size()) * 4;
}

}  // namespace

size_t ModelRaw::size_bytes() const {
  size_t t = word_q.size() + pos_q.size() + type_q.size() +
             (word_s.size() + pos_s.size() + type_s.size() + emb_ln_w.size() + emb_ln_b.size()) * 4;
  for (const auto& l : layers) {
    t += linear_bytes(l.qkv) + linear_bytes(l.attn_out) + linear_bytes(l.ffn_inter) + linear_bytes(l.ffn_out);
    if (l.has_split) t += linear_bytes(l.q_only) + linear_bytes(l.kv_only);
    t += (l.ln1_w.size() + l.ln1_b.size() + l.ln2_w.size() + l.ln2_b.size()) * 4;
  }
  return t;
}

int load_ae8(const std::string& path, ModelRaw& m, std::string& err) {
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) {
    err = "cannot open " + path;
    return AE_ERR_NOT_FOUND;
  }
  std::fseek(f, 0, SEEK_END);
  long sz = std::ftell(f);
  std::fseek(f, 0, SEEK_SET);
  std::vector<uint8_t> buf(sz > 0 ? size_t(sz) : 0);
  if (sz > 0 && std::fread(buf.data(), 1, buf.size(), f) != buf.size()) {
    std::fclose(f);
    err = "short read on " + path;
    return AE_ERR_NOT_FOUND;
  }
  std::fclose(f);
  Reader r{buf.data(), buf.size()};
  if (r.left < 8) {
    err = "truncated .ae8 (no magic)";
    return AE_ERR_EOF;
  }
  if (std::memcmp(r.p, kMagic, 8) != 0) {
    err = "invalid .ae8 magic header";
    return AE_ERR_INVALID_DATA;
  }
  r.p += 8;
  r.left -= 8;
  int rc;
  auto fail = [&](int code) {
    err = code == AE_ERR_EOF ? "truncated .ae8 pack" : "malformed .ae8 pack";
    return code;
  };
  if ((rc = r.i8v(m.word_q)) || (rc = r.f32v(m.word_s)) || (rc = r.i8v(m.pos_q)) || (rc = r.f32v(m.pos_s)) ||
      (rc = r.i8v(m.type_q)) || (rc = r.f32v(m.type_s)) || (rc = r.f32v(m.emb_ln_w)) ||
      (rc = r.f32v(m.emb_ln_b)))
    return fail(rc);
  m.layers.assign(kLayers, LayerRaw{});
  for (int i = 0; i < kLayers; i++) {  // src/quantize.rs:96-125
    LayerRaw& L = m.layers[i];
    uint8_t split = 0;
    if ((rc = r.linear(L.qkv)) || (rc = r.byte(split))) return fail(rc);
    L.has_split = split == 1;
    if (L.has_split && ((rc = r.linear(L.q_only)) || (rc = r.linear(L.kv_only)))) return fail(rc);
    if ((rc = r.linear(L.attn_out)) || (rc = r.f32v(L.ln1_w)) || (rc = r.f32v(L.ln1_b)) ||
        (rc = r.linear(L.ffn_inter)) || (rc = r.linear(L.ffn_out)) || (rc = r.f32v(L.ln2_w)) ||
        (rc = r.f32v(L.ln2_b)))
      return fail(rc);
  }
  return AE_OK;  // trailing bytes are ignored, as in the reference
}

namespace {
bool lin_ok(const LinearRaw& l, uint64_t n, uint64_t k) {
  return l.n_out == n && l.k_in == k && l.w_q.size() == n * k && l.w_scale.size() == n && l.bias.size() == n &&
         l.inv_smooth.size() == k;
}
}  // namespace

int validate_model(const ModelRaw& m, std::string& err) {
  auto bad = [&](const std::string& what) {
    err = "unexpected .ae8 shape: " + what;
    return AE_ERR_INVALID_DATA;
  };
  if (m.word_q.size() != size_t(kVocab) * kHidden || m.word_s.size() != size_t(kVocab)) return bad("word_emb");
  if (m.pos_q.size() != size_t(kMaxPos) * kHidden || m.pos_s.size() != size_t(kMaxPos)) return bad("pos_emb");
  if (m.type_q.size() < size_t(kHidden) || m.type_s.empty()) return bad("type_emb");
  if (m.emb_ln_w.size() != size_t(kHidden) || m.emb_ln_b.size() != size_t(kHidden)) return bad("emb_ln");
  for (int i = 0; i < kLayers; i++) {
    const LayerRaw& L = m.layers[i];
    std::string li = "layer " + std::to_string(i) + " ";
    if (i < kLayers - 1) {
      if (!lin_ok(L.qkv, 3 * kHidden, kHidden)) return bad(li + "qkv");
    } else {
      // layer 11 keeps only inv_smooth in `qkv` and must carry the Q / KV split
      if (L.qkv.inv_smooth.size() != size_t(kHidden)) return bad(li + "qkv.inv_smooth");
      if (!L.has_split || !lin_ok(L.q_only, kHidden, kHidden) || !lin_ok(L.kv_only, 2 * kHidden, kHidden))
        return bad(li + "q_only/kv_only");
    }
    if (!lin_ok(L.attn_out, kHidden, kHidden)) return bad(li + "attn_out");
    if (!lin_ok(L.ffn_inter, kInter, kHidden)) return bad(li + "ffn_inter");
    if (!lin_ok(L.ffn_out, kHidden, kInter)) return bad(li + "ffn_out");
    if (L.ln1_w.size() != size_t(kHidden) || L.ln1_b.size() != size_t(kHidden) || L.ln2_w.size() != size_t(kHidden) ||
        L.ln2_b.size() != size_t(kHidden))
      return bad(li + "layernorm");
  }
  return AE_OK;
}

// ---------------------------------------------------------------------------
// synthetic writer
// ---------------------------------------------------------------------------
namespace {

struct Rng {  // xoshiro256** seeded through SplitMix64
  uint64_t s[4];
  bool have_spare = false;
  double spare = 0.0;
  explicit Rng(uint64_t seed) {
    uint64_t x = seed;
    for (auto& v : s) {
      x += 0x9E3779B97F4A7C15ull;
      uint64_t z = x;
      z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
      z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
      v = z ^ (z >> 31);
    }
  }
  static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
  uint64_t next() {
    uint64_t r = rotl(s[1] * 5, 7) * 9, t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return r;
  }
  double uniform() { return double(next() >> 11) * 0x1.0p-53; }  // [0, 1)
  double uniform(double lo, double hi) { return lo + (hi - lo) * uniform(); }
  double normal() {  // Box-Muller, both outputs used
    if (have_spare) {
      have_spare = false;
      return spare;
    }
    double u1 = 1.0 - uniform(), u2 = uniform();
    double rad = std::sqrt(-2.0 * std::log(u1)), th = 6.283185307179586 * u2;
    spare = rad * std::sin(th);
    have_spare = true;
    return rad * std::cos(th);
  }
  int8_t int8_sym() { return int8_t(int(next() % 255u) - 127); }  // U{-127..127}
};

struct Writer {
  FILE* f;
  bool ok = true;
  void raw(const void* p, size_t n) { ok = ok && (n == 0 || std::fwrite(p, 1, n, f) == n); }
  void u64(uint64_t v) {
    uint8_t b[8];
    for (int i = 0; i < 8; i++) b[i] = uint8_t(v >> (8 * i));
    raw(b, 8);
  }
  void i8v(const std::vector<int8_t>& v) {
    u64(v.size());
    raw(v.data(), v.size());
  }
  void f32v(const std::vector<float>& v) {
    u64(v.size());
    std::vector<uint8_t> b(v.size() * 4);
    for (size_t i = 0; i < v.size(); i++) {
      uint32_t u;
      std::memcpy(&u, &v[i], 4);
      for (int k = 0; k < 4; k++) b[4 * i + k] = uint8_t(u >> (8 * k));
    }
    raw(b.data(), b.size());
  }
  void linear(const LinearRaw& l) {
    u64(l.n_out);
    u64(l.k_in);
    i8v(l.w_q);
    f32v(l.w_scale);
    f32v(l.bias);
    f32v(l.inv_smooth);
  }
};

// fp32 table ~N(0, 0.02), stored per row as int8 with scale max|row|/127
void quantized_table(Rng& g, int rows, std::vector<int8_t>& q, std::vector<float>& s) {
  q.resize(size_t(rows) * kHidden);
  s.resize(rows);
  std::vector<float> row(kHidden);
  for (int r = 0; r < rows; r++) {
    float mx = 0.f;
    for (int j = 0; j < kHidden; j++) {
      row[j] = float(0.02 * g.normal());
      mx = std::fmax(mx, std::fabs(row[j]));
    }
    float sc = mx > 0.f ? mx / 127.0f : 1.0f;
    s[r] = sc;
    for (int j = 0; j < kHidden; j++) {
      float v = std::round(row[j] / sc);
      v = std::fmin(127.f, std::fmax(-127.f, v));
      q[size_t(r) * kHidden + j] = int8_t(v);
    }
  }
}

LinearRaw synth_linear(Rng& g, int n, int k) {
  LinearRaw l;
  l.n_out = n;
  l.k_in = k;
  l.w_q.resize(size_t(n) * k);
  for (auto& w : l.w_q) w = g.int8_sym();
  l.w_scale.resize(n);
  for (auto& s : l.w_scale) s = float(0.05 / 127.0 * g.uniform(0.5, 1.5));
  l.bias.resize(n);
  for (auto& b : l.bias) b = float(0.02 * g.normal());
  l.inv_smooth.resize(k);
  for (auto& v : l.inv_smooth) v = float(1.0 / g.uniform(0.5, 2.0));
  return l;
}

void synth_ln(Rng& g, std::vector<float>& w, std::vector<float>& b) {
  w.resize(kHidden);
  b.resize(kHidden);
  for (auto& v : w) v = float(1.0 + 0.05 * g.normal());
  for (auto& v : b) v = float(0.02 * g.normal());
}

}  // namespace

int write_synthetic_ae8(const std::string& path, uint64_t seed, std::string& err) {
  Rng g(seed);
  ModelRaw m;
  quantized_table(g, kVocab, m.word_q, m.word_s);
  quantized_table(g, kMaxPos, m.pos_q, m.pos_s);
  quantized_table(g, 2, m.type_q, m.type_s);
  synth_ln(g, m.emb_ln_w, m.emb_ln_b);
  FILE* f = std::fopen(path.c_str(), "wb");
  if (!f) {
    err = "cannot create " + path;
    return AE_ERR_NOT_FOUND;
  }
  Writer w{f};
  w.raw(kMagic, 8);
  w.i8v(m.word_q);
  w.f32v(m.word_s);
  w.i8v(m.pos_q);
  w.f32v(m.pos_s);
  w.i8v(m.type_q);
  w.f32v(m.type_s);
  w.f32v(m.emb_ln_w);
  w.f32v(m.emb_ln_b);
  for (int i = 0; i < kLayers; i++) {
    LinearRaw qkv = synth_linear(g, 3 * kHidden, kHidden);
    LinearRaw attn_out = synth_linear(g, kHidden, kHidden);
    LayerRaw L;
    synth_ln(g, L.ln1_w, L.ln1_b);
    LinearRaw up = synth_linear(g, kInter, kHidden);
    LinearRaw down = synth_linear(g, kHidden, kInter);
    synth_ln(g, L.ln2_w, L.ln2_b);
    if (i < kLayers - 1) {
      w.linear(qkv);
      uint8_t z = 0;
      w.raw(&z, 1);
    } else {
      // layer 11: qkv keeps only inv_smooth; Q rows [0,384) and K|V rows [384,1152) split out
      LinearRaw stub;
      stub.n_out = 0;
      stub.k_in = kHidden;
      stub.inv_smooth = qkv.inv_smooth;
      w.linear(stub);
      uint8_t one = 1;
      w.raw(&one, 1);
      LinearRaw q, kv;
      q.n_out = kHidden;
      kv.n_out = 2 * kHidden;
      q.k_in = kv.k_in = kHidden;
      q.w_q.assign(qkv.w_q.begin(), qkv.w_q.begin() + size_t(kHidden) * kHidden);
      kv.w_q.assign(qkv.w_q.begin() + size_t(kHidden) * kHidden, qkv.w_q.end());
      q.w_scale.assign(qkv.w_scale.begin(), qkv.w_scale.begin() + kHidden);
      kv.w_scale.assign(qkv.w_scale.begin() + kHidden, qkv.w_scale.end());
      q.bias.assign(qkv.bias.begin(), qkv.bias.begin() + kHidden);
      kv.bias.assign(qkv.bias.begin() + kHidden, qkv.bias.end());
      q.inv_smooth = kv.inv_smooth = qkv.inv_smooth;
      w.linear(q);
      w.linear(kv);
    }
    w.linear(attn_out);
    w.f32v(L.ln1_w);
    w.f32v(L.ln1_b);
    w.linear(up);
    w.linear(down);
    w.f32v(L.ln2_w);
    w.f32v(L.ln2_b);
  }
  bool ok = w.ok;
  ok = (std::fclose(f) == 0) && ok;
  if (!ok) {
    err = "write failed for " + path;
    return AE_ERR_NOT_FOUND;
  }
  return AE_OK;
}

}  // namespace ae
