// ae8.hpp -- host-side `.ae8` quantized pack: reader and seeded synthetic writer.
//
// Byte layout (reference src/quantize.rs:76-137, :168-208): little-endian;
// vec_i8 = u64 len + bytes; vec_f32 = u64 len + len*f32; linear = u64 n_out,
// u64 k_in, vec_i8 w_q [n_out*k_in] row-major, vec_f32 w_scale[n_out],
// vec_f32 bias[n_out], vec_f32 inv_smooth[k_in].
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace ae {

constexpr int kHidden = 384;
constexpr int kInter = 1536;
constexpr int kHeads = 12;
constexpr int kHeadDim = 32;
constexpr int kLayers = 12;
constexpr int kVocab = 30522;
constexpr int kMaxPos = 512;
constexpr float kLnEps = 1e-12f;

// QuantizedLinearRaw (src/quantize.rs:23-30)
struct LinearRaw {
  uint64_t n_out = 0, k_in = 0;
  std::vector<int8_t> w_q;
  std::vector<float> w_scale, bias, inv_smooth;
};

// QuantizedLayerRaw (src/quantize.rs:47-59)
struct LayerRaw {
  LinearRaw qkv;
  bool has_split = false;
  LinearRaw q_only, kv_only;
  LinearRaw attn_out;
  std::vector<float> ln1_w, ln1_b;
  LinearRaw ffn_inter, ffn_out;
  std::vector<float> ln2_w, ln2_b;
};

// QuantizedModelRaw (src/quantize.rs:62-72)
struct ModelRaw {
  std::vector<int8_t> word_q, pos_q, type_q;
  std::vector<float> word_s, pos_s, type_s;
  std::vector<float> emb_ln_w, emb_ln_b;
  std::vector<LayerRaw> layers;
  size_t size_bytes() const;  // QuantizedModelRaw::size_bytes, src/quantize.rs:140-165
};

// Status codes shared with the C ABI (AE_OK / AE_ERR_*).
// QuantizedModelRaw::load_ae8 (src/quantize.rs:76-137).
int load_ae8(const std::string& path, ModelRaw& out, std::string& err);
// Checks the shapes the engine relies on (the reference asserts them later, in
// PackedLinearInt8::from_raw_row_major, src/gemm.rs:207-212, and forward_cls's
// unwraps of layer 11's split, src/model.rs:403-404).
int validate_model(const ModelRaw& m, std::string& err);

// Seeded synthetic model in `.ae8` layout: xoshiro256**
// seeded by SplitMix64, Box-Muller normals in double precision.
int write_synthetic_ae8(const std::string& path, uint64_t seed, std::string& err);

}  // namespace ae
