/*
 * oracle.h -- CPU restatement of the reference's scalar int8 encoder path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * engine.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it; the product library never links or calls it.
 *
 * Every function restates one scalar fallback of mdlockyer/snowflake-arctic-
 * embed-s-rust, in the same evaluation order (no FMA contraction, left-to-right
 * products, sequential float sums, round-half-away-from-zero).  The cited lines
 * are in the reference tree (src/...).  Transcendentals come from the platform
 * libm (glibc expf / sqrtf), exactly as Rust's f32::exp / f32::sqrt do on
 * x86_64 Linux.
 */
#ifndef AE_ORACLE_H
#define AE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/quantize.rs:9-18 */
#define OR_HIDDEN 384
#define OR_INTER 1536
#define OR_HEADS 12
#define OR_HEAD_DIM 32
#define OR_LAYERS 12
#define OR_VOCAB 30522
#define OR_MAX_POS 512
#define OR_LN_EPS 1e-12f

/* status codes, mirroring io::ErrorKind outcomes of load_ae8 (src/quantize.rs:76-137) */
#define OR_OK 0
#define OR_ERR_IO (-1)           /* file missing / unreadable (fs::read)          */
#define OR_ERR_INVALID_DATA (-2) /* bad magic (ErrorKind::InvalidData)            */
#define OR_ERR_EOF (-3)          /* truncated stream (read_exact -> UnexpectedEof) */
#define OR_ERR_ARG (-4)

/* QuantizedLinearRaw (src/quantize.rs:23-30); weights stay row-major [n_out, k_in]. */
typedef struct {
  uint64_t n_out, k_in;
  uint64_t w_len, s_len, b_len, is_len; /* vector lengths exactly as stored */
  int8_t* w_q;
  float* w_scale;
  float* bias;
  float* inv_smooth;
  int8_t* xpack;  /* x86 CPU baseline only: weights in pack_weights_x86 order, else NULL */
  int32_t* xcomp; /* x86 CPU baseline only: -128 * row sums (VNNI col_sum_comp), else NULL */
} or_linear;

/* QuantizedLayerRaw (src/quantize.rs:47-59) */
typedef struct {
  or_linear qkv;
  int has_split;
  or_linear q_only, kv_only;
  or_linear attn_out;
  float *ln1_w, *ln1_b;
  uint64_t ln1_w_len, ln1_b_len;
  or_linear ffn_inter, ffn_out;
  float *ln2_w, *ln2_b;
  uint64_t ln2_w_len, ln2_b_len;
} or_layer;

/* QuantizedModelRaw (src/quantize.rs:62-72) + PackedModel::type0_emb_f32 (src/model.rs:50-54) */
typedef struct {
  int8_t* word_q; uint64_t word_q_len;
  float* word_s;  uint64_t word_s_len;
  int8_t* pos_q;  uint64_t pos_q_len;
  float* pos_s;   uint64_t pos_s_len;
  int8_t* type_q; uint64_t type_q_len;
  float* type_s;  uint64_t type_s_len;
  float* emb_ln_w; uint64_t emb_ln_w_len;
  float* emb_ln_b; uint64_t emb_ln_b_len;
  or_layer layers[OR_LAYERS];
  float type0[OR_HIDDEN];
} or_model;

/* ---- format: src/quantize.rs:76-208 ------------------------------------ */
int or_load_ae8(const char* path, or_model** out);
void or_free(or_model* m);
size_t or_size_bytes(const or_model* m); /* QuantizedModelRaw::size_bytes, src/quantize.rs:140-165 */

/* ---- kernels: scalar fallbacks ------------------------------------------ */
/* gemm_scalar_fused, src/gemm.rs:2000-2029.  a:[m,k] row-major, res nullable. */
void or_gemm(int m, const int8_t* a, const float* a_scale, const or_linear* w,
             const float* res, float* out);
/* same, also returning the int32 accumulators (acc may be NULL) */
void or_gemm_acc(int m, int n, int k, const int8_t* a, const int8_t* w_rowmajor,
                 int32_t* acc);
/* layernorm_smooth_quantize_row_scalar, src/simd_math.rs:208-247 */
float or_ln_quant_row(float* x, const float* gamma, const float* beta,
                      const float* inv_smooth, int8_t* q, int n, float eps);
/* layernorm_inplace_row, src/simd_math.rs:481-497 */
void or_ln_row(float* x, const float* gamma, const float* beta, int n, float eps);
/* smooth_quantize_row scalar branch, src/simd_math.rs:513-530 */
float or_smooth_quant_row(const float* x, const float* inv_smooth, int8_t* q, int n);
/* scalar_gelu, src/simd_math.rs:15-23 */
float or_gelu(float x);
/* or_gelu over n floats */
void or_gelu_map(const float* x, float* y, size_t n);
/* gelu_smooth_quantize_row scalar branch, src/simd_math.rs:1295-1312 */
float or_gelu_quant_row(float* x, const float* inv_smooth, int8_t* q, int n);
/* dot32_f32 scalar branch, src/simd_math.rs:1461-1468 */
float or_dot32(const float* a, const float* b);
/* compute_scores_head32 scalar branch, src/simd_math.rs:1587-1590 */
void or_scores(const float* q, const float* k_head, float scale, float* scores, int len);
/* softmax_inplace scalar branch, src/simd_math.rs:1684-1702 */
void or_softmax(float* s, int len);
/* weighted_sum_head32 scalar branch, src/simd_math.rs:1812-1821 */
void or_wsum(const float* p, const float* v_head, int len, float* out32);
/* dequant_add_embeddings_row scalar branch, src/simd_math.rs:1877-1880 */
void or_emb_row(const int8_t* w_row, float w_s, const int8_t* p_row, float p_s,
                const float* t_row, float* h_row, int n);
/* l2_normalize_inplace, src/simd_math.rs:2892-2903 */
void or_l2(float* v, int n);
/* one attention head for one segment: qkv rows [len, stride], writes ctx rows (stride 384)
   (src/model.rs:663-694 restricted to one head) */
void or_attention_head(const float* qkv, int len, int stride, int q_off, int k_off,
                       int v_off, float* ctx, int ctx_stride);

/* Quantized attention of the reference's ArmSme backend over a packed batch of T
   tokens in B segments (cu[B+1]): attention_multihead_sme with seg_ranges
   (src/model.rs:607-621; src/simd_math.rs:1933-2192), restated in scalar C:
   per-token int8 Q and K (quantize_head32_row_neon, :2482-2526; K's scale also
   carries log2(e)/sqrt(32)), per-column int8 V over all T tokens
   (pack_qkv_head_int8_neon, :2564-2640; quantize_v_row_neon, :2530-2559),
   integer scores, the two-pass exact-range int16 softmax per segment row
   (softmax_quantize_i16_from_acc_neon, :2291-2336, with exp2_q_neon's
   polynomial for 8-aligned chunks and exp2f for the row's last len % 8 keys,
   :2353-2410), integer P @ V and ctx = f32(acc) * (v_scale * p_scale).
   qkv: [T, 1152] f32; ctx: [T, 384] f32. */
void or_attention_sme(const float* qkv, int T, const int* cu, int B, float* ctx);
/* exp2_q_neon for one lane: round(scale * 2^x) for x <= 0, x clamped at x_min
   (src/simd_math.rs:2353-2370) */
int32_t or_exp2_q(float x, float scale, float x_min);

/* ---- backend kernel table ------------------------------------------------
 * The drivers below (src/model.rs forward passes, src/lib.rs embed_batch) call
 * their row / GEMM / attention kernels through this table, as the reference
 * dispatches per SimdBackend (src/gemm.rs:630-671, src/simd_math.rs dispatchers).
 * or_scalar_kernels is the oracle; oracle/x86.c provides the reference's x86
 * backend for the CPU baseline. */
typedef struct {
  void (*gemm)(int m, const int8_t* a, const float* a_scale, const or_linear* w, const float* res, float* out);
  float (*ln_quant_row)(float* x, const float* gamma, const float* beta, const float* inv_smooth, int8_t* q,
                        int n, float eps);
  float (*smooth_quant_row)(const float* x, const float* inv_smooth, int8_t* q, int n);
  float (*gelu_quant_row)(float* x, const float* inv_smooth, int8_t* q, int n);
  void (*scores)(const float* q, const float* k_head, float scale, float* scores, int len);
  void (*softmax)(float* s, int len);
  void (*wsum)(const float* p, const float* v_head, int len, float* out32);
} or_kernels;
extern const or_kernels or_scalar_kernels;
/* oracle/x86.c: the reference's x86 backend, used as the CPU baseline.
 * or_x86_backend: 2 AVX-VNNI, 1 AVX2+FMA, 0 none (src/gemm.rs:100-125).
 * or_x86_prepare packs every linear (pack_weights_x86, col_sum_comp). */
int or_x86_backend(void);
int or_x86_prepare(or_model* m);
int or_x86_embed_batch_tokens(const or_model* m, const uint16_t* ids, const uint32_t* offsets, size_t n,
                              int num_threads, float* out);
int or_x86_gemm(int m, const int8_t* a, const float* a_scale, or_linear* w, const float* res, float* out,
                int variant);
/* embed_batch over ids with an explicit backend table */
int or_embed_batch_tokens_k(const or_model* m, const uint16_t* ids, const uint32_t* offsets, size_t n,
                            int num_threads, float* out, const or_kernels* k);

/* ---- drivers ------------------------------------------------------------ */
/* PackedModel::forward_cls, src/model.rs:185-513 */
int or_forward_cls(const or_model* m, const uint16_t* ids, size_t n, float* out384);
/* same forward with layer 11 run unpruned over all rows (CLS row returned); test hook */
int or_forward_cls_unpruned(const or_model* m, const uint16_t* ids, size_t n, float* out384);
/* PackedModel::forward_ragged_cls, src/model.rs:521-914 (<= 64 seqs, 512 total tokens) */
int or_forward_ragged_cls(const or_model* m, const uint16_t* ids, const uint32_t* offsets,
                          int b, float* out);
/* ArcticEmbedS::embed_batch scheduling (src/lib.rs:138-260) over pre-tokenized ids;
   offsets has n+1 entries; num_threads worker threads with atomic work stealing. */
int or_embed_batch_tokens(const or_model* m, const uint16_t* ids, const uint32_t* offsets,
                          size_t n, int num_threads, float* out);

/* per-layer intermediate taps for kernel-level parity tests.  Runs forward_cls
   semantics on one packed batch of segments (offsets[b+1]) through the embedding
   and layers [0, upto_layer) and returns hidden/act_q/act_scale at that point. */
int or_run_prefix(const or_model* m, const uint16_t* ids, const uint32_t* offsets, int b,
                  int upto_layer, float* hidden, int8_t* act_q, float* act_scale);
/* or_run_prefix with the ArmSme backend's quantized attention in layers 0-10,
   per sequence as forward_cls runs it (src/model.rs:244-259): or_attention_sme
   over the sequence alone when it has >= 16 tokens, the exact attention below */
int or_run_prefix_sme(const or_model* m, const uint16_t* ids, const uint32_t* offsets, int b,
                      int upto_layer, float* hidden, int8_t* act_q, float* act_scale);
/* test hook: forward_cls with act_q[row][col] moved one int8 step (+1, or -1 at
   127) at the input of encoder layer `layer` (0..10) */
int or_forward_cls_perturbed(const or_model* m, const uint16_t* ids, size_t n, int layer, int row, int col,
                             float* out384);
/* the whole forward_cls of each of the b sequences (offsets[b+1], each truncated
   to 512) with the ArmSme backend's attention as or_run_prefix_sme applies it;
   out [b, 384] */
int or_embed_tokens_sme(const or_model* m, const uint16_t* ids, const uint32_t* offsets, int b, float* out);

#ifdef __cplusplus
}
#endif
#endif
