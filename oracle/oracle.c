/*
 * oracle.c -- CPU restatement of the reference's scalar int8 encoder path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker); see oracle.h.  Build with
 * -ffp-contract=off and without -ffast-math: every float operation below is a
 * single IEEE-754 binary32 operation, evaluated in the order the reference's
 * scalar Rust code evaluates it.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* .ae8 reader: src/quantize.rs:76-137 (layout) and :168-208 (vector readers) */
/* ------------------------------------------------------------------------- */

typedef struct {
  const uint8_t* p;
  size_t left;
} cursor_t;

static int rd_u64(cursor_t* c, uint64_t* v) {
  if (c->left < 8) return OR_ERR_EOF;
  uint64_t x = 0;
  for (int i = 0; i < 8; i++) x |= (uint64_t)c->p[i] << (8 * i); /* u64::from_le_bytes */
  c->p += 8;
  c->left -= 8;
  *v = x;
  return OR_OK;
}

static int rd_i8_vec(cursor_t* c, int8_t** out, uint64_t* len) { /* read_i8_vec :168-176 */
  int rc = rd_u64(c, len);
  if (rc) return rc;
  if (*len > c->left) return OR_ERR_EOF;
  *out = (int8_t*)malloc(*len ? *len : 1);
  memcpy(*out, c->p, *len);
  c->p += *len;
  c->left -= *len;
  return OR_OK;
}

static int rd_f32_vec(cursor_t* c, float** out, uint64_t* len) { /* read_f32_vec :178-189 */
  int rc = rd_u64(c, len);
  if (rc) return rc;
  if (*len > c->left / 4) return OR_ERR_EOF;
  *out = (float*)malloc(*len ? *len * 4 : 4);
  for (uint64_t i = 0; i < *len; i++) {
    uint32_t u = (uint32_t)c->p[4 * i] | ((uint32_t)c->p[4 * i + 1] << 8) |
                 ((uint32_t)c->p[4 * i + 2] << 16) | ((uint32_t)c->p[4 * i + 3] << 24);
    memcpy(&(*out)[i], &u, 4); /* f32::from_le_bytes */
  }
  c->p += *len * 4;
  c->left -= *len * 4;
  return OR_OK;
}

static int rd_linear(cursor_t* c, or_linear* l) { /* read_linear :191-208 */
  int rc;
  if ((rc = rd_u64(c, &l->n_out))) return rc;
  if ((rc = rd_u64(c, &l->k_in))) return rc;
  if ((rc = rd_i8_vec(c, &l->w_q, &l->w_len))) return rc;
  if ((rc = rd_f32_vec(c, &l->w_scale, &l->s_len))) return rc;
  if ((rc = rd_f32_vec(c, &l->bias, &l->b_len))) return rc;
  if ((rc = rd_f32_vec(c, &l->inv_smooth, &l->is_len))) return rc;
  return OR_OK;
}

static void free_linear(or_linear* l) {
  free(l->w_q);
  free(l->w_scale);
  free(l->bias);
  free(l->inv_smooth);
  free(l->xpack);
  free(l->xcomp);
}

void or_free(or_model* m) {
  if (!m) return;
  free(m->word_q); free(m->word_s); free(m->pos_q); free(m->pos_s);
  free(m->type_q); free(m->type_s); free(m->emb_ln_w); free(m->emb_ln_b);
  for (int i = 0; i < OR_LAYERS; i++) {
    or_layer* L = &m->layers[i];
    free_linear(&L->qkv); free_linear(&L->q_only); free_linear(&L->kv_only);
    free_linear(&L->attn_out); free_linear(&L->ffn_inter); free_linear(&L->ffn_out);
    free(L->ln1_w); free(L->ln1_b); free(L->ln2_w); free(L->ln2_b);
  }
  free(m);
}

int or_load_ae8(const char* path, or_model** out) {
  *out = NULL;
  FILE* f = fopen(path, "rb"); /* fs::read */
  if (!f) return OR_ERR_IO;
  fseek(f, 0, SEEK_END);
  long sz = ftell(f);
  fseek(f, 0, SEEK_SET);
  if (sz < 0) { fclose(f); return OR_ERR_IO; }
  uint8_t* buf = (uint8_t*)malloc(sz ? (size_t)sz : 1);
  if (sz && fread(buf, 1, (size_t)sz, f) != (size_t)sz) { fclose(f); free(buf); return OR_ERR_IO; }
  fclose(f);

  cursor_t c = {buf, (size_t)sz};
  or_model* m = (or_model*)calloc(1, sizeof(or_model));
  int rc = OR_OK;
  static const uint8_t magic[8] = {'A', 'R', 'C', 'T', 'I', 'C', '8', 0x01}; /* :20 */
  if (c.left < 8) { rc = OR_ERR_EOF; goto done; }
  if (memcmp(c.p, magic, 8) != 0) { rc = OR_ERR_INVALID_DATA; goto done; } /* :81-86 */
  c.p += 8; c.left -= 8;
  if ((rc = rd_i8_vec(&c, &m->word_q, &m->word_q_len))) goto done;
  if ((rc = rd_f32_vec(&c, &m->word_s, &m->word_s_len))) goto done;
  if ((rc = rd_i8_vec(&c, &m->pos_q, &m->pos_q_len))) goto done;
  if ((rc = rd_f32_vec(&c, &m->pos_s, &m->pos_s_len))) goto done;
  if ((rc = rd_i8_vec(&c, &m->type_q, &m->type_q_len))) goto done;
  if ((rc = rd_f32_vec(&c, &m->type_s, &m->type_s_len))) goto done;
  if ((rc = rd_f32_vec(&c, &m->emb_ln_w, &m->emb_ln_w_len))) goto done;
  if ((rc = rd_f32_vec(&c, &m->emb_ln_b, &m->emb_ln_b_len))) goto done;
  for (int i = 0; i < OR_LAYERS; i++) { /* :96-125 */
    or_layer* L = &m->layers[i];
    if ((rc = rd_linear(&c, &L->qkv))) goto done;
    if (c.left < 1) { rc = OR_ERR_EOF; goto done; }
    uint8_t split = c.p[0];
    c.p += 1; c.left -= 1;
    L->has_split = split == 1;
    if (L->has_split) {
      if ((rc = rd_linear(&c, &L->q_only))) goto done;
      if ((rc = rd_linear(&c, &L->kv_only))) goto done;
    }
    if ((rc = rd_linear(&c, &L->attn_out))) goto done;
    if ((rc = rd_f32_vec(&c, &L->ln1_w, &L->ln1_w_len))) goto done;
    if ((rc = rd_f32_vec(&c, &L->ln1_b, &L->ln1_b_len))) goto done;
    if ((rc = rd_linear(&c, &L->ffn_inter))) goto done;
    if ((rc = rd_linear(&c, &L->ffn_out))) goto done;
    if ((rc = rd_f32_vec(&c, &L->ln2_w, &L->ln2_w_len))) goto done;
    if ((rc = rd_f32_vec(&c, &L->ln2_b, &L->ln2_b_len))) goto done;
  }
  /* PackedModel::from_raw pre-dequantizes type row 0 (src/model.rs:50-54) */
  if (m->type_q_len >= OR_HIDDEN && m->type_s_len >= 1)
    for (int j = 0; j < OR_HIDDEN; j++) m->type0[j] = (float)m->type_q[j] * m->type_s[0];
done:
  free(buf);
  if (rc) { or_free(m); return rc; }
  *out = m;
  return OR_OK;
}

size_t or_size_bytes(const or_model* m) { /* src/quantize.rs:140-165 */
  size_t t = m->word_q_len + m->pos_q_len + m->type_q_len +
             (m->word_s_len + m->pos_s_len + m->type_s_len + m->emb_ln_w_len + m->emb_ln_b_len) * 4;
  for (int i = 0; i < OR_LAYERS; i++) {
    const or_layer* L = &m->layers[i];
    const or_linear* ls[4] = {&L->qkv, &L->attn_out, &L->ffn_inter, &L->ffn_out};
    for (int j = 0; j < 4; j++) t += ls[j]->w_len + (ls[j]->s_len + ls[j]->b_len + ls[j]->is_len) * 4;
    if (L->has_split) {
      const or_linear* ss[2] = {&L->q_only, &L->kv_only};
      for (int j = 0; j < 2; j++) t += ss[j]->w_len + (ss[j]->s_len + ss[j]->b_len + ss[j]->is_len) * 4;
    }
    t += (L->ln1_w_len + L->ln1_b_len + L->ln2_w_len + L->ln2_b_len) * 4;
  }
  return t;
}

/* ------------------------------------------------------------------------- */
/* scalar kernels                                                            */
/* ------------------------------------------------------------------------- */

/* `(v).round().clamp(-127.0, 127.0) as i8`: f32::round is half away from zero
   (roundf); `as i8` saturates and maps NaN to 0. */
static inline int8_t q_round_clamp(float v) {
  float r = roundf(v);
  if (r != r) return 0; /* clamp(NaN) = NaN; NaN as i8 = 0 */
  if (r < -127.0f) r = -127.0f;
  if (r > 127.0f) r = 127.0f;
  return (int8_t)r;
}

void or_gemm_acc(int m, int n, int k, const int8_t* a, const int8_t* w, int32_t* acc) {
  for (int r = 0; r < m; r++)
    for (int c = 0; c < n; c++) {
      int32_t s = 0;
      const int8_t* ar = a + (size_t)r * k;
      const int8_t* wr = w + (size_t)c * k;
      for (int i = 0; i < k; i++) s += (int32_t)ar[i] * (int32_t)wr[i];
      acc[(size_t)r * n + c] = s;
    }
}

void or_gemm(int m, const int8_t* a, const float* a_scale, const or_linear* w,
             const float* res, float* out) { /* gemm_scalar_fused, src/gemm.rs:2000-2029 */
  const int n_out = (int)w->n_out, k_in = (int)w->k_in;
  for (int r = 0; r < m; r++) {
    const int8_t* a_row = a + (size_t)r * k_in;
    const float s_r = a_scale[r];
    const size_t row_off = (size_t)r * n_out;
    for (int n = 0; n < n_out; n++) {
      const int8_t* w_row = w->w_q + (size_t)n * k_in;
      int32_t acc = 0;
      for (int k = 0; k < k_in; k++) acc += (int32_t)a_row[k] * (int32_t)w_row[k];
      float b_val = w->bias[n];
      if (res) b_val += res[row_off + n];
      /* (acc as f32).mul_add(s_r * w_scale[n], b_val) */
      out[row_off + n] = fmaf((float)acc, s_r * w->w_scale[n], b_val);
    }
  }
}

float or_ln_quant_row(float* x, const float* gamma, const float* beta, const float* inv_smooth,
                      int8_t* q, int n, float eps) { /* src/simd_math.rs:208-247 */
  float sum = 0.0f;
  for (int j = 0; j < n; j++) sum += x[j];
  const float mean = sum / (float)n;
  float var_sum = 0.0f;
  for (int j = 0; j < n; j++) {
    const float d = x[j] - mean;
    var_sum += d * d;
  }
  const float rstd = 1.0f / sqrtf(var_sum / (float)n + eps);
  float max_abs = 1e-8f;
  for (int j = 0; j < n; j++) {
    const float y = (x[j] - mean) * rstd * gamma[j] + beta[j];
    x[j] = y;
    const float a = fabsf(y * inv_smooth[j]);
    if (a > max_abs) max_abs = a;
  }
  const float scale = max_abs / 127.0f;
  const float inv_scale = 127.0f / max_abs;
  for (int j = 0; j < n; j++) q[j] = q_round_clamp(x[j] * inv_smooth[j] * inv_scale);
  return scale;
}

void or_ln_row(float* x, const float* gamma, const float* beta, int n, float eps) {
  /* layernorm_inplace_row, src/simd_math.rs:481-497 */
  float sum = 0.0f;
  for (int j = 0; j < n; j++) sum += x[j];
  const float mean = sum / (float)n;
  float var_sum = 0.0f;
  for (int j = 0; j < n; j++) {
    const float d = x[j] - mean;
    var_sum += d * d;
  }
  const float rstd = 1.0f / sqrtf(var_sum / (float)n + eps);
  for (int j = 0; j < n; j++) x[j] = (x[j] - mean) * rstd * gamma[j] + beta[j];
}

float or_smooth_quant_row(const float* x, const float* inv_smooth, int8_t* q, int n) {
  /* smooth_quantize_row scalar branch, src/simd_math.rs:513-530 */
  float max_abs = 1e-8f;
  for (int j = 0; j < n; j++) {
    const float a = fabsf(x[j] * inv_smooth[j]);
    if (a > max_abs) max_abs = a;
  }
  const float scale = max_abs / 127.0f;
  const float inv_scale = 127.0f / max_abs;
  for (int j = 0; j < n; j++) q[j] = q_round_clamp(x[j] * inv_smooth[j] * inv_scale);
  return scale;
}

float or_gelu(float x) { /* scalar_gelu, src/simd_math.rs:15-23 */
  const float z = fabsf(x) * 0.70710677f; /* std::f32::consts::FRAC_1_SQRT_2 */
  const float t = 1.0f / (1.0f + 0.3275911f * z);
  const float poly =
      t * (0.254829592f + t * (-0.284496736f + t * (1.421413741f + t * (-1.453152027f + t * 1.061405429f))));
  const float erf_val = copysignf(1.0f - poly * expf(-z * z), x);
  return 0.5f * x * (1.0f + erf_val);
}

void or_gelu_map(const float* x, float* y, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = or_gelu(x[i]);
}

float or_gelu_quant_row(float* x, const float* inv_smooth, int8_t* q, int n) {
  /* gelu_smooth_quantize_row scalar branch, src/simd_math.rs:1295-1312 */
  float max_abs = 1e-8f;
  for (int j = 0; j < n; j++) {
    const float g = or_gelu(x[j]) * inv_smooth[j];
    x[j] = g;
    const float a = fabsf(g);
    if (a > max_abs) max_abs = a;
  }
  const float scale = max_abs / 127.0f;
  const float inv_scale = 127.0f / max_abs;
  for (int j = 0; j < n; j++) q[j] = q_round_clamp(x[j] * inv_scale);
  return scale;
}

float or_dot32(const float* a, const float* b) { /* src/simd_math.rs:1461-1468 */
  float sum = 0.0f;
  for (int i = 0; i < 32; i++) sum += a[i] * b[i];
  return sum;
}

void or_scores(const float* q, const float* k_head, float scale, float* scores, int len) {
  for (int tk = 0; tk < len; tk++) scores[tk] = or_dot32(q, k_head + (size_t)tk * 32) * scale;
}

void or_softmax(float* s, int len) { /* src/simd_math.rs:1684-1702 */
  if (len == 0) return;
  float max_val = -INFINITY;
  for (int i = 0; i < len; i++)
    if (s[i] > max_val) max_val = s[i];
  float sum = 0.0f;
  for (int i = 0; i < len; i++) {
    const float e = expf(s[i] - max_val);
    s[i] = e;
    sum += e;
  }
  const float inv_sum = 1.0f / sum;
  for (int i = 0; i < len; i++) s[i] *= inv_sum;
}

void or_wsum(const float* p, const float* v_head, int len, float* out32) { /* :1812-1821 */
  for (int d = 0; d < 32; d++) out32[d] = 0.0f;
  for (int t = 0; t < len; t++) {
    const float* row = v_head + (size_t)t * 32;
    for (int d = 0; d < 32; d++) out32[d] += p[t] * row[d];
  }
}

void or_emb_row(const int8_t* w_row, float w_s, const int8_t* p_row, float p_s, const float* t_row,
                float* h_row, int n) { /* src/simd_math.rs:1877-1880 */
  for (int j = 0; j < n; j++) h_row[j] = (float)w_row[j] * w_s + (float)p_row[j] * p_s + t_row[j];
}

void or_l2(float* v, int n) { /* src/simd_math.rs:2892-2903 */
  float sum_sq = 0.0f;
  for (int i = 0; i < n; i++) sum_sq += v[i] * v[i];
  if (sum_sq > 0.0f) {
    const float inv_norm = 1.0f / sqrtf(sum_sq);
    for (int i = 0; i < n; i++) v[i] *= inv_norm;
  }
}

static void attention_head_k(const float* qkv, int len, int stride, int q_off, int k_off, int v_off,
                             float* ctx, int ctx_stride, const or_kernels* K) {
  /* src/model.rs:663-694 for one (segment, head): copy K/V head rows, then per query
     compute_scores_head32 -> softmax_inplace -> weighted_sum_head32 */
  float* kh = (float*)malloc((size_t)(len ? len : 1) * 32 * sizeof(float));
  float* vh = (float*)malloc((size_t)(len ? len : 1) * 32 * sizeof(float));
  float* sc = (float*)malloc((size_t)(len ? len : 1) * sizeof(float));
  const float inv_sqrt_d = 1.0f / sqrtf(32.0f); /* src/model.rs:590 */
  for (int t = 0; t < len; t++) {
    memcpy(kh + (size_t)t * 32, qkv + (size_t)t * stride + k_off, 32 * sizeof(float));
    memcpy(vh + (size_t)t * 32, qkv + (size_t)t * stride + v_off, 32 * sizeof(float));
  }
  for (int tq = 0; tq < len; tq++) {
    K->scores(qkv + (size_t)tq * stride + q_off, kh, inv_sqrt_d, sc, len);
    K->softmax(sc, len);
    K->wsum(sc, vh, len, ctx + (size_t)tq * ctx_stride);
  }
  free(kh); free(vh); free(sc);
}

const or_kernels or_scalar_kernels = {or_gemm, or_ln_quant_row, or_smooth_quant_row, or_gelu_quant_row,
                                      or_scores, or_softmax, or_wsum};

void or_attention_head(const float* qkv, int len, int stride, int q_off, int k_off, int v_off,
                       float* ctx, int ctx_stride) {
  attention_head_k(qkv, len, stride, q_off, k_off, v_off, ctx, ctx_stride, &or_scalar_kernels);
}

/* ------------------------------------------------------------------------- */
/* packed forward: embedding + layers 0..10 + layer 11 (src/model.rs:521-914) */
/* ------------------------------------------------------------------------- */

#define H OR_HIDDEN
#define I OR_INTER

typedef struct {
  int T, B;
  const int* seg_start; /* [B] */
  const int* seg_len;   /* [B] */
  int sme;              /* attention of the reference's ArmSme backend (or_attention_sme) */
  int pert_layer;       /* test hook: 1 + the layer whose input act_q gets pert_row/pert_col moved by one step */
  int pert_row, pert_col;
  float *hidden, *tmp, *qkv, *ctx, *inter;
  int8_t *act_q, *inter_q;
  float* act_scale;
} fwd_ws;

static void embed_tokens(const or_model* m, const uint16_t* const* seq_ids, fwd_ws* w, const or_kernels* K) {
  /* src/model.rs:549-586: local positions 0..len per segment */
  const float* first_inv_smooth = m->layers[0].qkv.inv_smooth;
  for (int b = 0; b < w->B; b++) {
    for (int lt = 0; lt < w->seg_len[b]; lt++) {
      const int gt = w->seg_start[b] + lt;
      const int tok = seq_ids[b][lt];
      float* h_row = w->hidden + (size_t)gt * H;
      or_emb_row(m->word_q + (size_t)tok * H, m->word_s[tok], m->pos_q + (size_t)lt * H,
                 m->pos_s[lt], m->type0, h_row, H);
      w->act_scale[gt] = K->ln_quant_row(h_row, m->emb_ln_w, m->emb_ln_b, first_inv_smooth,
                                         w->act_q + (size_t)gt * H, H, OR_LN_EPS);
    }
  }
}

static void swap_f(float** a, float** b) { float* t = *a; *a = *b; *b = t; }

static void full_layer(const or_model* m, int l, fwd_ws* w, int quant_next, const or_kernels* K) {
  /* one layer over all T rows: src/model.rs:593-767 */
  const or_layer* L = &m->layers[l];
  const int T = w->T;
  if (w->pert_layer == l + 1) { /* test hook: one int8 activation one step off */
    int8_t* q = &w->act_q[(size_t)w->pert_row * H + w->pert_col];
    *q = (int8_t)(*q < 127 ? *q + 1 : *q - 1);
  }
  K->gemm(T, w->act_q, w->act_scale, &L->qkv, NULL, w->qkv);
  if (w->sme) {
    /* each sequence as forward_cls computes it on the ArmSme backend
       (src/model.rs:244-259): the quantized attention over that sequence alone
       (its own V column scales) from 16 tokens on, the exact path below */
    for (int b = 0; b < w->B; b++) {
      const int s0 = w->seg_start[b], len = w->seg_len[b];
      if (len >= 16) {
        const int cu[2] = {0, len};
        or_attention_sme(w->qkv + (size_t)s0 * 3 * H, len, cu, 1, w->ctx + (size_t)s0 * H);
      } else {
        for (int h = 0; h < OR_HEADS; h++) {
          const int ho = h * 32;
          attention_head_k(w->qkv + (size_t)s0 * 3 * H, len, 3 * H, ho, H + ho, 2 * H + ho,
                           w->ctx + (size_t)s0 * H + ho, H, K);
        }
      }
    }
  } else {
    for (int b = 0; b < w->B; b++)
      for (int h = 0; h < OR_HEADS; h++) {
        const int ho = h * 32;
        attention_head_k(w->qkv + (size_t)w->seg_start[b] * 3 * H, w->seg_len[b], 3 * H, ho, H + ho,
                         2 * H + ho, w->ctx + (size_t)w->seg_start[b] * H + ho, H, K);
      }
  }
  for (int t = 0; t < T; t++)
    w->act_scale[t] = K->smooth_quant_row(w->ctx + (size_t)t * H, L->attn_out.inv_smooth,
                                          w->act_q + (size_t)t * H, H);
  K->gemm(T, w->act_q, w->act_scale, &L->attn_out, w->hidden, w->tmp);
  swap_f(&w->hidden, &w->tmp);
  for (int t = 0; t < T; t++)
    w->act_scale[t] = K->ln_quant_row(w->hidden + (size_t)t * H, L->ln1_w, L->ln1_b,
                                      L->ffn_inter.inv_smooth, w->act_q + (size_t)t * H, H, OR_LN_EPS);
  K->gemm(T, w->act_q, w->act_scale, &L->ffn_inter, NULL, w->inter);
  for (int t = 0; t < T; t++)
    w->act_scale[t] = K->gelu_quant_row(w->inter + (size_t)t * I, L->ffn_out.inv_smooth,
                                        w->inter_q + (size_t)t * I, I);
  K->gemm(T, w->inter_q, w->act_scale, &L->ffn_out, w->hidden, w->tmp);
  swap_f(&w->hidden, &w->tmp);
  if (quant_next) {
    const float* next_smooth = m->layers[l + 1].qkv.inv_smooth;
    for (int t = 0; t < T; t++)
      w->act_scale[t] = K->ln_quant_row(w->hidden + (size_t)t * H, L->ln2_w, L->ln2_b, next_smooth,
                                        w->act_q + (size_t)t * H, H, OR_LN_EPS);
  }
}

static void last_layer_pruned(const or_model* m, fwd_ws* w, float* out, const or_kernels* K) {
  /* src/model.rs:770-913 */
  const or_layer* L = &m->layers[OR_LAYERS - 1];
  const int T = w->T, B = w->B;
  float* kv = (float*)malloc((size_t)T * 2 * H * sizeof(float));
  K->gemm(T, w->act_q, w->act_scale, &L->kv_only, NULL, kv);
  /* compact CLS rows to 0..B (:787-800); forward order keeps it in-place safe */
  for (int b = 0; b < B; b++) {
    const int cls_t = w->seg_start[b];
    if (cls_t != b) {
      memmove(w->act_q + (size_t)b * H, w->act_q + (size_t)cls_t * H, H);
      w->act_scale[b] = w->act_scale[cls_t];
      memmove(w->hidden + (size_t)b * H, w->hidden + (size_t)cls_t * H, H * sizeof(float));
    }
  }
  float* q_cls = (float*)malloc((size_t)B * H * sizeof(float));
  K->gemm(B, w->act_q, w->act_scale, &L->q_only, NULL, q_cls);
  const float inv_sqrt_d = 1.0f / sqrtf(32.0f);
  float* kh = (float*)malloc((size_t)OR_MAX_POS * 32 * sizeof(float));
  float* vh = (float*)malloc((size_t)OR_MAX_POS * 32 * sizeof(float));
  float* sc = (float*)malloc((size_t)OR_MAX_POS * sizeof(float));
  for (int b = 0; b < B; b++) { /* :814-843 */
    const int s0 = w->seg_start[b], len = w->seg_len[b];
    for (int h = 0; h < OR_HEADS; h++) {
      const int ho = h * 32;
      for (int lt = 0; lt < len; lt++) {
        memcpy(kh + (size_t)lt * 32, kv + (size_t)(s0 + lt) * 2 * H + ho, 32 * sizeof(float));
        memcpy(vh + (size_t)lt * 32, kv + (size_t)(s0 + lt) * 2 * H + H + ho, 32 * sizeof(float));
      }
      K->scores(q_cls + (size_t)b * H + ho, kh, inv_sqrt_d, sc, len);
      K->softmax(sc, len);
      K->wsum(sc, vh, len, w->ctx + (size_t)b * H + ho);
    }
  }
  for (int b = 0; b < B; b++) /* :846-852 */
    w->act_scale[b] = K->smooth_quant_row(w->ctx + (size_t)b * H, L->attn_out.inv_smooth,
                                          w->act_q + (size_t)b * H, H);
  K->gemm(B, w->act_q, w->act_scale, &L->attn_out, w->hidden, w->tmp);
  for (int b = 0; b < B; b++)
    w->act_scale[b] = K->ln_quant_row(w->tmp + (size_t)b * H, L->ln1_w, L->ln1_b,
                                      L->ffn_inter.inv_smooth, w->act_q + (size_t)b * H, H, OR_LN_EPS);
  K->gemm(B, w->act_q, w->act_scale, &L->ffn_inter, NULL, w->inter);
  for (int b = 0; b < B; b++)
    w->act_scale[b] = K->gelu_quant_row(w->inter + (size_t)b * I, L->ffn_out.inv_smooth,
                                        w->inter_q + (size_t)b * I, I);
  K->gemm(B, w->inter_q, w->act_scale, &L->ffn_out, w->tmp, w->hidden);
  for (int b = 0; b < B; b++) {
    float* row = w->hidden + (size_t)b * H;
    or_ln_row(row, L->ln2_w, L->ln2_b, H, OR_LN_EPS);
    or_l2(row, H);
    memcpy(out + (size_t)b * H, row, H * sizeof(float));
  }
  free(kv); free(q_cls); free(kh); free(vh); free(sc);
}

static int fwd_alloc(fwd_ws* w, int T) {
  size_t t = (size_t)(T > 0 ? T : 1);
  w->hidden = (float*)malloc(t * H * 4);
  w->tmp = (float*)malloc(t * H * 4);
  w->qkv = (float*)malloc(t * 3 * H * 4);
  w->ctx = (float*)malloc(t * H * 4);
  w->inter = (float*)malloc(t * I * 4);
  w->act_q = (int8_t*)malloc(t * H);
  w->inter_q = (int8_t*)malloc(t * I);
  w->act_scale = (float*)malloc(t * 4);
  return (w->hidden && w->tmp && w->qkv && w->ctx && w->inter && w->act_q && w->inter_q && w->act_scale)
             ? OR_OK : OR_ERR_ARG;
}

static void fwd_free(fwd_ws* w) {
  free(w->hidden); free(w->tmp); free(w->qkv); free(w->ctx); free(w->inter);
  free(w->act_q); free(w->inter_q); free(w->act_scale);
}

/* runs one packed batch of B segments (already truncated) */
typedef struct {
  int sme;                       /* fwd_ws.sme */
  int pert_layer, pert_row, pert_col; /* fwd_ws.pert_* */
} fwd_opts;

static int forward_packed_k(const or_model* m, const uint16_t* const* seq_ids, const int* lens, int B,
                            int prune, float* out, const or_kernels* K, const fwd_opts* o) {
  int* starts = (int*)malloc(sizeof(int) * (B > 0 ? B : 1));
  int T = 0;
  for (int b = 0; b < B; b++) {
    if (lens[b] < 1 || lens[b] > OR_MAX_POS) { free(starts); return OR_ERR_ARG; }
    for (int t = 0; t < lens[b]; t++)
      if (seq_ids[b][t] >= m->word_s_len) { free(starts); return OR_ERR_ARG; }
    starts[b] = T;
    T += lens[b];
  }
  fwd_ws w = {0};
  w.T = T; w.B = B; w.seg_start = starts; w.seg_len = lens;
  if (o) {
    w.sme = o->sme;
    w.pert_layer = o->pert_layer;
    w.pert_row = o->pert_row;
    w.pert_col = o->pert_col;
  }
  if (fwd_alloc(&w, T)) { fwd_free(&w); free(starts); return OR_ERR_ARG; }
  embed_tokens(m, seq_ids, &w, K);
  for (int l = 0; l < OR_LAYERS - 1; l++) full_layer(m, l, &w, 1, K);
  if (prune) {
    last_layer_pruned(m, &w, out, K);
  } else {
    /* unpruned layer 11: the full QKV of layer 11 is q_only rows ++ kv_only rows */
    const or_layer* L = &m->layers[OR_LAYERS - 1];
    or_linear full = {0};
    full.n_out = 3 * H; full.k_in = H;
    full.w_q = (int8_t*)malloc(3 * H * H);
    full.w_scale = (float*)malloc(3 * H * 4);
    full.bias = (float*)malloc(3 * H * 4);
    memcpy(full.w_q, L->q_only.w_q, (size_t)H * H);
    memcpy(full.w_q + (size_t)H * H, L->kv_only.w_q, (size_t)2 * H * H);
    memcpy(full.w_scale, L->q_only.w_scale, H * 4);
    memcpy(full.w_scale + H, L->kv_only.w_scale, 2 * H * 4);
    memcpy(full.bias, L->q_only.bias, H * 4);
    memcpy(full.bias + H, L->kv_only.bias, 2 * H * 4);
    or_model m2;
    memcpy(&m2, m, sizeof(or_model));
    m2.layers[OR_LAYERS - 1].qkv.n_out = 3 * H;
    m2.layers[OR_LAYERS - 1].qkv.w_q = full.w_q;
    m2.layers[OR_LAYERS - 1].qkv.w_scale = full.w_scale;
    m2.layers[OR_LAYERS - 1].qkv.bias = full.bias;
    full_layer(&m2, OR_LAYERS - 1, &w, 0, K);
    for (int b = 0; b < B; b++) {
      float* row = w.hidden + (size_t)starts[b] * H;
      or_ln_row(row, L->ln2_w, L->ln2_b, H, OR_LN_EPS);
      or_l2(row, H);
      memcpy(out + (size_t)b * H, row, H * sizeof(float));
    }
    free(full.w_q); free(full.w_scale); free(full.bias);
  }
  fwd_free(&w);
  free(starts);
  return OR_OK;
}

static int forward_packed(const or_model* m, const uint16_t* const* seq_ids, const int* lens, int B,
                          int prune, float* out) {
  return forward_packed_k(m, seq_ids, lens, B, prune, out, &or_scalar_kernels, NULL);
}

static int forward_cls_k(const or_model* m, const uint16_t* ids, size_t n, float* out384, const or_kernels* K) {
  /* src/model.rs:191-192: seq_len = min(len, 512); empty input is rejected */
  int len = (int)(n < OR_MAX_POS ? n : OR_MAX_POS);
  if (len < 1) return OR_ERR_ARG;
  return forward_packed_k(m, &ids, &len, 1, 1, out384, K, NULL);
}

int or_forward_cls(const or_model* m, const uint16_t* ids, size_t n, float* out384) {
  return forward_cls_k(m, ids, n, out384, &or_scalar_kernels);
}

int or_forward_cls_unpruned(const or_model* m, const uint16_t* ids, size_t n, float* out384) {
  int len = (int)(n < OR_MAX_POS ? n : OR_MAX_POS);
  if (len < 1) return OR_ERR_ARG;
  return forward_packed(m, &ids, &len, 1, 0, out384);
}

static int forward_ragged_cls_k(const or_model* m, const uint16_t* ids, const uint32_t* offsets, int b,
                                float* out, const or_kernels* K) {
  if (b == 0) return OR_OK; /* src/model.rs:529-531 */
  if (b == 1) return forward_cls_k(m, ids + offsets[0], offsets[1] - offsets[0], out, K);
  if (b > 64) return OR_ERR_ARG; /* :540-543 */
  const uint16_t* seqs[64];
  int lens[64];
  int cursor = 0;
  for (int i = 0; i < b; i++) { /* :550: s_len = min(len, MAX_POSITIONS - cursor) */
    int len = (int)(offsets[i + 1] - offsets[i]);
    int room = OR_MAX_POS - cursor;
    lens[i] = len < room ? len : room;
    if (lens[i] < 1) return OR_ERR_ARG; /* :551 */
    seqs[i] = ids + offsets[i];
    cursor += lens[i];
  }
  return forward_packed_k(m, seqs, lens, b, 1, out, K, NULL);
}

int or_forward_ragged_cls(const or_model* m, const uint16_t* ids, const uint32_t* offsets, int b,
                          float* out) {
  return forward_ragged_cls_k(m, ids, offsets, b, out, &or_scalar_kernels);
}

static int run_prefix(const or_model* m, const uint16_t* ids, const uint32_t* offsets, int b, int upto_layer,
                      float* hidden, int8_t* act_q, float* act_scale, int sme);

int or_run_prefix(const or_model* m, const uint16_t* ids, const uint32_t* offsets, int b,
                  int upto_layer, float* hidden, int8_t* act_q, float* act_scale) {
  return run_prefix(m, ids, offsets, b, upto_layer, hidden, act_q, act_scale, 0);
}

int or_run_prefix_sme(const or_model* m, const uint16_t* ids, const uint32_t* offsets, int b,
                      int upto_layer, float* hidden, int8_t* act_q, float* act_scale) {
  return run_prefix(m, ids, offsets, b, upto_layer, hidden, act_q, act_scale, 1);
}

int or_forward_cls_perturbed(const or_model* m, const uint16_t* ids, size_t n, int layer, int row, int col,
                             float* out384) {
  /* forward_cls with act_q[row][col] one step off (+1, or -1 at 127) at the
     input of encoder layer `layer`: the sensitivity of the model to one int8
     activation */
  const int len = (int)(n > OR_MAX_POS ? OR_MAX_POS : n);
  if (len < 1 || layer < 0 || layer > OR_LAYERS - 2 || row < 0 || row >= len || col < 0 || col >= H) return OR_ERR_ARG;
  const fwd_opts o = {0, layer + 1, row, col};
  return forward_packed_k(m, &ids, &len, 1, 1, out384, &or_scalar_kernels, &o);
}

int or_embed_tokens_sme(const or_model* m, const uint16_t* ids, const uint32_t* offsets, int b, float* out) {
  /* forward_cls (src/model.rs:185-513) of each sequence on the ArmSme backend,
     run as one packed batch: every layer acts per sequence (full_layer's sme
     branch), so each output equals that sequence's own forward_cls */
  if (b < 1) return OR_ERR_ARG;
  const uint16_t** seqs = (const uint16_t**)malloc(sizeof(void*) * b);
  int* lens = (int*)malloc(sizeof(int) * b);
  for (int i = 0; i < b; i++) {
    int len = (int)(offsets[i + 1] - offsets[i]);
    lens[i] = len > OR_MAX_POS ? OR_MAX_POS : len; /* src/model.rs:191 */
    seqs[i] = ids + offsets[i];
  }
  const fwd_opts o = {1, 0, 0, 0};
  const int rc = forward_packed_k(m, seqs, lens, b, 1, out, &or_scalar_kernels, &o);
  free(seqs);
  free(lens);
  return rc;
}

static int run_prefix(const or_model* m, const uint16_t* ids, const uint32_t* offsets, int b, int upto_layer,
                      float* hidden, int8_t* act_q, float* act_scale, int sme) {
  if (b < 1 || upto_layer < 0 || upto_layer > OR_LAYERS - 1) return OR_ERR_ARG;
  const uint16_t** seqs = (const uint16_t**)malloc(sizeof(void*) * b);
  int* lens = (int*)malloc(sizeof(int) * b);
  int* starts = (int*)malloc(sizeof(int) * b);
  int T = 0;
  for (int i = 0; i < b; i++) {
    int len = (int)(offsets[i + 1] - offsets[i]);
    if (len > OR_MAX_POS) len = OR_MAX_POS;
    if (len < 1) { free(seqs); free(lens); free(starts); return OR_ERR_ARG; }
    seqs[i] = ids + offsets[i];
    lens[i] = len;
    starts[i] = T;
    T += len;
  }
  fwd_ws w = {0};
  w.T = T; w.B = b; w.seg_start = starts; w.seg_len = lens; w.sme = sme;
  fwd_alloc(&w, T);
  embed_tokens(m, seqs, &w, &or_scalar_kernels);
  for (int l = 0; l < upto_layer; l++) full_layer(m, l, &w, 1, &or_scalar_kernels);
  memcpy(hidden, w.hidden, (size_t)T * H * 4);
  memcpy(act_q, w.act_q, (size_t)T * H);
  memcpy(act_scale, w.act_scale, (size_t)T * 4);
  fwd_free(&w);
  free(seqs); free(lens); free(starts);
  return OR_OK;
}

/* ------------------------------------------------------------------------- */
/* embed_batch scheduling: src/lib.rs:138-260 over pre-tokenized ids          */
/* ------------------------------------------------------------------------- */

typedef struct {
  const or_model* m;
  const uint16_t* ids;
  const uint32_t* offsets;
  size_t n;
  float* out;
  const or_kernels* k;
  atomic_size_t next;
  atomic_int err;
} batch_job;

static int run_single(batch_job* j, size_t idx) {
  return forward_cls_k(j->m, j->ids + j->offsets[idx], j->offsets[idx + 1] - j->offsets[idx],
                       j->out + idx * H, j->k);
}

static void* batch_worker(void* arg) {
  batch_job* j = (batch_job*)arg;
  const size_t MAX_PACK_TOKENS = 32;
  for (;;) {
    size_t idx0 = atomic_fetch_add(&j->next, 1);
    if (idx0 >= j->n) break;
    size_t len0 = j->offsets[idx0 + 1] - j->offsets[idx0];
    if (len0 >= 16) { /* :172-180 */
      int rc = run_single(j, idx0);
      if (rc) atomic_store(&j->err, rc);
      continue;
    }
    size_t idxs[4] = {idx0, 0, 0, 0};
    size_t pack_count = 1, pack_tokens = len0;
    while (pack_count < 4 && pack_tokens + 12 <= MAX_PACK_TOKENS) { /* :187-212 */
      size_t ni = atomic_fetch_add(&j->next, 1);
      if (ni >= j->n) break;
      size_t ln = j->offsets[ni + 1] - j->offsets[ni];
      if (pack_tokens + ln <= MAX_PACK_TOKENS) {
        idxs[pack_count++] = ni;
        pack_tokens += ln;
      } else {
        int rc = run_single(j, ni);
        if (rc) atomic_store(&j->err, rc);
        break;
      }
    }
    if (pack_count == 1) {
      int rc = run_single(j, idx0);
      if (rc) atomic_store(&j->err, rc);
    } else { /* :221-238 */
      uint16_t buf[32];
      uint32_t offs[5];
      offs[0] = 0;
      for (size_t k = 0; k < pack_count; k++) {
        size_t ln = j->offsets[idxs[k] + 1] - j->offsets[idxs[k]];
        memcpy(buf + offs[k], j->ids + j->offsets[idxs[k]], ln * sizeof(uint16_t));
        offs[k + 1] = offs[k] + (uint32_t)ln;
      }
      float staging[4 * H];
      int rc = forward_ragged_cls_k(j->m, buf, offs, (int)pack_count, staging, j->k);
      if (rc) atomic_store(&j->err, rc);
      for (size_t k = 0; k < pack_count; k++)
        memcpy(j->out + idxs[k] * H, staging + k * H, H * sizeof(float));
    }
  }
  return NULL;
}

int or_embed_batch_tokens(const or_model* m, const uint16_t* ids, const uint32_t* offsets, size_t n,
                          int num_threads, float* out) {
  return or_embed_batch_tokens_k(m, ids, offsets, n, num_threads, out, &or_scalar_kernels);
}

int or_embed_batch_tokens_k(const or_model* m, const uint16_t* ids, const uint32_t* offsets, size_t n,
                            int num_threads, float* out, const or_kernels* k) {
  if (n == 0) return OR_OK; /* :145-147 */
  size_t threads = num_threads < 1 ? 1 : (size_t)num_threads;
  if (threads > n) threads = n;
  batch_job j;
  j.m = m; j.ids = ids; j.offsets = offsets; j.n = n; j.out = out; j.k = k;
  atomic_init(&j.next, 0);
  atomic_init(&j.err, 0);
  if (threads == 1) {
    batch_worker(&j);
  } else {
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * threads);
    for (size_t i = 0; i < threads; i++) pthread_create(&th[i], NULL, batch_worker, &j);
    for (size_t i = 0; i < threads; i++) pthread_join(th[i], NULL);
    free(th);
  }
  return atomic_load(&j.err);
}


/* ===========================================================================
 * Quantized (ArmSme backend) attention, src/simd_math.rs:1933-2192 with the
 * helpers it calls; see oracle.h.  NEON semantics restated per lane:
 * vcvtnq_s32_f32 = round to nearest, ties to even (rintf in the default
 * rounding mode), saturating to int32; vqmovn = saturating narrow; vfmaq_f32(a,
 * b, c) = fmaf(b, c, a); vcvtmq_s32_f32 = floor to int32.
 * ======================================================================== */
static int32_t cvtn_s32(float x) {
  if (x != x) return 0;
  const float r = rintf(x);
  if (r >= 2147483648.0f) return INT32_MAX;
  if (r < -2147483648.0f) return INT32_MIN;
  return (int32_t)r;
}
static int8_t sat_s8(int32_t v) { return (int8_t)(v > 127 ? 127 : (v < -128 ? -128 : v)); }
static float fmax_nn(float a, float b) { return b > a ? b : a; } /* vmaxq on non-NaN data */

int32_t or_exp2_q(float x, float scale, float x_min) {
  /* src/simd_math.rs:2353-2370 */
  x = x > x_min ? x : x_min; /* vmaxq_f32(x, x_min) */
  const int32_t n = (int32_t)floorf(x);
  const float f = x - (float)n;
  float p = fmaf(f, 0.07842169f * scale, 0.22511937f * scale);
  p = fmaf(f, p, 0.6963853f * scale);
  p = fmaf(f, p, 0.999857f * scale);
  uint32_t bits;
  memcpy(&bits, &p, 4);
  bits = (uint32_t)((int32_t)bits + (int32_t)((uint32_t)n << 23));
  float scaled;
  memcpy(&scaled, &bits, 4);
  return cvtn_s32(scaled);
}

/* quantize_head32_row_neon (src/simd_math.rs:2482-2526): int8 row, returns the scale */
static float sme_quant_row32(const float* src, float out_scale_mul, int8_t* q) {
  float m = 0.0f;
  for (int i = 0; i < 32; i++) m = fmax_nn(m, fabsf(src[i]));
  const float max_abs = m > 1e-8f ? m : 1e-8f; /* f32::max(1e-8) */
  const float inv_s = 127.0f / max_abs;
  for (int i = 0; i < 32; i++) q[i] = sat_s8(cvtn_s32(src[i] * inv_s));
  return (max_abs / 127.0f) * out_scale_mul;
}

void or_attention_sme(const float* qkv, int T, const int* cu, int B, float* ctx) {
  const int HID = 384, STR = 3 * 384;
  const float inv_sqrt_d = 1.0f / sqrtf(32.0f);
  const float k_scale_mul = inv_sqrt_d * 1.44269504088896340736f; /* inv_sqrt_d * LOG2_E in f32 */
  const float p_q16_max = 16383.0f;
  int8_t* qi = (int8_t*)malloc((size_t)T * 32);
  int8_t* ki = (int8_t*)malloc((size_t)T * 32);
  int8_t* vi = (int8_t*)malloc((size_t)T * 32);
  float* qs = (float*)malloc((size_t)T * 4);
  float* ks = (float*)malloc((size_t)T * 4);
  float* srow = (float*)malloc((size_t)T * 4);
  int32_t* prow = (int32_t*)malloc((size_t)T * 4);
  int* seg = (int*)malloc((size_t)T * sizeof(int));
  for (int b = 0; b < B; b++)
    for (int t = cu[b]; t < cu[b + 1]; t++) seg[t] = b;
  for (int h = 0; h < 12; h++) {
    const int ho = h * 32;
    /* V: per-column max over all T tokens, scales, int8 (pack_qkv_head_int8_neon step 1) */
    float vm[32], vscale[32], vinv[32];
    for (int c = 0; c < 32; c++) vm[c] = 1e-8f;
    for (int t = 0; t < T; t++)
      for (int c = 0; c < 32; c++) vm[c] = fmax_nn(vm[c], fabsf(qkv[(size_t)t * STR + 2 * HID + ho + c]));
    for (int c = 0; c < 32; c++) {
      vscale[c] = vm[c] * (1.0f / 127.0f);
      vinv[c] = 127.0f / vm[c];
    }
    for (int t = 0; t < T; t++)
      for (int c = 0; c < 32; c++) vi[(size_t)t * 32 + c] = sat_s8(cvtn_s32(qkv[(size_t)t * STR + 2 * HID + ho + c] * vinv[c]));
    /* Q, K: per-token int8 (step 2) */
    for (int t = 0; t < T; t++) {
      qs[t] = sme_quant_row32(qkv + (size_t)t * STR + ho, 1.0f, qi + (size_t)t * 32);
      ks[t] = sme_quant_row32(qkv + (size_t)t * STR + HID + ho, k_scale_mul, ki + (size_t)t * 32);
    }
    for (int r = 0; r < T; r++) {
      const int s0 = cu[seg[r]], s1 = cu[seg[r] + 1], len = s1 - s0;
      /* raw scores and their dequantization: s = (f32(acc) * k_scale) * q_scale, log2 units */
      float mx = -INFINITY;
      const int nv = len & ~7; /* the NEON loop's 8-aligned part */
      for (int j = 0; j < len; j++) {
        int32_t acc = 0;
        for (int i = 0; i < 32; i++) acc += (int32_t)qi[(size_t)r * 32 + i] * (int32_t)ki[(size_t)(s0 + j) * 32 + i];
        const float v = ((float)acc * ks[s0 + j]) * qs[r];
        srow[j] = v;
        if (j < nv) mx = fmax_nn(mx, v);
      }
      for (int j = nv; j < len; j++)
        if (srow[j] > mx) mx = srow[j];
      /* exact-range int16 quantization and its integer sum */
      int32_t isum = 0;
      for (int j = 0; j < len; j++) {
        int32_t q;
        if (j < nv) {
          q = or_exp2_q(srow[j] - mx, p_q16_max, -16.0f);
        } else { /* ((s - max).exp2() * 16383).round() as i32, clamped */
          const float e = roundf(exp2f(srow[j] - mx) * p_q16_max);
          q = e != e ? 0 : (e >= 2147483648.0f ? INT32_MAX : (e < -2147483648.0f ? INT32_MIN : (int32_t)e));
          q = q < 0 ? 0 : (q > 16383 ? 16383 : q);
        }
        isum += q;
        prow[j] = q > 32767 ? 32767 : (q < -32768 ? -32768 : q); /* vqmovn to the i16 row */
      }
      const float p_scale = 1.0f / (float)(isum > 1 ? isum : 1);
      for (int c = 0; c < 32; c++) {
        int32_t acc = 0;
        for (int j = 0; j < len; j++) acc += prow[j] * (int32_t)vi[(size_t)(s0 + j) * 32 + c];
        ctx[(size_t)r * HID + ho + c] = (float)acc * (vscale[c] * p_scale);
      }
    }
  }
  free(qi); free(ki); free(vi); free(qs); free(ks); free(srow); free(prow); free(seg);
}
