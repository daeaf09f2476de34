/*
 * x86.c -- the reference's x86 backend (AVX-VNNI / AVX2+FMA), restated in C for
 * the CPU baseline of bench.py.
 *
 * TEST INFRASTRUCTURE ONLY (like oracle.c): it is timed beside the GPU as the
 * reference's best x86 path; it is not the parity oracle (its row and attention
 * kernels round differently from the scalar path, exactly as the reference's
 * do).  Each kernel restates the reference item cited beside it; the forward
 * and embed_batch drivers are oracle.c's, called through or_kernels.
 *
 * Backend choice follows SimdBackend::detect (src/gemm.rs:100-125): AVX2 and
 * FMA required; AVX-VNNI (the VEX form, CPUID.(7,1):EAX[4]) selects the VNNI
 * GEMM, AVX-512-VNNI alone does not.  Functions carry their own target
 * attributes, so nothing here runs an instruction the host lacks.
 */
#include <cpuid.h>
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define H OR_HIDDEN

/* 0: neither (scalar), 1: AVX2+FMA, 2: AVX-VNNI */
int or_x86_backend(void) {
  unsigned a, b, c, d;
  if (!__get_cpuid_count(1, 0, &a, &b, &c, &d)) return 0;
  const int fma = (c >> 12) & 1, osxsave = (c >> 27) & 1, avx = (c >> 28) & 1;
  if (!(fma && osxsave && avx)) return 0;
  if (!__get_cpuid_count(7, 0, &a, &b, &c, &d)) return 0;
  const int avx2 = (b >> 5) & 1;
  if (!avx2) return 0;
  if (__get_cpuid_count(7, 1, &a, &b, &c, &d) && ((a >> 4) & 1)) return 2;
  return 1;
}

/* ---- weights: pack_weights_x86 (src/gemm.rs:456-476) + col_sum_comp (:214-224) ---- */
static int pack_linear(or_linear* l, int vnni) {
  if (l->n_out == 0 || l->xpack) return OR_OK;
  const int n = (int)l->n_out, k = (int)l->k_in;
  if (n % 16 || k % 4) return OR_ERR_ARG;
  l->xpack = (int8_t*)aligned_alloc(64, ((size_t)n * k + 63) / 64 * 64);
  if (!l->xpack) return OR_ERR_ARG;
  /* [N/16 panels][K/4 steps][2 groups of 8 columns][4 k bytes] */
  size_t o = 0;
  for (int nb = 0; nb < n / 16; nb++)
    for (int ks = 0; ks < k / 4; ks++)
      for (int col = nb * 16; col < nb * 16 + 16; col++, o += 4)
        memcpy(l->xpack + o, l->w_q + (size_t)col * k + ks * 4, 4);
  if (vnni) {
    l->xcomp = (int32_t*)malloc(sizeof(int32_t) * n);
    if (!l->xcomp) return OR_ERR_ARG;
    for (int col = 0; col < n; col++) {
      int32_t s = 0;
      for (int j = 0; j < k; j++) s += l->w_q[(size_t)col * k + j];
      l->xcomp[col] = -128 * s;
    }
  }
  return OR_OK;
}

int or_x86_prepare(or_model* m) {
  const int be = or_x86_backend();
  if (be == 0) return OR_ERR_ARG;
  for (int i = 0; i < OR_LAYERS; i++) {
    or_layer* L = &m->layers[i];
    or_linear* ls[6] = {&L->qkv, &L->q_only, &L->kv_only, &L->attn_out, &L->ffn_inter, &L->ffn_out};
    for (int j = 0; j < 6; j++)
      if (ls[j]->w_q && pack_linear(ls[j], be == 2)) return OR_ERR_ARG;
  }
  return OR_OK;
}

/* ---- horizontal reductions (src/simd_math.rs hsum256_ps / hmax256_ps) ---- */
__attribute__((target("avx2"))) static inline float hsum256(__m256 v) {
  __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  s = _mm_add_ps(s, _mm_movehdup_ps(s));
  return _mm_cvtss_f32(_mm_add_ss(s, _mm_movehl_ps(s, s)));
}
__attribute__((target("avx2"))) static inline float hmax256(__m256 v) {
  __m128 s = _mm_max_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  s = _mm_max_ps(s, _mm_movehdup_ps(s));
  return _mm_cvtss_f32(_mm_max_ss(s, _mm_movehl_ps(s, s)));
}

/* ---- GEMMs ---------------------------------------------------------------
 * Both are exact in int32 (u8*s8 pairs stay below the i16 saturation limit), and
 * the epilogue fma(f32(acc), sa*ws, bias+res) matches gemm_scalar_fused. */

/* gemm_x86_avx2_fused (src/gemm.rs:1717-1908): |a| * sign(w, a) via maddubs,
 * 4 rows x 16 columns per inner block */
__attribute__((target("avx2,fma"))) static void gemm_avx2(int m, const int8_t* a, const float* a_scale,
                                                         const or_linear* w, const float* res, float* out) {
  const int n = (int)w->n_out, k = (int)w->k_in, ksteps = k / 4;
  const __m256i ones = _mm256_set1_epi16(1);
  for (int nb = 0; nb < n / 16; nb++) {
    const int col = nb * 16;
    const int8_t* panel = w->xpack + (size_t)nb * ksteps * 64;
    const __m256 ws0 = _mm256_loadu_ps(w->w_scale + col), ws1 = _mm256_loadu_ps(w->w_scale + col + 8);
    const __m256 bi0 = _mm256_loadu_ps(w->bias + col), bi1 = _mm256_loadu_ps(w->bias + col + 8);
    int r = 0;
    for (; r < m; r += 4) {
      const int rows = m - r < 4 ? m - r : 4;
      __m256i c[4][2];
      for (int i = 0; i < 4; i++) c[i][0] = c[i][1] = _mm256_setzero_si256();
      const int8_t* pb = panel;
      for (int ks = 0; ks < ksteps; ks++, pb += 64) {
        const __m256i b0 = _mm256_loadu_si256((const __m256i*)pb);
        const __m256i b1 = _mm256_loadu_si256((const __m256i*)(pb + 32));
        for (int i = 0; i < rows; i++) {
          int32_t a4;
          memcpy(&a4, a + (size_t)(r + i) * k + ks * 4, 4);
          const __m256i va = _mm256_set1_epi32(a4);
          const __m256i vabs = _mm256_abs_epi8(va);
          c[i][0] = _mm256_add_epi32(c[i][0], _mm256_madd_epi16(_mm256_maddubs_epi16(vabs, _mm256_sign_epi8(b0, va)), ones));
          c[i][1] = _mm256_add_epi32(c[i][1], _mm256_madd_epi16(_mm256_maddubs_epi16(vabs, _mm256_sign_epi8(b1, va)), ones));
        }
      }
      for (int i = 0; i < rows; i++) {
        const __m256 s = _mm256_set1_ps(a_scale[r + i]);
        const size_t off = (size_t)(r + i) * n + col;
        __m256 b0 = bi0, b1 = bi1;
        if (res) {
          b0 = _mm256_add_ps(b0, _mm256_loadu_ps(res + off));
          b1 = _mm256_add_ps(b1, _mm256_loadu_ps(res + off + 8));
        }
        _mm256_storeu_ps(out + off, _mm256_fmadd_ps(_mm256_cvtepi32_ps(c[i][0]), _mm256_mul_ps(s, ws0), b0));
        _mm256_storeu_ps(out + off + 8, _mm256_fmadd_ps(_mm256_cvtepi32_ps(c[i][1]), _mm256_mul_ps(s, ws1), b1));
      }
    }
  }
}

/* gemm_x86_avx_vnni_fused (src/gemm.rs:1911-1998): A shifted to u8 (x ^ 0x80),
 * vpdpbusd from the -128*colsum correction, row by row */
__attribute__((target("avx2,fma,avxvnni"))) static void gemm_vnni(int m, const int8_t* a, const float* a_scale,
                                                                 const or_linear* w, const float* res, float* out) {
  const int n = (int)w->n_out, k = (int)w->k_in, ksteps = k / 4;
  uint8_t* au = (uint8_t*)malloc((size_t)m * k);
  for (size_t i = 0; i < (size_t)m * k; i++) au[i] = (uint8_t)a[i] ^ 0x80u;
  for (int r = 0; r < m; r++) {
    const __m256 s = _mm256_set1_ps(a_scale[r]);
    const uint8_t* arow = au + (size_t)r * k;
    for (int nb = 0; nb < n / 16; nb++) {
      const int col = nb * 16;
      const int8_t* pb = w->xpack + (size_t)nb * ksteps * 64;
      __m256i c0 = _mm256_loadu_si256((const __m256i*)(w->xcomp + col));
      __m256i c1 = _mm256_loadu_si256((const __m256i*)(w->xcomp + col + 8));
      for (int ks = 0; ks < ksteps; ks++, pb += 64) {
        int32_t a4;
        memcpy(&a4, arow + ks * 4, 4);
        const __m256i va = _mm256_set1_epi32(a4);
        c0 = _mm256_dpbusd_avx_epi32(c0, va, _mm256_loadu_si256((const __m256i*)pb));
        c1 = _mm256_dpbusd_avx_epi32(c1, va, _mm256_loadu_si256((const __m256i*)(pb + 32)));
      }
      const size_t off = (size_t)r * n + col;
      const __m256 ws0 = _mm256_mul_ps(s, _mm256_loadu_ps(w->w_scale + col));
      const __m256 ws1 = _mm256_mul_ps(s, _mm256_loadu_ps(w->w_scale + col + 8));
      __m256 b0 = _mm256_loadu_ps(w->bias + col), b1 = _mm256_loadu_ps(w->bias + col + 8);
      if (res) {
        b0 = _mm256_add_ps(b0, _mm256_loadu_ps(res + off));
        b1 = _mm256_add_ps(b1, _mm256_loadu_ps(res + off + 8));
      }
      _mm256_storeu_ps(out + off, _mm256_fmadd_ps(_mm256_cvtepi32_ps(c0), ws0, b0));
      _mm256_storeu_ps(out + off + 8, _mm256_fmadd_ps(_mm256_cvtepi32_ps(c1), ws1, b1));
    }
  }
  free(au);
}

/* ---- row kernels ---------------------------------------------------------- */
/* 16 floats -> 16 int8 with cvtps (round to nearest even) after the clamp, as the
 * reference's AVX2 quantizers pack them */
__attribute__((target("avx2"))) static inline void store_q16(int8_t* q, __m256 v0, __m256 v1) {
  const __m256 lo = _mm256_set1_ps(-127.0f), hi = _mm256_set1_ps(127.0f);
  v0 = _mm256_min_ps(_mm256_max_ps(v0, lo), hi);
  v1 = _mm256_min_ps(_mm256_max_ps(v1, lo), hi);
  const __m256i q16 = _mm256_permute4x64_epi64(_mm256_packs_epi32(_mm256_cvtps_epi32(v0), _mm256_cvtps_epi32(v1)), 0xD8);
  _mm_storeu_si128((__m128i*)q, _mm_packs_epi16(_mm256_castsi256_si128(q16), _mm256_extracti128_si256(q16, 1)));
}

/* layernorm_smooth_quantize_row_avx2 (src/simd_math.rs:367-477) */
__attribute__((target("avx2,fma"))) static float ln_quant_avx2(float* x, const float* g, const float* b,
                                                              const float* sm, int8_t* q, int n, float eps) {
  __m256 s0 = _mm256_setzero_ps(), s1 = _mm256_setzero_ps();
  for (int i = 0; i < n; i += 16) {
    s0 = _mm256_add_ps(s0, _mm256_loadu_ps(x + i));
    s1 = _mm256_add_ps(s1, _mm256_loadu_ps(x + i + 8));
  }
  const float mean = hsum256(_mm256_add_ps(s0, s1)) / (float)n;
  const __m256 vm = _mm256_set1_ps(mean);
  __m256 v0 = _mm256_setzero_ps(), v1 = _mm256_setzero_ps();
  for (int i = 0; i < n; i += 16) {
    const __m256 d0 = _mm256_sub_ps(_mm256_loadu_ps(x + i), vm), d1 = _mm256_sub_ps(_mm256_loadu_ps(x + i + 8), vm);
    v0 = _mm256_fmadd_ps(d0, d0, v0);
    v1 = _mm256_fmadd_ps(d1, d1, v1);
  }
  const float var = hsum256(_mm256_add_ps(v0, v1)) / (float)n;
  const __m256 rstd = _mm256_set1_ps(1.0f / sqrtf(var + eps));
  const __m256 sign = _mm256_set1_ps(-0.0f);
  __m256 vmax = _mm256_set1_ps(1e-8f);
  for (int i = 0; i < n; i += 16) {
    const __m256 y0 = _mm256_fmadd_ps(_mm256_mul_ps(_mm256_sub_ps(_mm256_loadu_ps(x + i), vm), rstd),
                                      _mm256_loadu_ps(g + i), _mm256_loadu_ps(b + i));
    const __m256 y1 = _mm256_fmadd_ps(_mm256_mul_ps(_mm256_sub_ps(_mm256_loadu_ps(x + i + 8), vm), rstd),
                                      _mm256_loadu_ps(g + i + 8), _mm256_loadu_ps(b + i + 8));
    _mm256_storeu_ps(x + i, y0);
    _mm256_storeu_ps(x + i + 8, y1);
    const __m256 a0 = _mm256_andnot_ps(sign, _mm256_mul_ps(y0, _mm256_loadu_ps(sm + i)));
    const __m256 a1 = _mm256_andnot_ps(sign, _mm256_mul_ps(y1, _mm256_loadu_ps(sm + i + 8)));
    vmax = _mm256_max_ps(vmax, _mm256_max_ps(a0, a1));
  }
  const float max_abs = hmax256(vmax);
  const __m256 inv = _mm256_set1_ps(127.0f / max_abs);
  for (int i = 0; i < n; i += 16)
    store_q16(q + i, _mm256_mul_ps(_mm256_loadu_ps(x + i), _mm256_mul_ps(_mm256_loadu_ps(sm + i), inv)),
              _mm256_mul_ps(_mm256_loadu_ps(x + i + 8), _mm256_mul_ps(_mm256_loadu_ps(sm + i + 8), inv)));
  return max_abs / 127.0f;
}

/* smooth_quantize_row_avx2 (src/simd_math.rs:584-649) */
__attribute__((target("avx2,fma"))) static float smooth_quant_avx2(const float* x, const float* sm, int8_t* q, int n) {
  const __m256 sign = _mm256_set1_ps(-0.0f);
  __m256 vmax = _mm256_set1_ps(1e-8f);
  for (int i = 0; i < n; i += 16) {
    const __m256 a0 = _mm256_andnot_ps(sign, _mm256_mul_ps(_mm256_loadu_ps(x + i), _mm256_loadu_ps(sm + i)));
    const __m256 a1 = _mm256_andnot_ps(sign, _mm256_mul_ps(_mm256_loadu_ps(x + i + 8), _mm256_loadu_ps(sm + i + 8)));
    vmax = _mm256_max_ps(vmax, _mm256_max_ps(a0, a1));
  }
  const float max_abs = hmax256(vmax);
  const __m256 inv = _mm256_set1_ps(127.0f / max_abs);
  for (int i = 0; i < n; i += 16)
    store_q16(q + i, _mm256_mul_ps(_mm256_loadu_ps(x + i), _mm256_mul_ps(_mm256_loadu_ps(sm + i), inv)),
              _mm256_mul_ps(_mm256_loadu_ps(x + i + 8), _mm256_mul_ps(_mm256_loadu_ps(sm + i + 8), inv)));
  return max_abs / 127.0f;
}

/* avx2_exp_f32 (src/simd_math.rs:113-143): clamp to [-87.3, 88], n = rint(y*log2e),
 * two-part ln2 reduction, degree-5 polynomial, scale by 2^n */
__attribute__((target("avx2,fma"))) static inline __m256 exp8(__m256 y) {
  y = _mm256_max_ps(_mm256_min_ps(y, _mm256_set1_ps(88.0f)), _mm256_set1_ps(-87.3f));
  const __m256 nf = _mm256_round_ps(_mm256_mul_ps(y, _mm256_set1_ps(1.44269504088896341f)),
                                    _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  const __m256 r = _mm256_fnmadd_ps(nf, _mm256_set1_ps(1.428606765330187e-6f),
                                    _mm256_fnmadd_ps(nf, _mm256_set1_ps(0.693145751953125f), y));
  const __m256 one = _mm256_set1_ps(1.0f);
  __m256 p = _mm256_fmadd_ps(r, _mm256_set1_ps(0.008333334f), _mm256_set1_ps(0.041666668f));
  p = _mm256_fmadd_ps(r, p, _mm256_set1_ps(0.16666667f));
  p = _mm256_fmadd_ps(r, p, _mm256_set1_ps(0.5f));
  p = _mm256_fmadd_ps(r, p, one);
  p = _mm256_fmadd_ps(r, p, one);
  const __m256i e = _mm256_slli_epi32(_mm256_add_epi32(_mm256_cvtps_epi32(nf), _mm256_set1_epi32(127)), 23);
  return _mm256_mul_ps(p, _mm256_castsi256_ps(e));
}

/* avx2_gelu_f32 (src/simd_math.rs:152-175): rational erf on x clamped to +-4.8,
 * reciprocal estimate + one Newton step */
__attribute__((target("avx2,fma"))) static inline __m256 gelu8(__m256 x) {
  const __m256 xc = _mm256_min_ps(_mm256_max_ps(x, _mm256_set1_ps(-4.8f)), _mm256_set1_ps(4.8f));
  const __m256 u = _mm256_mul_ps(xc, xc);
  __m256 num = _mm256_fmadd_ps(u, _mm256_set1_ps(6.4292e-5f), _mm256_set1_ps(0.007572631f));
  num = _mm256_fmadd_ps(u, num, _mm256_set1_ps(0.055282866f));
  num = _mm256_fmadd_ps(u, num, _mm256_set1_ps(0.797882463f));
  __m256 den = _mm256_fmadd_ps(u, _mm256_set1_ps(0.001139532f), _mm256_set1_ps(0.02381135f));
  den = _mm256_fmadd_ps(u, den, _mm256_set1_ps(0.235943093f));
  den = _mm256_fmadd_ps(u, den, _mm256_set1_ps(1.0f));
  const __m256 est = _mm256_rcp_ps(den);
  const __m256 inv = _mm256_mul_ps(est, _mm256_fnmadd_ps(den, est, _mm256_set1_ps(2.0f)));
  const __m256 erf = _mm256_min_ps(_mm256_max_ps(_mm256_mul_ps(xc, _mm256_mul_ps(num, inv)), _mm256_set1_ps(-1.0f)),
                                   _mm256_set1_ps(1.0f));
  return _mm256_mul_ps(_mm256_mul_ps(x, _mm256_set1_ps(0.5f)), _mm256_add_ps(_mm256_set1_ps(1.0f), erf));
}

/* gelu_smooth_quantize_row_avx2 (src/simd_math.rs:1371-1435) */
__attribute__((target("avx2,fma"))) static float gelu_quant_avx2(float* x, const float* sm, int8_t* q, int n) {
  const __m256 sign = _mm256_set1_ps(-0.0f);
  __m256 vmax = _mm256_set1_ps(1e-8f);
  for (int i = 0; i < n; i += 16) {
    const __m256 g0 = _mm256_mul_ps(gelu8(_mm256_loadu_ps(x + i)), _mm256_loadu_ps(sm + i));
    const __m256 g1 = _mm256_mul_ps(gelu8(_mm256_loadu_ps(x + i + 8)), _mm256_loadu_ps(sm + i + 8));
    _mm256_storeu_ps(x + i, g0);
    _mm256_storeu_ps(x + i + 8, g1);
    vmax = _mm256_max_ps(vmax, _mm256_max_ps(_mm256_andnot_ps(sign, g0), _mm256_andnot_ps(sign, g1)));
  }
  const float max_abs = hmax256(vmax);
  const __m256 inv = _mm256_set1_ps(127.0f / max_abs);
  for (int i = 0; i < n; i += 16)
    store_q16(q + i, _mm256_mul_ps(_mm256_loadu_ps(x + i), inv), _mm256_mul_ps(_mm256_loadu_ps(x + i + 8), inv));
  return max_abs / 127.0f;
}

/* ---- attention (src/simd_math.rs:2905-3075) ---- */
/* dot32x4_avx2: 8-lane partial dot of a key with q held in 4 registers */
__attribute__((target("avx2,fma"))) static inline __m256 dot32x4(__m256 q0, __m256 q1, __m256 q2, __m256 q3,
                                                               const float* k) {
  const __m256 a = _mm256_fmadd_ps(q1, _mm256_loadu_ps(k + 8), _mm256_mul_ps(q0, _mm256_loadu_ps(k)));
  const __m256 b = _mm256_fmadd_ps(q3, _mm256_loadu_ps(k + 24), _mm256_mul_ps(q2, _mm256_loadu_ps(k + 16)));
  return _mm256_add_ps(a, b);
}

/* compute_scores_head32_avx2: scores[t] = dot(q*scale, k_t), 4 keys reduced by a hadd tree */
__attribute__((target("avx2,fma"))) static void scores_avx2(const float* q, const float* k, float scale, float* sp,
                                                           int len) {
  const __m256 vs = _mm256_set1_ps(scale);
  const __m256 q0 = _mm256_mul_ps(_mm256_loadu_ps(q), vs), q1 = _mm256_mul_ps(_mm256_loadu_ps(q + 8), vs);
  const __m256 q2 = _mm256_mul_ps(_mm256_loadu_ps(q + 16), vs), q3 = _mm256_mul_ps(_mm256_loadu_ps(q + 24), vs);
  int t = 0;
  for (; t + 4 <= len; t += 4) {
    const float* k0 = k + (size_t)t * 32;
    const __m256 s0 = dot32x4(q0, q1, q2, q3, k0), s1 = dot32x4(q0, q1, q2, q3, k0 + 32);
    const __m256 s2 = dot32x4(q0, q1, q2, q3, k0 + 64), s3 = dot32x4(q0, q1, q2, q3, k0 + 96);
    const __m256 h = _mm256_hadd_ps(_mm256_hadd_ps(s0, s1), _mm256_hadd_ps(s2, s3));
    _mm_storeu_ps(sp + t, _mm_add_ps(_mm256_castps256_ps128(h), _mm256_extractf128_ps(h, 1)));
  }
  for (; t < len; t++) sp[t] = hsum256(dot32x4(q0, q1, q2, q3, k + (size_t)t * 32));
}

/* softmax_inplace_avx2: vector max, exps 16 then 8 at a time (two partial sums),
 * libm expf for the tail, then scale by 1/sum */
__attribute__((target("avx2,fma"))) static void softmax_avx2(float* s, int len) {
  if (len <= 0) return;
  int i = 0;
  __m256 vmax = _mm256_set1_ps(-INFINITY);
  for (; i + 8 <= len; i += 8) vmax = _mm256_max_ps(vmax, _mm256_loadu_ps(s + i));
  float mx = hmax256(vmax);
  for (; i < len; i++) mx = fmaxf(mx, s[i]);
  const __m256 vm = _mm256_set1_ps(mx);
  __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
  i = 0;
  for (; i + 16 <= len; i += 16) {
    const __m256 e0 = exp8(_mm256_sub_ps(_mm256_loadu_ps(s + i), vm));
    const __m256 e1 = exp8(_mm256_sub_ps(_mm256_loadu_ps(s + i + 8), vm));
    _mm256_storeu_ps(s + i, e0);
    _mm256_storeu_ps(s + i + 8, e1);
    a0 = _mm256_add_ps(a0, e0);
    a1 = _mm256_add_ps(a1, e1);
  }
  for (; i + 8 <= len; i += 8) {
    const __m256 e = exp8(_mm256_sub_ps(_mm256_loadu_ps(s + i), vm));
    _mm256_storeu_ps(s + i, e);
    a0 = _mm256_add_ps(a0, e);
  }
  float sum = hsum256(_mm256_add_ps(a0, a1));
  for (; i < len; i++) {
    const float e = expf(s[i] - mx);
    s[i] = e;
    sum += e;
  }
  const float inv = 1.0f / sum;
  const __m256 vi = _mm256_set1_ps(inv);
  i = 0;
  for (; i + 8 <= len; i += 8) _mm256_storeu_ps(s + i, _mm256_mul_ps(_mm256_loadu_ps(s + i), vi));
  for (; i < len; i++) s[i] *= inv;
}

/* weighted_sum_head32_avx2: two rows per step into two accumulator sets */
__attribute__((target("avx2,fma"))) static void wsum_avx2(const float* p, const float* v, int len, float* out) {
  __m256 a[4], b[4];
  for (int j = 0; j < 4; j++) a[j] = b[j] = _mm256_setzero_ps();
  int t = 0;
  for (; t + 2 <= len; t += 2) {
    const __m256 pa = _mm256_set1_ps(p[t]), pb = _mm256_set1_ps(p[t + 1]);
    const float *ra = v + (size_t)t * 32, *rb = ra + 32;
    for (int j = 0; j < 4; j++) {
      a[j] = _mm256_fmadd_ps(_mm256_loadu_ps(ra + 8 * j), pa, a[j]);
      b[j] = _mm256_fmadd_ps(_mm256_loadu_ps(rb + 8 * j), pb, b[j]);
    }
  }
  if (t < len) {
    const __m256 pa = _mm256_set1_ps(p[t]);
    for (int j = 0; j < 4; j++) a[j] = _mm256_fmadd_ps(_mm256_loadu_ps(v + (size_t)t * 32 + 8 * j), pa, a[j]);
  }
  for (int j = 0; j < 4; j++) _mm256_storeu_ps(out + 8 * j, _mm256_add_ps(a[j], b[j]));
}

static const or_kernels k_avx2 = {gemm_avx2, ln_quant_avx2, smooth_quant_avx2, gelu_quant_avx2,
                                  scores_avx2, softmax_avx2, wsum_avx2};
static const or_kernels k_vnni = {gemm_vnni, ln_quant_avx2, smooth_quant_avx2, gelu_quant_avx2,
                                  scores_avx2, softmax_avx2, wsum_avx2};

/* ArcticEmbedS::embed_batch (src/lib.rs:138-260) on the x86 backend; the model
 * must have been through or_x86_prepare.  Returns OR_ERR_ARG without AVX2+FMA. */
int or_x86_embed_batch_tokens(const or_model* m, const uint16_t* ids, const uint32_t* offsets, size_t n,
                              int num_threads, float* out) {
  const int be = or_x86_backend();
  if (be == 0) return OR_ERR_ARG;
  return or_embed_batch_tokens_k(m, ids, offsets, n, num_threads, out, be == 2 ? &k_vnni : &k_avx2);
}

/* test hook: one GEMM on the x86 backend (variant 1: AVX2 maddubs, 2: AVX-VNNI);
 * packs `w` on first use.  Both must equal or_gemm bit for bit. */
int or_x86_gemm(int m, const int8_t* a, const float* a_scale, or_linear* w, const float* res, float* out,
                int variant) {
  const int be = or_x86_backend();
  if (variant < 1 || variant > be) return OR_ERR_ARG;
  if (!w->xpack || (variant == 2 && !w->xcomp)) {
    free(w->xpack);
    free(w->xcomp);
    w->xpack = NULL;
    w->xcomp = NULL;
    if (pack_linear(w, 1)) return OR_ERR_ARG;
  }
  if (variant == 2) gemm_vnni(m, a, a_scale, w, res, out);
  else gemm_avx2(m, a, a_scale, w, res, out);
  return OR_OK;
}
