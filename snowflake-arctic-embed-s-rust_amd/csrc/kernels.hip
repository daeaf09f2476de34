// kernels.hip -- CDNA4 (gfx950) kernels of the W8A8 arctic-embed-s encoder.
//
// Build flags that carry semantics: -ffp-contract=off (no a*b+c fusion: the
// reference is Rust, which never contracts), correctly rounded f32 divide and
// sqrt (HIP's default), no fast-math.  Every kernel whose output is int8 or a
// GEMM f32 result evaluates exactly the reference's scalar expression order, so
// those outputs are bit-identical to the reference's scalar backend on the same
// inputs.  Attention is f32 with a different summation order (tolerance-level).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.hpp"

namespace aek {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int H = 384;
constexpr int HQKV = 3 * 384;
constexpr float kInvSqrtD = 0.17677669529663687f;  // 1.0f / sqrtf(32.0f), src/model.rs:222

// ---------------------------------------------------------------------------
// exact scalar building blocks
// ---------------------------------------------------------------------------

// `(v).round().clamp(-127.0, 127.0) as i8` (f32::round = half away from zero;
// `as i8` maps NaN to 0).
__device__ __forceinline__ int qround(float v) {
  float r = roundf(v);
  if (__builtin_isnan(r)) return 0;
  r = fminf(fmaxf(r, -127.0f), 127.0f);
  return (int)r;
}

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
  return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
         ((uint32_t)(d & 0xff) << 24);
}

// max(m, a) that ignores a NaN `a`, like `if a > max_abs { max_abs = a }`.
__device__ __forceinline__ float nanless_max(float m, float a) { return a > m ? a : m; }

// expf as glibc computes it on x86_64 (sysdeps/ieee754/flt-32/e_expf.c, the
// ARM optimized-routines design with a 32-entry 2^(i/32) table and a cubic
// polynomial, evaluated in double with the FMA contractions of glibc's -mfma
// build).  The reference's scalar GELU calls f32::exp, i.e. this function.
// Verified equal to glibc expf on every float in [-104, -0]; valid for x <= 0.
// `tab` holds bits(2^(i/32)) - (i << 47).
__device__ __forceinline__ float expf_libm(float x, const uint64_t* tab) {
  if (x < -0x1.9fe368p6f) return 0.0f;  // below log(2^-150): glibc's underflow branch
  const double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
  const double kShift = 0x1.8p+52;
  const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
  const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
  const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  const double xd = (double)x;
  double kd = __builtin_fma(kInvLn2N, xd, kShift);
  const uint64_t ki = (uint64_t)__double_as_longlong(kd);
  kd -= kShift;
  const double r = __builtin_fma(kInvLn2N, xd, -kd);
  const uint64_t t = tab[ki & 31] + (ki << 47);
  const double s = __longlong_as_double((long long)t);
  const double z = __builtin_fma(c0, r, c1);
  const double r2 = r * r;
  double y = __builtin_fma(c2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return (float)y;
}

// scalar_gelu (reference src/simd_math.rs:15-23), same operation order.
__device__ __forceinline__ float gelu_exact(float x, const uint64_t* tab) {
  const float z = fabsf(x) * 0.70710677f;
  const float t = 1.0f / (1.0f + 0.3275911f * z);
  const float poly =
      t * (0.254829592f + t * (-0.284496736f + t * (1.421413741f + t * (-1.453152027f + t * 1.061405429f))));
  const float erf_val = copysignf(1.0f - poly * expf_libm(-z * z, tab), x);
  return 0.5f * x * (1.0f + erf_val);
}

// bits(2^(i/32) rounded to double) - (i << 47), i = 0..31: the exp2 table of the
// algorithm above (computed from 2^(i/32) in quad precision).
__constant__ uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

__device__ __forceinline__ void load_exp_tab(uint64_t* s_tab) {
  if (threadIdx.x < 32) s_tab[threadIdx.x] = kExp2Tab[threadIdx.x];
}

// index of the segment containing token t: largest b with cu[b] <= t (cu has B+1 entries)
__device__ __forceinline__ int find_segment(const int* cu, int B, int t) {
  int lo = 0, hi = B - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// ---------------------------------------------------------------------------
// W8A8 GEMM: out[m,n] = fma(f32(sum_k a[m,k]*w[n,k]), sa[m]*ws[n], bias[n] (+res[m,n]))
//
// WG = 4 waves (2x2), WG tile 128x128, wave tile 64x64 = 4x4 v_mfma_i32_16x16x64_i8,
// K step 64, A and W tiles double-buffered in LDS with an 80-byte row pitch
// (conflict-free 16-byte fragment reads).  W is pre-swizzled at load time into
// [N/128][K/64][128 rows][64 bytes] tiles so each tile is one contiguous 8 KiB.
//
// MFMA operand layout (16x16x64 i8): lane l supplies row (l%16) of A and column
// (l%16) of B, 16 k-values each from k-group (l/16); any k-permutation shared by
// A and B gives the same exact integer sum.  Output: lane l, register r holds
// D[4*(l/16)+r][l%16].
// ---------------------------------------------------------------------------
constexpr int kPitch = 80;

template <int AM, int EM>
__global__ __launch_bounds__(256) void gemm_w8a8_kernel(GemmArgs p) {
  __shared__ __attribute__((aligned(16))) int8_t sA[2][128 * kPitch];
  __shared__ __attribute__((aligned(16))) int8_t sW[2][128 * kPitch];
  __shared__ uint64_t sTab[32];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.x * 128, n0 = blockIdx.y * 128;  // M tiles on x (y is limited to 65536)
  const int KT = p.K >> 6;
  if (EM == kEpiGelu) load_exp_tab(sTab);

  // loader: 2 threads per row, 32 bytes each
  const int lrow = tid >> 1, lhalf = tid & 1;
  const int arow = min(m0 + lrow, p.M - 1);
  float a_inv = 0.0f;
  if (AM != kAI8) {
    const float mx = __uint_as_float(p.a_rowmax[arow]);
    a_inv = 127.0f / mx;  // inv_scale = 127.0 / max_abs
  }
  v4i ra0, ra1, rw0, rw1;
  auto gload = [&](int kt) {
    const int kb = kt * 64 + lhalf * 32;
    if (AM == kAI8) {
      const int8_t* src = reinterpret_cast<const int8_t*>(p.A) + (size_t)arow * p.K + kb;
      ra0 = *reinterpret_cast<const v4i*>(src);
      ra1 = *reinterpret_cast<const v4i*>(src + 16);
    } else {
      const float4* src = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p.A) + (size_t)arow * p.K + kb);
      uint32_t w[8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        float4 x = src[i];
        if (AM == kAF32QSmooth) {  // (x * inv_smooth[j]) * inv_scale
          const float4 s = reinterpret_cast<const float4*>(p.a_smooth + kb)[i];
          x.x = x.x * s.x; x.y = x.y * s.y; x.z = x.z * s.z; x.w = x.w * s.w;
        }
        w[i] = pack4(qround(x.x * a_inv), qround(x.y * a_inv), qround(x.z * a_inv), qround(x.w * a_inv));
      }
      ra0 = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
      ra1 = v4i{(int)w[4], (int)w[5], (int)w[6], (int)w[7]};
    }
    const int8_t* wsrc = p.w + ((size_t)blockIdx.y * KT + kt) * 8192 + lrow * 64 + lhalf * 32;
    rw0 = *reinterpret_cast<const v4i*>(wsrc);
    rw1 = *reinterpret_cast<const v4i*>(wsrc + 16);
  };
  auto lstore = [&](int buf) {
    int8_t* a = &sA[buf][lrow * kPitch + lhalf * 32];
    int8_t* w = &sW[buf][lrow * kPitch + lhalf * 32];
    *reinterpret_cast<v4i*>(a) = ra0;
    *reinterpret_cast<v4i*>(a + 16) = ra1;
    *reinterpret_cast<v4i*>(w) = rw0;
    *reinterpret_cast<v4i*>(w + 16) = rw1;
  };

  v4i acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = v4i{0, 0, 0, 0};

  gload(0);
  lstore(0);
  __syncthreads();
  const int fr = lane & 15, fk = (lane >> 4) * 16;
  for (int kt = 0; kt < KT; kt++) {
    const int buf = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
    v4i af[4], bf[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      af[i] = *reinterpret_cast<const v4i*>(&sA[buf][(wm * 64 + i * 16 + fr) * kPitch + fk]);
      bf[i] = *reinterpret_cast<const v4i*>(&sW[buf][(wn * 64 + i * 16 + fr) * kPitch + fk]);
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
    if (kt + 1 < KT) lstore(buf ^ 1);
    __syncthreads();
  }

  // epilogue
  const int col_base = n0 + wn * 64 + fr;
  float wsc[4], bia[4], gsm[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int col = col_base + j * 16;
    wsc[j] = p.w_scale[col];
    bia[j] = p.bias[col];
    gsm[j] = (EM == kEpiGelu) ? p.g_smooth[col] : 0.0f;
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int row = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
      const bool ok = row < p.M;
      const int rrow = ok ? row : p.M - 1;
      float sa;
      if (AM == kAI8) sa = p.a_scale[rrow];
      else sa = __uint_as_float(p.a_rowmax[rrow]) / 127.0f;  // scale = max_abs / 127.0
      float gmax = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int col = col_base + j * 16;
        float bval = bia[j];
        if (p.res) bval = bval + p.res[(size_t)rrow * p.N + col];
        const float v = fmaf((float)acc[i][j][r], sa * wsc[j], bval);
        if (EM == kEpiGelu) {
          const float g = gelu_exact(v, sTab) * gsm[j];
          if (ok) p.out[(size_t)row * p.N + col] = g;
          gmax = nanless_max(gmax, fabsf(g));
        } else {
          if (ok) p.out[(size_t)row * p.N + col] = v;
        }
      }
      if (EM == kEpiGelu) {
        // reduce over the 16 lanes that share this row (same lane>>4)
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) gmax = nanless_max(gmax, __shfl_xor(gmax, off, 64));
        if (ok && fr == 0) atomicMax(&p.g_rowmax[row], __float_as_uint(gmax));
      }
    }
  }
}

void launch_gemm(const GemmArgs& p, int amode, int emode, hipStream_t st) {
  dim3 grid((p.M + 127) / 128, p.N / 128);
  if (amode == kAI8 && emode == kEpiF32) hipLaunchKernelGGL((gemm_w8a8_kernel<kAI8, kEpiF32>), grid, dim3(256), 0, st, p);
  else if (amode == kAI8 && emode == kEpiGelu) hipLaunchKernelGGL((gemm_w8a8_kernel<kAI8, kEpiGelu>), grid, dim3(256), 0, st, p);
  else if (amode == kAF32Q && emode == kEpiF32) hipLaunchKernelGGL((gemm_w8a8_kernel<kAF32Q, kEpiF32>), grid, dim3(256), 0, st, p);
  else if (amode == kAF32QSmooth && emode == kEpiF32) hipLaunchKernelGGL((gemm_w8a8_kernel<kAF32QSmooth, kEpiF32>), grid, dim3(256), 0, st, p);
}

// ---------------------------------------------------------------------------
// LayerNorm + SmoothQuant + dynamic int8 quantization over 384-wide rows
// (layernorm_smooth_quantize_row_scalar, reference src/simd_math.rs:208-247).
//
// WG = 256 threads, 32 rows.  Phase A stages x into LDS; phase B gives each
// row to one lane, which forms the mean and variance with the reference's
// sequential left-to-right sums; phase C normalizes, takes the order-free row
// absmax and quantizes with 8 lanes per row.  Source modes: f32 rows, or the
// embedding gather ((w*ws + p*ps) + type0, src/simd_math.rs:1877-1880).
// ---------------------------------------------------------------------------
constexpr int kLnRows = 32;
constexpr int kLnPitch = 388;

template <int SRC>
__global__ __launch_bounds__(256) void ln_quant_kernel(LnArgs p) {
  __shared__ __attribute__((aligned(16))) float tile[kLnRows * kLnPitch];
  __shared__ float s_mean[kLnRows], s_rstd[kLnRows];
  const int tid = threadIdx.x, rl = tid >> 3, sub = tid & 7;
  const int row = blockIdx.x * kLnRows + rl;
  const bool valid = row < p.T;
  const int rrow = valid ? row : p.T - 1;

  float4 xv[12];
  if (SRC == kLnSrcEmb) {
    // ids and positions are validated on the host; the clamps keep a malformed
    // device-resident batch inside the tables
    const int tok = min((int)p.ids[rrow], 30522 - 1);
    const int seg = find_segment(p.cu, p.B, rrow);
    const int pos = max(0, min(rrow - p.cu[seg], 512 - 1));
    const float ws = p.word_s[tok], ps = p.pos_s[pos];
    const int8_t* wr = p.word_q + (size_t)tok * H;
    const int8_t* pr = p.pos_q + (size_t)pos * H;
#pragma unroll
    for (int i = 0; i < 12; i++) {
      const int c = (sub + 8 * i) * 4;
      const uint32_t wv = *reinterpret_cast<const uint32_t*>(wr + c);
      const uint32_t pv = *reinterpret_cast<const uint32_t*>(pr + c);
      const float4 t = *reinterpret_cast<const float4*>(p.type0 + c);
      float x[4];
      const float tt[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const float w = (float)(int8_t)(wv >> (8 * k));
        const float q = (float)(int8_t)(pv >> (8 * k));
        x[k] = w * ws + q * ps + tt[k];
      }
      xv[i] = make_float4(x[0], x[1], x[2], x[3]);
    }
  } else {
    const float4* src = reinterpret_cast<const float4*>(p.src + (size_t)rrow * H);
#pragma unroll
    for (int i = 0; i < 12; i++) xv[i] = src[sub + 8 * i];
  }
#pragma unroll
  for (int i = 0; i < 12; i++) *reinterpret_cast<float4*>(&tile[rl * kLnPitch + (sub + 8 * i) * 4]) = xv[i];
  __syncthreads();

  if (tid < kLnRows) {
    const float* xr = &tile[tid * kLnPitch];
    float sum = 0.0f;
    for (int j = 0; j < H; j += 4) {
      const float4 v = *reinterpret_cast<const float4*>(xr + j);
      sum += v.x; sum += v.y; sum += v.z; sum += v.w;
    }
    const float mean = sum / 384.0f;
    float var_sum = 0.0f;
    for (int j = 0; j < H; j += 4) {
      const float4 v = *reinterpret_cast<const float4*>(xr + j);
      float d;
      d = v.x - mean; var_sum += d * d;
      d = v.y - mean; var_sum += d * d;
      d = v.z - mean; var_sum += d * d;
      d = v.w - mean; var_sum += d * d;
    }
    s_mean[tid] = mean;
    s_rstd[tid] = 1.0f / sqrtf(var_sum / 384.0f + 1e-12f);
  }
  __syncthreads();

  const float mean = s_mean[rl], rstd = s_rstd[rl];
  float amax = 0.0f;
  float4 ys[12];
#pragma unroll
  for (int i = 0; i < 12; i++) {
    const int c = (sub + 8 * i) * 4;
    const float4 g = *reinterpret_cast<const float4*>(p.gamma + c);
    const float4 b = *reinterpret_cast<const float4*>(p.beta + c);
    const float4 s = *reinterpret_cast<const float4*>(p.smooth + c);
    float4 y;
    y.x = (xv[i].x - mean) * rstd * g.x + b.x;
    y.y = (xv[i].y - mean) * rstd * g.y + b.y;
    y.z = (xv[i].z - mean) * rstd * g.z + b.z;
    y.w = (xv[i].w - mean) * rstd * g.w + b.w;
    if (valid) *reinterpret_cast<float4*>(p.dst + (size_t)row * H + c) = y;
    ys[i] = make_float4(y.x * s.x, y.y * s.y, y.z * s.z, y.w * s.w);
    amax = nanless_max(amax, fabsf(ys[i].x));
    amax = nanless_max(amax, fabsf(ys[i].y));
    amax = nanless_max(amax, fabsf(ys[i].z));
    amax = nanless_max(amax, fabsf(ys[i].w));
  }
#pragma unroll
  for (int off = 1; off < 8; off <<= 1) amax = nanless_max(amax, __shfl_xor(amax, off, 64));
  const float max_abs = nanless_max(1e-8f, amax);
  const float inv_scale = 127.0f / max_abs;
  if (valid) {
#pragma unroll
    for (int i = 0; i < 12; i++) {
      const int c = (sub + 8 * i) * 4;
      *reinterpret_cast<uint32_t*>(p.q + (size_t)row * H + c) =
          pack4(qround(ys[i].x * inv_scale), qround(ys[i].y * inv_scale), qround(ys[i].z * inv_scale),
                qround(ys[i].w * inv_scale));
    }
    if (sub == 0) {
      p.scale[row] = max_abs / 127.0f;
      if (p.rowmax_init) p.rowmax_init[row] = __float_as_uint(1e-8f);
      if (p.rowmax_init2) p.rowmax_init2[row] = __float_as_uint(1e-8f);
    }
  }
}

void launch_ln_quant(const LnArgs& p, int src_mode, hipStream_t st) {
  dim3 grid((p.T + kLnRows - 1) / kLnRows);
  if (src_mode == kLnSrcEmb) hipLaunchKernelGGL((ln_quant_kernel<kLnSrcEmb>), grid, dim3(256), 0, st, p);
  else hipLaunchKernelGGL((ln_quant_kernel<kLnSrcF32>), grid, dim3(256), 0, st, p);
}

// ---------------------------------------------------------------------------
// Stand-alone row quantizers (operator-level API): one wave per row.
// smooth_quantize_row (src/simd_math.rs:513-530), gelu_smooth_quantize_row
// (src/simd_math.rs:1295-1312).
// ---------------------------------------------------------------------------
template <bool GELU>
__global__ __launch_bounds__(256) void row_quant_kernel(int m, int n, float* x, const float* smooth, int8_t* q,
                                                        float* scale) {
  __shared__ uint64_t sTab[32];
  if (GELU) load_exp_tab(sTab);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= m) return;
  float* xr = x + (size_t)row * n;
  float amax = 0.0f;
  for (int j = lane; j < n; j += 64) {
    float v = xr[j];
    if (GELU) {
      v = gelu_exact(v, sTab) * smooth[j];
      xr[j] = v;
    } else {
      v = v * smooth[j];
    }
    amax = nanless_max(amax, fabsf(v));
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) amax = nanless_max(amax, __shfl_xor(amax, off, 64));
  const float max_abs = nanless_max(1e-8f, amax);
  const float inv_scale = 127.0f / max_abs;
  for (int j = lane; j < n; j += 64) {
    const float v = GELU ? xr[j] * inv_scale : xr[j] * smooth[j] * inv_scale;
    q[(size_t)row * n + j] = (int8_t)qround(v);
  }
  if (lane == 0) scale[row] = max_abs / 127.0f;
}

void launch_row_quant(int m, int n, float* x, const float* smooth, int8_t* q, float* scale, bool gelu,
                      hipStream_t st) {
  dim3 grid((m + 3) / 4);
  if (gelu) hipLaunchKernelGGL((row_quant_kernel<true>), grid, dim3(256), 0, st, m, n, x, smooth, q, scale);
  else hipLaunchKernelGGL((row_quant_kernel<false>), grid, dim3(256), 0, st, m, n, x, smooth, q, scale);
}

// ---------------------------------------------------------------------------
// Varlen attention, head_dim 32.  tile_start[b] = sum_{b'<b} ceil(L_b'/64) is
// built on the device from cu_seqlens; WG (tile, head) owns 64 queries of one
// sequence; 4 lanes per query (8 dims each); keys/values stream through LDS in
// chunks of 64 with an online softmax.  Also folds the SmoothQuant row absmax
// of the attention output (|ctx_j * inv_smooth_j|) into `rowmax` (atomicMax on
// the non-negative float bits), which the attn_out GEMM prologue consumes.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void tile_starts_kernel(const int* cu, int B, int* tile_start) {
  __shared__ int part[256];
  const int tid = threadIdx.x;
  const int per = (B + 255) / 256;
  const int b0 = min(B, tid * per), b1 = min(B, b0 + per);
  int s = 0;
  for (int b = b0; b < b1; b++) s += (cu[b + 1] - cu[b] + 63) >> 6;
  part[tid] = s;
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    for (int i = 0; i < 256; i++) {
      int v = part[i];
      part[i] = acc;
      acc += v;
    }
  }
  __syncthreads();
  int acc = part[tid];
  for (int b = b0; b < b1; b++) {
    tile_start[b] = acc;
    acc += (cu[b + 1] - cu[b] + 63) >> 6;
  }
  if (b1 == B && b0 < b1) tile_start[B] = acc;
  if (B == 0 && tid == 0) tile_start[0] = 0;
}

__global__ __launch_bounds__(256) void attention_kernel(AttnArgs p) {
  __shared__ __attribute__((aligned(16))) float sK[64 * 32];
  __shared__ __attribute__((aligned(16))) float sV[64 * 32];
  const int tile = blockIdx.x, h = blockIdx.y;
  if (tile >= p.tile_start[p.B]) return;
  int lo = 0, hi = p.B - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (p.tile_start[mid] <= tile) lo = mid; else hi = mid - 1;
  }
  const int b = lo;
  const int s0 = p.cu[b], L = p.cu[b + 1] - s0;
  const int q0 = (tile - p.tile_start[b]) * 64;
  const int tid = threadIdx.x, qi = tid >> 2, sub = tid & 3;
  const int qrow = q0 + qi;
  const bool qvalid = qrow < L;
  const int qr = min(qrow, L - 1);
  float q[8];
  {
    const float4* qs = reinterpret_cast<const float4*>(p.qkv + (size_t)(s0 + qr) * HQKV + h * 32 + sub * 8);
    float4 a = qs[0], c = qs[1];
    q[0] = a.x; q[1] = a.y; q[2] = a.z; q[3] = a.w; q[4] = c.x; q[5] = c.y; q[6] = c.z; q[7] = c.w;
  }
  float m = -INFINITY, l = 0.0f, o[8];
#pragma unroll
  for (int d = 0; d < 8; d++) o[d] = 0.0f;

  for (int k0 = 0; k0 < L; k0 += 64) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int idx = tid + i * 256, key = idx >> 3, c4 = idx & 7;
      const int kr = k0 + key;
      float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
      if (kr < L) {
        const float* base = p.qkv + (size_t)(s0 + kr) * HQKV + h * 32 + c4 * 4;
        kv = *reinterpret_cast<const float4*>(base + H);
        vv = *reinterpret_cast<const float4*>(base + 2 * H);
      }
      *reinterpret_cast<float4*>(&sK[key * 32 + c4 * 4]) = kv;
      *reinterpret_cast<float4*>(&sV[key * 32 + c4 * 4]) = vv;
    }
    __syncthreads();
    const int nk = min(64, L - k0);
    float s[64];
    float cmax = -INFINITY;
#pragma unroll
    for (int j = 0; j < 64; j++) {
      const float4 ka = *reinterpret_cast<const float4*>(&sK[j * 32 + sub * 8]);
      const float4 kb = *reinterpret_cast<const float4*>(&sK[j * 32 + sub * 8 + 4]);
      float d = q[0] * ka.x + q[1] * ka.y + q[2] * ka.z + q[3] * ka.w + q[4] * kb.x + q[5] * kb.y + q[6] * kb.z +
                q[7] * kb.w;
      d += __shfl_xor(d, 1, 64);
      d += __shfl_xor(d, 2, 64);
      s[j] = j < nk ? d * kInvSqrtD : -INFINITY;
      cmax = fmaxf(cmax, s[j]);
    }
    const float mnew = fmaxf(m, cmax);
    const float corr = __expf(m - mnew);
    l *= corr;
#pragma unroll
    for (int d = 0; d < 8; d++) o[d] *= corr;
#pragma unroll
    for (int j = 0; j < 64; j++) {
      const float pj = __expf(s[j] - mnew);
      l += pj;
      const float4 va = *reinterpret_cast<const float4*>(&sV[j * 32 + sub * 8]);
      const float4 vb = *reinterpret_cast<const float4*>(&sV[j * 32 + sub * 8 + 4]);
      o[0] += pj * va.x; o[1] += pj * va.y; o[2] += pj * va.z; o[3] += pj * va.w;
      o[4] += pj * vb.x; o[5] += pj * vb.y; o[6] += pj * vb.z; o[7] += pj * vb.w;
    }
    m = mnew;
  }
  const float inv_l = 1.0f / l;
  float amax = 0.0f;
#pragma unroll
  for (int d = 0; d < 8; d++) {
    o[d] = o[d] * inv_l;
    if (p.smooth) amax = nanless_max(amax, fabsf(o[d] * p.smooth[h * 32 + sub * 8 + d]));
  }
  if (qvalid) {
    float4* dst = reinterpret_cast<float4*>(p.ctx + (size_t)(s0 + qrow) * H + h * 32 + sub * 8);
    dst[0] = make_float4(o[0], o[1], o[2], o[3]);
    dst[1] = make_float4(o[4], o[5], o[6], o[7]);
  }
  if (p.rowmax) {
    amax = nanless_max(amax, __shfl_xor(amax, 1, 64));
    amax = nanless_max(amax, __shfl_xor(amax, 2, 64));
    if (qvalid && sub == 0) atomicMax(&p.rowmax[s0 + qrow], __float_as_uint(amax));
  }
}

void launch_attention(const AttnArgs& p, int max_tiles, hipStream_t st) {
  hipLaunchKernelGGL(tile_starts_kernel, dim3(1), dim3(256), 0, st, p.cu, p.B, p.tile_start);
  if (max_tiles > 0) hipLaunchKernelGGL(attention_kernel, dim3(max_tiles, 12), dim3(256), 0, st, p);
}

// ---------------------------------------------------------------------------
// Layer-11 [CLS] pruning (reference src/model.rs:770-913)
// ---------------------------------------------------------------------------
// gather the B [CLS] rows (act_q, act_scale, hidden) into compact buffers
__global__ __launch_bounds__(128) void gather_cls_kernel(ClsArgs p) {
  const int b = blockIdx.x, t = threadIdx.x;
  const int src = p.cu[b];
  if (t < 96) {
    reinterpret_cast<float4*>(p.hidden_c + (size_t)b * H)[t] = reinterpret_cast<const float4*>(p.hidden + (size_t)src * H)[t];
    reinterpret_cast<uint32_t*>(p.act_q_c + (size_t)b * H)[t] = reinterpret_cast<const uint32_t*>(p.act_q + (size_t)src * H)[t];
  }
  if (t == 0) {
    p.act_scale_c[b] = p.act_scale[src];
    p.rowmax_init[b] = __float_as_uint(1e-8f);
  }
}

// one wave per (sequence, head): the [CLS] query attends to its segment
__global__ __launch_bounds__(64) void cls_attention_kernel(ClsArgs p) {
  const int b = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int s0 = p.cu[b], L = p.cu[b + 1] - s0;
  float q[32];
#pragma unroll
  for (int d = 0; d < 32; d += 4) {
    const float4 v = *reinterpret_cast<const float4*>(p.q_c + (size_t)b * H + h * 32 + d);
    q[d] = v.x; q[d + 1] = v.y; q[d + 2] = v.z; q[d + 3] = v.w;
  }
  float sc[8];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int j = lane + 64 * i;
    sc[i] = -INFINITY;
    if (j < L) {
      const float* kr = p.kv + (size_t)(s0 + j) * 2 * H + h * 32;
      float d = 0.0f;
#pragma unroll
      for (int e = 0; e < 32; e += 4) {
        const float4 k = *reinterpret_cast<const float4*>(kr + e);
        d += q[e] * k.x + q[e + 1] * k.y + q[e + 2] * k.z + q[e + 3] * k.w;
      }
      sc[i] = d * kInvSqrtD;
      m = fmaxf(m, sc[i]);
    }
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  float o[32];
#pragma unroll
  for (int d = 0; d < 32; d++) o[d] = 0.0f;
  float l = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int j = lane + 64 * i;
    if (j < L) {
      const float pj = __expf(sc[i] - m);
      l += pj;
      const float* vr = p.kv + (size_t)(s0 + j) * 2 * H + H + h * 32;
#pragma unroll
      for (int e = 0; e < 32; e += 4) {
        const float4 v = *reinterpret_cast<const float4*>(vr + e);
        o[e] += pj * v.x; o[e + 1] += pj * v.y; o[e + 2] += pj * v.z; o[e + 3] += pj * v.w;
      }
    }
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    l += __shfl_xor(l, off, 64);
#pragma unroll
    for (int d = 0; d < 32; d++) o[d] += __shfl_xor(o[d], off, 64);
  }
  const float inv_l = 1.0f / l;
  float mine = 0.0f;
#pragma unroll
  for (int d = 0; d < 32; d++)
    if (lane == d) mine = o[d] * inv_l;
  if (lane < 32) p.ctx_c[(size_t)b * H + h * 32 + lane] = mine;
  float a = lane < 32 ? fabsf(mine * p.smooth[h * 32 + lane]) : 0.0f;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) a = nanless_max(a, __shfl_xor(a, off, 64));
  if (lane == 0) atomicMax(&p.rowmax_ctx_c[b], __float_as_uint(a));
}

// final LayerNorm (no quantization, src/simd_math.rs:481-497) and L2 normalize
// (src/simd_math.rs:2892-2903), one lane per row, sequential sums
__global__ __launch_bounds__(64) void final_ln_l2_kernel(int B, const float* src, const float* gamma,
                                                         const float* beta, float* out) {
  const int b = blockIdx.x * 64 + threadIdx.x;
  if (b >= B) return;
  const float* x = src + (size_t)b * H;
  float* y = out + (size_t)b * H;
  float sum = 0.0f;
  for (int j = 0; j < H; j++) sum += x[j];
  const float mean = sum / 384.0f;
  float var_sum = 0.0f;
  for (int j = 0; j < H; j++) {
    const float d = x[j] - mean;
    var_sum += d * d;
  }
  const float rstd = 1.0f / sqrtf(var_sum / 384.0f + 1e-12f);
  float sum_sq = 0.0f;
  for (int j = 0; j < H; j++) {
    const float v = (x[j] - mean) * rstd * gamma[j] + beta[j];
    y[j] = v;
    sum_sq += v * v;
  }
  if (sum_sq > 0.0f) {
    const float inv_norm = 1.0f / sqrtf(sum_sq);
    for (int j = 0; j < H; j++) y[j] = y[j] * inv_norm;
  }
}

void launch_cls(const ClsArgs& p, int stage, hipStream_t st) {
  if (stage == 0) hipLaunchKernelGGL(gather_cls_kernel, dim3(p.B), dim3(128), 0, st, p);
  else if (stage == 1) hipLaunchKernelGGL(cls_attention_kernel, dim3(p.B, 12), dim3(64), 0, st, p);
}

void launch_final_ln_l2(int B, const float* src, const float* gamma, const float* beta, float* out, hipStream_t st) {
  hipLaunchKernelGGL(final_ln_l2_kernel, dim3((B + 63) / 64), dim3(64), 0, st, B, src, gamma, beta, out);
}

// fills a u32 buffer (row-absmax initial values, bits of 1e-8f)
__global__ void fill_u32_kernel(uint32_t* dst, int n, uint32_t v) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = v;
}
void launch_fill_u32(uint32_t* dst, int n, uint32_t v, hipStream_t st) {
  if (n > 0) hipLaunchKernelGGL(fill_u32_kernel, dim3((n + 255) / 256), dim3(256), 0, st, dst, n, v);
}

// exact GELU elementwise (test hook for exhaustive checks)
__global__ void gelu_map_kernel(const float* x, float* y, size_t n) {
  __shared__ uint64_t sTab[32];
  load_exp_tab(sTab);
  __syncthreads();
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) y[i] = gelu_exact(x[i], sTab);
}
void launch_gelu_map(const float* x, float* y, size_t n, hipStream_t st) {
  if (n > 0) hipLaunchKernelGGL(gelu_map_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, y, n);
}

}  // namespace aek
