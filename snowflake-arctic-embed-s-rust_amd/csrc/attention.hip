// attention.hip -- varlen multi-head attention (head_dim 32) and the layer-11
// [CLS]-only attention, both in the reference's exact scalar evaluation order.
#include <hip/hip_runtime.h>

#include "device_common.hpp"
#include "kernels.hpp"

namespace aek {

// ---------------------------------------------------------------------------
// Varlen attention, head_dim 32, bit-exact with the reference's scalar path
// (src/model.rs:663-694 with compute_scores_head32 / softmax_inplace /
// weighted_sum_head32 scalar branches, src/simd_math.rs:1461-1821):
//   s_t  = (sum_{i=0..31, in order} q_i*k_t,i) * (1/sqrt(32))
//   e_t  = expf(s_t - max_t s_t)            (glibc expf, restated above)
//   sum  = sum_{t in order} e_t ; inv = 1/sum ; p_t = e_t * inv
//   ctx_d = sum_{t in order} p_t * v_t,d
// every sum left to right with separately rounded products.
//
// WG (tile, head) owns kAttnQ queries of one sequence.  Scores for all keys of
// the sequence stay in LDS (row pitch = padded max length); the score, exp and
// PV phases use all 256 lanes, only the in-order softmax denominator is one
// lane per query.  tile_start[b] = sum_{b'<b} ceil(L_b'/kAttnQ) is built on the
// device from cu_seqlens.  Also folds the SmoothQuant row absmax of the output
// (|ctx_j * inv_smooth_j|) into `rowmax` (atomicMax on non-negative f32 bits),
// which the attn_out GEMM prologue consumes.
// ---------------------------------------------------------------------------
constexpr int kAttnQ = 32;     // queries per workgroup
constexpr int kKeyChunk = 64;  // keys per K/V staging chunk
constexpr int kKPitch = 36;    // K chunk row pitch (floats): conflict-free 16-byte reads

__global__ __launch_bounds__(256) void tile_starts_kernel(const int* cu, int B, int* tile_start) {
  __shared__ int part[256];
  const int tid = threadIdx.x;
  const int per = (B + 255) / 256;
  const int b0 = min(B, tid * per), b1 = min(B, b0 + per);
  int s = 0;
  for (int b = b0; b < b1; b++) s += (cu[b + 1] - cu[b] + kAttnQ - 1) / kAttnQ;
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
    acc += (cu[b + 1] - cu[b] + kAttnQ - 1) / kAttnQ;
  }
  if (b1 == B && b0 < b1) tile_start[B] = acc;
  if (B == 0 && tid == 0) tile_start[0] = 0;
}

// dynamic LDS: S[kAttnQ][s_pitch] scores/probabilities, then K/V chunk, Q tile
__global__ __launch_bounds__(256) void attention_kernel(AttnArgs p) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  __shared__ float s_inv[kAttnQ];
  const int tile = blockIdx.x, h = blockIdx.y;
  if (tile >= p.tile_start[p.B]) return;
  int lo = 0, hi = p.B - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (p.tile_start[mid] <= tile) lo = mid; else hi = mid - 1;
  }
  const int b = lo;
  const int s0 = p.cu[b];
  const int L = min(p.cu[b + 1] - s0, p.s_pitch - 4);  // the host sizes s_pitch >= L + 4
  const int q0 = (tile - p.tile_start[b]) * kAttnQ;
  const int nq = min(kAttnQ, L - q0);
  const int pitch = p.s_pitch;
  float* S = smem;                                   // [kAttnQ][pitch]
  float* KV = smem + kAttnQ * pitch;                 // [kKeyChunk][kKPitch]
  float* Qs = KV + kKeyChunk * kKPitch;              // [kAttnQ][32]
  const int tid = threadIdx.x;
  const ExpTab tb = exp_tab_regs();
  {  // Q tile (rows past the segment are clamped; their results are never stored)
    const int r = tid >> 3, c4 = tid & 7;
    const int qr = min(q0 + r, L - 1);
    *reinterpret_cast<float4*>(&Qs[r * 32 + c4 * 4]) =
        *reinterpret_cast<const float4*>(p.qkv + (size_t)(s0 + qr) * HQKV + h * 32 + c4 * 4);
  }

  // phase 1: scores.  thread -> 2 queries (held in registers) x 4 keys of each
  // 64-key chunk: 8 independent dot chains, each summed in order i = 0..31
  // (dot32_f32 scalar branch: separately rounded products, sequential adds).
  // Keys kq + 16j: the 4 rows one wave reads per instruction fall in distinct
  // LDS bank groups.
  const int qa = 2 * (tid & 15), kq = tid >> 4;
  __syncthreads();
  float qv0[32], qv1[32];
#pragma unroll
  for (int c = 0; c < 32; c += 4) {
    const float4 a = *reinterpret_cast<const float4*>(&Qs[qa * 32 + c]);
    const float4 bq = *reinterpret_cast<const float4*>(&Qs[(qa + 1) * 32 + c]);
    qv0[c] = a.x; qv0[c + 1] = a.y; qv0[c + 2] = a.z; qv0[c + 3] = a.w;
    qv1[c] = bq.x; qv1[c + 1] = bq.y; qv1[c + 2] = bq.z; qv1[c + 3] = bq.w;
  }
  for (int k0 = 0; k0 < L; k0 += kKeyChunk) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int idx = tid + i * 256, key = idx >> 3, c4 = idx & 7;
      const int kr = min(k0 + key, L - 1);
      *reinterpret_cast<float4*>(&KV[key * kKPitch + c4 * 4]) =
          *reinterpret_cast<const float4*>(p.qkv + (size_t)(s0 + kr) * HQKV + H + h * 32 + c4 * 4);
    }
    __syncthreads();
    float acc0[4] = {0.0f, 0.0f, 0.0f, 0.0f}, acc1[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < 32; c += 4) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float4 k = *reinterpret_cast<const float4*>(&KV[(kq + 16 * j) * kKPitch + c]);
        acc0[j] += qv0[c] * k.x;
        acc1[j] += qv1[c] * k.x;
        acc0[j] += qv0[c + 1] * k.y;
        acc1[j] += qv1[c + 1] * k.y;
        acc0[j] += qv0[c + 2] * k.z;
        acc1[j] += qv1[c + 2] * k.z;
        acc0[j] += qv0[c + 3] * k.w;
        acc1[j] += qv1[c + 3] * k.w;
      }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      if (k0 + kq + 16 * j < L) {
        S[qa * pitch + k0 + kq + 16 * j] = acc0[j] * kInvSqrtD;
        S[(qa + 1) * pitch + k0 + kq + 16 * j] = acc1[j] * kInvSqrtD;
      }
    }
  }
  __syncthreads();

  // phases 2, 3 and 5 give one wave a whole row at a time: lane l covers the
  // float4 columns 4l + 256i, so each LDS access is one contiguous run
  const int wv = tid >> 6, ln = tid & 63;
  // phase 2: row max (order-free) and phase 3: e_t = expf(s_t - max), 4 at a
  // time (a row tail past L lies in the pitch padding and is never read back
  // as a probability)
  for (int q = wv; q < kAttnQ; q += 4) {
    float* row = &S[q * pitch];
    float m = -INFINITY;
    for (int t = ln * 4; t < L; t += 256) {
      const float4 v = *reinterpret_cast<const float4*>(row + t);
      m = nanless_max(m, v.x);
      if (t + 1 < L) m = nanless_max(m, v.y);
      if (t + 2 < L) m = nanless_max(m, v.z);
      if (t + 3 < L) m = nanless_max(m, v.w);
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) m = nanless_max(m, __shfl_xor(m, off, 64));
    for (int t0 = 0; t0 < L; t0 += 256) {  // wave-uniform trip count (expf_libm needs all lanes)
      const int t = t0 + ln * 4;
      const bool in = t < L;
      float4 v = in ? *reinterpret_cast<const float4*>(row + t) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      v.x = expf_libm(v.x - m, tb);
      v.y = expf_libm(v.y - m, tb);
      v.z = expf_libm(v.z - m, tb);
      v.w = expf_libm(v.w - m, tb);
      if (in) *reinterpret_cast<float4*>(row + t) = v;
    }
  }
  __syncthreads();
  // phase 4: in-order denominator, one lane per query
  if (tid < kAttnQ) {
    const float* e = &S[tid * pitch];
    float sum = 0.0f;
    int t = 0;
    for (; t + 4 <= L; t += 4) {
      const float4 v = *reinterpret_cast<const float4*>(e + t);
      sum += v.x; sum += v.y; sum += v.z; sum += v.w;
    }
    for (; t < L; t++) sum += e[t];
    s_inv[tid] = 1.0f / sum;
  }
  __syncthreads();
  // phase 5: p_t = e_t * inv
  for (int q = wv; q < kAttnQ; q += 4) {
    float* row = &S[q * pitch];
    const float inv = s_inv[q];
    for (int t = ln * 4; t < L; t += 256) {
      float4 v = *reinterpret_cast<const float4*>(row + t);
      v.x = v.x * inv; v.y = v.y * inv; v.z = v.z * inv; v.w = v.w * inv;
      *reinterpret_cast<float4*>(row + t) = v;
    }
  }

  // phase 6: ctx_d = sum_t p_t * v_t,d in order. thread -> d (tid % 32) x 4 queries
  const int d = tid & 31, pg = tid >> 5;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int k0 = 0; k0 < L; k0 += kKeyChunk) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int idx = tid + i * 256, key = idx >> 3, c4 = idx & 7;
      const int kr = min(k0 + key, L - 1);
      *reinterpret_cast<float4*>(&KV[key * kKPitch + c4 * 4]) =
          *reinterpret_cast<const float4*>(p.qkv + (size_t)(s0 + kr) * HQKV + 2 * H + h * 32 + c4 * 4);
    }
    __syncthreads();
    const int nk = min(kKeyChunk, L - k0);
    int t = 0;
    for (; t + 4 <= nk; t += 4) {
      const float v0 = KV[t * kKPitch + d], v1 = KV[(t + 1) * kKPitch + d];
      const float v2 = KV[(t + 2) * kKPitch + d], v3 = KV[(t + 3) * kKPitch + d];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float4 pp = *reinterpret_cast<const float4*>(&S[(pg * 4 + j) * pitch + k0 + t]);
        acc[j] = acc[j] + pp.x * v0;
        acc[j] = acc[j] + pp.y * v1;
        acc[j] = acc[j] + pp.z * v2;
        acc[j] = acc[j] + pp.w * v3;
      }
    }
    for (; t < nk; t++) {
      const float v = KV[t * kKPitch + d];
#pragma unroll
      for (int j = 0; j < 4; j++) acc[j] = acc[j] + S[(pg * 4 + j) * pitch + k0 + t] * v;
    }
  }
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int q = pg * 4 + j;
    const float o = acc[j];
    if (q < nq) p.ctx[(size_t)(s0 + q0 + q) * H + h * 32 + d] = o;
    if (p.rowmax) {
      float a = q < nq ? fabsf(o * p.smooth[h * 32 + d]) : 0.0f;
#pragma unroll
      for (int off = 1; off < 32; off <<= 1) a = nanless_max(a, __shfl_xor(a, off, 64));
      if (q < nq && d == 0) atomicMax(&p.rowmax[s0 + q0 + q], __float_as_uint(a));
    }
  }
}

size_t attention_lds_bytes(int s_pitch) {
  return sizeof(float) * ((size_t)kAttnQ * s_pitch + kKeyChunk * kKPitch + kAttnQ * 32);
}

int attention_pitch(int max_len) {
  const int L = max(1, min(max_len, 512));
  return ((L + 3) / 4) * 4 + 4;
}

void launch_attention(const AttnArgs& p, int max_tiles, hipStream_t st) {
  static bool lds_raised = false;  // once per process: allow > 64 KiB of dynamic LDS
  if (!lds_raised) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(attention_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)attention_lds_bytes(attention_pitch(512)));
    lds_raised = true;
  }
  hipLaunchKernelGGL(tile_starts_kernel, dim3(1), dim3(256), 0, st, p.cu, p.B, p.tile_start);
  if (max_tiles > 0)
    hipLaunchKernelGGL(attention_kernel, dim3(max_tiles, 12), dim3(256), attention_lds_bytes(p.s_pitch), st, p);
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

// one wave per (sequence, head): the [CLS] query attends to its segment with the
// same exact scalar order as attention_kernel (src/model.rs:814-843)
__global__ __launch_bounds__(64) void cls_attention_kernel(ClsArgs p) {
  __shared__ __attribute__((aligned(16))) float S[512];
  __shared__ float s_inv;
  const int b = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int s0 = p.cu[b], L = min(p.cu[b + 1] - s0, 512);
  const ExpTab tb = exp_tab_regs();
  float q[32];
#pragma unroll
  for (int d = 0; d < 32; d += 4) {
    const float4 v = *reinterpret_cast<const float4*>(p.q_c + (size_t)b * H + h * 32 + d);
    q[d] = v.x; q[d + 1] = v.y; q[d + 2] = v.z; q[d + 3] = v.w;
  }
  float m = -INFINITY;
  for (int j = lane; j < L; j += 64) {
    const float* kr = p.kv + (size_t)(s0 + j) * 2 * H + h * 32;
    float sum = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; e += 4) {
      const float4 k = *reinterpret_cast<const float4*>(kr + e);
      sum += q[e] * k.x;
      sum += q[e + 1] * k.y;
      sum += q[e + 2] * k.z;
      sum += q[e + 3] * k.w;
    }
    const float sc = sum * kInvSqrtD;
    S[j] = sc;
    m = nanless_max(m, sc);
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) m = nanless_max(m, __shfl_xor(m, off, 64));
  __syncthreads();
  for (int j0 = 0; j0 < L; j0 += 64) {  // wave-uniform trip count (expf_libm needs all lanes)
    const int j = j0 + lane;
    const float e = expf_libm((j < L ? S[j] : 0.0f) - m, tb);
    if (j < L) S[j] = e;
  }
  __syncthreads();
  if (lane == 0) {
    float sum = 0.0f;
    for (int j = 0; j < L; j++) sum += S[j];
    s_inv = 1.0f / sum;
  }
  __syncthreads();
  const float inv = s_inv;
  for (int j = lane; j < L; j += 64) S[j] = S[j] * inv;
  __syncthreads();
  float o = 0.0f;
  if (lane < 32) {
    const float* vr = p.kv + (size_t)s0 * 2 * H + H + h * 32 + lane;
    for (int t = 0; t < L; t++) o = o + S[t] * vr[(size_t)t * 2 * H];
    p.ctx_c[(size_t)b * H + h * 32 + lane] = o;
  }
  float a = lane < 32 ? fabsf(o * p.smooth[h * 32 + lane]) : 0.0f;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) a = nanless_max(a, __shfl_xor(a, off, 64));
  if (lane == 0) atomicMax(&p.rowmax_ctx_c[b], __float_as_uint(a));
}

void launch_cls(const ClsArgs& p, int stage, hipStream_t st) {
  if (stage == 0) hipLaunchKernelGGL(gather_cls_kernel, dim3(p.B), dim3(128), 0, st, p);
  else if (stage == 1) hipLaunchKernelGGL(cls_attention_kernel, dim3(p.B, 12), dim3(64), 0, st, p);
}

}  // namespace aek
