// Pre-norm support for the projection kernels: per-row statistics of the
// norm's input, and the load-time fold of the norm weight into the
// projection weight.
//
// A bias-free LayerNorm with weight g followed by a projection W is
//   y[m,n] = sum_k ((x[m,k] - mu_m) r_m g_k) W[n,k]
//          = r_m (sum_k x[m,k] W'[n,k] - mu_m c_n),   W' = W (.) g,  c_n = sum_k W'[n,k]
// and an RMSNorm with alpha = 1 + w is y[m,n] = r_m sum_k x[m,k] W'[n,k],
// W' = W (.) alpha.  The GEMM therefore reads the raw activations; the
// kernels below supply (mu_m, r_m) per row and W', c at load time, and the
// GEMM epilogue applies r_m (acc - mu_m c_n).
//   LayerNorm: src/archs/modernbert.rs:1005-1034 (Norm, LayerNorm::new_no_bias;
//              candle-nn 0.11.0 LayerNorm: mean, then the mean of squared
//              deviations, r = 1/sqrt(var + eps), all in f32).
//   RMSNorm:   src/archs/qwen35_text.rs:178-203 (variance = mean(x^2) in f32,
//              scale = 1/sqrt(variance + eps), alpha = 1 + weight).
#pragma once

#include "common.hpp"

namespace sys1 {

// Sum over the 64 lanes of a wave, the same order on every call.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// One wave per row: stats[2m] = mean (0 for RMSNorm), stats[2m+1] =
// 1/sqrt(var + eps).  LayerNorm takes the variance about the mean, as the
// reference does: the row is loaded once into registers (all its loads in
// flight at once; CH x 512 elements, CH chosen at launch from K), then
// reduced twice.  Rows longer than 16 x 512 take a second pass over memory.
// Requires K % 8 == 0 and 16-byte aligned rows.
template <int NORM, int CH>
__global__ __launch_bounds__(256) void row_stats_kernel(const __bf16* __restrict__ x, int64_t ldx, int M,
                                                        int K, float eps, float* __restrict__ stats) {
  constexpr int kRowChunks = CH;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * 4 + wave;
  if (m >= M) return;  // whole waves only; no barrier below
  const __bf16* row = x + m * ldx;
  float mean = 0.0f, var;
  if (K <= kRowChunks * 512) {
    bf16x8 v[kRowChunks];
#pragma unroll
    for (int c = 0; c < kRowChunks; ++c) {
      const int k = c * 512 + lane * 8;
      if (k < K) v[c] = *reinterpret_cast<const bf16x8*>(row + k);
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < kRowChunks; ++c)
      if (c * 512 + lane * 8 < K) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float f = to_f32(v[c][e]);
          s += NORM == kNormLayer ? f : f * f;
        }
      }
    s = wave_sum(s);
    if constexpr (NORM == kNormLayer) {
      mean = s / (float)K;
      float d2 = 0.0f;
#pragma unroll
      for (int c = 0; c < kRowChunks; ++c)
        if (c * 512 + lane * 8 < K) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float d = to_f32(v[c][e]) - mean;
            d2 += d * d;
          }
        }
      var = wave_sum(d2) / (float)K;
    } else {
      var = s / (float)K;
    }
  } else {
    float s = 0.0f;
    for (int k = lane * 8; k < K; k += 64 * 8) {
      const bf16x8 v = *reinterpret_cast<const bf16x8*>(row + k);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = to_f32(v[e]);
        s += NORM == kNormLayer ? f : f * f;
      }
    }
    s = wave_sum(s);
    if constexpr (NORM == kNormLayer) {
      mean = s / (float)K;
      float d2 = 0.0f;
      for (int k = lane * 8; k < K; k += 64 * 8) {
        const bf16x8 v = *reinterpret_cast<const bf16x8*>(row + k);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = to_f32(v[e]) - mean;
          d2 += d * d;
        }
      }
      var = wave_sum(d2) / (float)K;
    } else {
      var = s / (float)K;
    }
  }
  if (lane == 0) {
    stats[2 * m] = mean;
    stats[2 * m + 1] = 1.0f / sqrtf(var + eps);
  }
}

// One wave per weight row: w_out[n,k] = bf16(w[n,k] * a_k) with a = g
// (LayerNorm) or 1 + g (RMSNorm), and colsum[n] = sum_k of the rounded
// w_out[n,k] (the values the GEMM multiplies by), if colsum is non-null.
// Requires K % 8 == 0 and 16-byte aligned rows.
template <int NORM>
__global__ __launch_bounds__(256) void fold_norm_kernel(const __bf16* __restrict__ w, const float* __restrict__ g,
                                                        __bf16* __restrict__ w_out, float* __restrict__ colsum,
                                                        int N, int K) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + wave;
  if (n >= N) return;
  const __bf16* src = w + n * K;
  __bf16* dst = w_out + n * K;
  float s = 0.0f;
  for (int k = lane * 8; k < K; k += 64 * 8) {
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(src + k);
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float a = NORM == kNormRms ? 1.0f + g[k + e] : g[k + e];
      o[e] = to_bf16(to_f32(v[e]) * a);
      s += to_f32(o[e]);
    }
    *reinterpret_cast<bf16x8*>(dst + k) = o;
  }
  s = wave_sum(s);
  if (colsum && lane == 0) colsum[n] = s;
}

}  // namespace sys1
