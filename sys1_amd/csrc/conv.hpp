// DeltaNet causal conv + SiLU applied in place to a projection already in
// HBM (the two-pass form of the in_proj with conv; the fused form is the
// GEMM's conv epilogue).  Same arithmetic as that epilogue: taps over the
// bf16 projection accumulated in f32, taps before a sequence start reading
// zeros, SiLU with the hardware exp and reciprocal, rounded once
// (src/archs/qwen35_text.rs:632-650; src/kernels/qwen35.cu:3-29).
//
// In place and parallel over rows: rows are cut into segments of S; a first
// kernel saves the kConvHalo rows before every segment start, then each
// thread walks one segment of one channel pair top to bottom, keeping the
// last kConvHalo inputs in registers, so no thread reads a row another
// thread has already overwritten.
#pragma once

#include "common.hpp"

namespace sys1 {

// Channels per thread: 8 (one 16-byte access per row).
constexpr int kConvVec = 8;
constexpr int kConvChunk = 16;

// halo[s][h][c] = y[s*S - kConvHalo + h][c] for segments s >= 1, c < C.
__global__ __launch_bounds__(256) void conv_halo_kernel(const __bf16* __restrict__ y, int64_t ldy, int M, int C,
                                                        int S, __bf16* __restrict__ halo) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int vecs = C / kConvVec;
  const int64_t row = idx / vecs;  // halo row: segment row / kConvHalo + 1, tap row % kConvHalo
  const int c = (int)(idx % vecs) * kConvVec;
  const int64_t seg = row / kConvHalo + 1;
  const int h = (int)(row % kConvHalo);
  if (seg * S >= M) return;
  const int64_t r = seg * S - kConvHalo + h;
  *reinterpret_cast<bf16x8*>(halo + (seg * kConvHalo + h) * (int64_t)C + c) =
      *reinterpret_cast<const bf16x8*>(y + r * ldy + c);
}

// Rows are walked in chunks of kConvChunk: a chunk's loads are all issued
// before any of its stores, so a thread keeps kConvChunk loads in flight
// instead of serialising each row's load behind the previous row's store.
__global__ __launch_bounds__(256) void conv_silu_inplace_kernel(__bf16* __restrict__ y, int64_t ldy, int M, int C,
                                                                int S, const __bf16* __restrict__ halo,
                                                                const __bf16* __restrict__ conv_w,
                                                                const int* __restrict__ pos) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int vecs = C / kConvVec;
  const int64_t seg = idx / vecs;
  const int c = (int)(idx % vecs) * kConvVec;
  const int64_t r0 = seg * S;
  if (r0 >= M) return;
  float w[kConvVec][kConvTaps];  // taps oldest first
#pragma unroll
  for (int v = 0; v < kConvVec; v += 2) {
    const bf16x8 t8 = *reinterpret_cast<const bf16x8*>(conv_w + (int64_t)(c + v) * kConvTaps);
#pragma unroll
    for (int q = 0; q < kConvTaps; ++q) {
      w[v][q] = to_f32(t8[q]);
      w[v + 1][q] = to_f32(t8[kConvTaps + q]);
    }
  }
  float win[kConvHalo][kConvVec];  // win[kConvHalo - t] = input of row r - t
#pragma unroll
  for (int h = 0; h < kConvHalo; ++h) {
    bf16x8 hv = {};
    if (seg > 0) hv = *reinterpret_cast<const bf16x8*>(halo + (seg * kConvHalo + h) * (int64_t)C + c);
#pragma unroll
    for (int v = 0; v < kConvVec; ++v) win[h][v] = to_f32(hv[v]);
  }
  const int64_t r1 = min<int64_t>(r0 + S, M);
  for (int64_t rc = r0; rc < r1; rc += kConvChunk) {
    bf16x8 in[kConvChunk];
    int ps[kConvChunk];
#pragma unroll
    for (int q = 0; q < kConvChunk; ++q) {
      const int64_t r = rc + q;
      if (r < r1) {
        in[q] = *reinterpret_cast<const bf16x8*>(y + r * ldy + c);
        ps[q] = pos[r];
      } else {
        in[q] = bf16x8{};
        ps[q] = 0;
      }
    }
#pragma unroll
    for (int q = 0; q < kConvChunk; ++q) {
      const int64_t r = rc + q;
      // A row at least kConvTaps - 1 positions into its sequence uses every
      // tap (the common case; the row, and so the branch, is the same for
      // the whole wave); the rows before it mask the taps that reach back
      // past the sequence start.  Both add the same terms in the same order.
      const bool full = ps[q] >= kConvTaps - 1;
      bf16x8 o;
#pragma unroll
      for (int v = 0; v < kConvVec; ++v) {
        const float cur = to_f32(in[q][v]);
        float acc = 0.0f;
        if (full) {
#pragma unroll
          for (int t = kConvTaps - 1; t >= 0; --t)
            acc = fmaf(t == 0 ? cur : win[kConvHalo - t][v], w[v][kConvTaps - 1 - t], acc);
        } else {
#pragma unroll
          for (int t = kConvTaps - 1; t >= 0; --t) {
            const float xin = t == 0 ? cur : win[kConvHalo - t][v];
            const float keep = ps[q] >= t ? 1.0f : 0.0f;
            acc = fmaf(xin * keep, w[v][kConvTaps - 1 - t], acc);
          }
        }
#pragma unroll
        for (int h = 0; h + 1 < kConvHalo; ++h) win[h][v] = win[h + 1][v];
        win[kConvHalo - 1][v] = cur;
        o[v] = to_bf16(silu(acc));
      }
      if (r < r1) *reinterpret_cast<bf16x8*>(y + r * ldy + c) = o;
    }
  }
}

}  // namespace sys1
