// Skinny-M projection for gfx950: y[M,N] = epi(x[M,K] . w[N,K]^T) for a
// few hundred packed tokens at most, on v_mfma_f32_16x16x32_bf16.
//
// The small-M regime is a weight stream: every weight byte is read once and
// used for M outputs.  Up to ~32 MB of weight the stream is short next to
// the latency of a memory round trip, so this kernel is built to need as
// few dependent round trips as possible and no cross-workgroup fix-up:
//   - workgroup b owns one BM x BN output tile (BM = 16 FM rows, BN = 16 FN
//     columns; tile rows vary fastest over b, so neighbouring workgroups
//     share their weight rows) over the whole K;
//   - its NW waves split K into equal contiguous ranges of 32-wide k-steps
//     and each loads its weight and activation fragments straight from
//     memory into registers (no LDS staging), U k-steps per load group,
//     double-buffered, so a wave's whole share is usually in flight at once;
//   - the waves' f32 partial tiles are summed in LDS in wave order (fixed,
//     so the result is deterministic) and the epilogue runs on the sum.
// No partials leave the workgroup, no counters, no second pass.
//
// MFMA operands: the weight block is A (16 rows n x 32 k: lane l holds row
// l % 16, k-chunk l / 16 of 8 values, one 16-byte load), the activation
// block is B (the same layout over token rows).  The 16x16 result block
// holds, in lane l, register e: feature 4 (l / 16) + e of token l % 16.
//
// Gated epilogues (GeGLU / SwiGLU) need an even FN: the packed gate/up
// layout puts 16 gate rows and then the 16 matching up rows in each 32-row
// group, i.e. in the workgroup's blocks 2g and 2g + 1.
#pragma once
#define SYS1_SKINNY_HPP

#include "common.hpp"

namespace sys1 {

__device__ __forceinline__ f32x4 mfma16(const i32x4& a, const i32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}

template <int FM, int FN, int NW>
struct SkinnyShape {
  static constexpr int BM = FM * 16;
  static constexpr int BN = FN * 16;
  static constexpr int kRowF32 = BN + 4;  // LDS row of one wave's partial (16-byte aligned, padded)
  static constexpr int kLdsBytes = NW * BM * kRowF32 * 4;
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget of one gfx950 CU");
};

template <int FM, int FN, int NW, int U, int EPI>
__global__ __launch_bounds__(NW * 64) void skinny_kernel(GemmArgs a) {
  using S = SkinnyShape<FM, FN, NW>;
  constexpr int BM = S::BM, BN = S::BN;
  constexpr int E = epi_base(EPI);
  constexpr int NORM = epi_norm(EPI);
  constexpr bool kGated = epi_gated(E);
  static_assert(!kGated || FN % 2 == 0, "gated epilogues: whole 32-row gate/up groups per workgroup");
  static_assert(E != kEpiRopeQkv && E != kEpiConvSilu, "RoPE and conv epilogues run on the tile kernels");
  __shared__ __attribute__((aligned(16))) float red[NW * BM * S::kRowF32];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tiles_m = (a.M + BM - 1) / BM;
  const int m0 = (int)(blockIdx.x % tiles_m) * BM;
  const int n0 = (int)(blockIdx.x / tiles_m) * BN;
  const int r16 = lane & 15, q = lane >> 4;
  const int ksteps = (a.K + 31) / 32;
  const int s0 = wave * ksteps / NW, s1 = (wave + 1) * ksteps / NW;
  const rsrc_t xr = make_rsrc_uniform(a.x, 0x7ffffff0);
  const rsrc_t wr = make_rsrc_uniform(a.w, 0x7ffffff0);
  // Byte offsets of this lane's rows at k-chunk q of k-step 0 (rows past M
  // or N read the last row: computed, never stored).
  unsigned xo[FM], wo[FN];
#pragma unroll
  for (int j = 0; j < FM; ++j) xo[j] = (unsigned)((int64_t)min(m0 + j * 16 + r16, a.M - 1) * a.ldx * 2 + q * 16);
#pragma unroll
  for (int i = 0; i < FN; ++i) {
    const int n = min(n0 + i * 16 + r16, a.N - 1);
    wo[i] = a.w_kt ? (unsigned)((n / kBlkRows) * a.w_kt * kBlkBytes + (n % kBlkRows) * (kBlkK * 2) + q * 16)
                   : (unsigned)((int64_t)n * a.ldw * 2 + q * 16);
  }
  // Byte offset of k-step st (32 k values) from k = 0: 64 bytes of a
  // row-major weight row, or for the blocked layout half of a 4 KB block.
  auto wstep = [&](int st) { return a.w_kt ? (st >> 1) * kBlkBytes + (st & 1) * 64 : st * 64; };

  f32x4 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // Output vectors (8 columns of one row) per thread in the epilogue below.
  constexpr int kOutCols = kGated ? BN / 2 : BN;
  constexpr int kVecs = kOutCols / 8;
  const int out_n0 = kGated ? n0 / 2 : n0;
  // When every thread has at most one output vector, its residual is
  // loaded now, before the k-loop: it depends on nothing the kernel
  // computes, and the epilogue then does not wait a memory round trip for
  // it.  (The thread reads exactly the elements it later writes, so y may
  // alias the residual.)
  // The bias (bias epilogues) likewise.
  constexpr bool kOnePerThread = !kGated && BM * kVecs <= NW * 64;
  constexpr bool kResPre = epi_has_resid<E>() && kOnePerThread;
  constexpr bool kBiasPre = epi_has_bias<E>() && kOnePerThread;
  bf16x8 res_pre = {}, bias_pre = {};
  if constexpr (kResPre || kBiasPre) {
    const int t = threadIdx.x;
    const int m = m0 + t / kVecs, n = out_n0 + (t % kVecs) * 8;
    if (t < BM * kVecs && m < a.M && n < a.Nout) {
      if constexpr (kResPre) res_pre = load8_bf16(a.resid + (int64_t)m * a.ldr + n, a.Nout - n);
      if constexpr (kBiasPre) bias_pre = load8_bf16(a.bias + n, a.Nout - n);
    }
  }
  // The pre-norm epilogues' row statistics and column sums (written by
  // the statistics pass before this launch), likewise.
  constexpr bool kNormPre = NORM != kNormNone && kOnePerThread;
  float rs_pre = 0.0f, mu_pre = 0.0f, cs_pre[kNormPre && NORM == kNormLayer ? 8 : 1] = {};
  if constexpr (kNormPre) {
    const int t = threadIdx.x;
    const int m = min(m0 + t / kVecs, a.M - 1), c0 = (t % kVecs) * 8;
    rs_pre = a.stats[2 * (int64_t)m + 1];
    if constexpr (NORM == kNormLayer) {
      mu_pre = a.stats[2 * (int64_t)m];
      if (n0 + c0 + 8 <= a.N) {  // two 16-byte reads (kNormPre implies not gated)
        const f32x4 c0v = *reinterpret_cast<const f32x4*>(a.colsum + n0 + c0);
        const f32x4 c1v = *reinterpret_cast<const f32x4*>(a.colsum + n0 + c0 + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          cs_pre[e] = c0v[e];
          cs_pre[4 + e] = c1v[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) cs_pre[e] = a.colsum[min(n0 + c0 + e, a.N - 1)];
      }
    }
  }

  // Two register buffers of U k-steps each: one in flight while the other
  // feeds the MFMAs.  A k-chunk at or past K (or a k-step past the wave's
  // range) reads zeros through an out-of-range offset.
  i32x4 bx[2][U][FM], bw[2][U][FN];
  auto load = [&](int b, int s) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int st = s + u;
      const bool ok = st < s1 && st * 32 + q * 8 < a.K;
      const int sc = min(st, s1 - 1);
      const int so = __builtin_amdgcn_readfirstlane(sc * 64);
      const int sw = __builtin_amdgcn_readfirstlane(wstep(sc));
#pragma unroll
      for (int i = 0; i < FN; ++i)
        bw[b][u][i] = __builtin_amdgcn_raw_buffer_load_b128(wr, ok ? (int)wo[i] : (int)kOutOfRange, sw, 0);
#pragma unroll
      for (int j = 0; j < FM; ++j)
        bx[b][u][j] = __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? (int)xo[j] : (int)kOutOfRange, so, 0);
    }
  };
  auto compute = [&](int b) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = mfma16(bw[b][u][i], bx[b][u][j], acc[i][j]);
  };
  if (s0 < s1) {
    load(0, s0);
    int s = s0;
    for (; s + U < s1; s += 2 * U) {
      load(1, s + U);
      compute(0);
      if (s + 2 * U < s1) load(0, s + 2 * U);
      compute(1);
    }
    if (s < s1) compute(0);
  }

  // Partials to LDS: wave w's block (i, j) lands at rows 16 j + l % 16,
  // columns 16 i + 4 (l / 16) .. + 3 of its [BM][kRowF32] slab.
  float* mine = red + wave * BM * S::kRowF32;
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
      *reinterpret_cast<f32x4*>(mine + (j * 16 + r16) * S::kRowF32 + i * 16 + 4 * q) = acc[i][j];
  __syncthreads();

  // Epilogue: each thread takes 8 consecutive output columns of one row,
  // sums the waves' partials in wave order, applies the epilogue in the
  // reference's rounding order and stores 16 bytes.
  for (int t = threadIdx.x; t < BM * kVecs; t += NW * 64) {
    const int r = t / kVecs, c0 = (t % kVecs) * 8;
    const int m = m0 + r;
    if (m >= a.M) continue;
    const int n = out_n0 + c0;
    // partial-slab column of the output column (gated: the gate block of
    // its 32-row group; the up block is 16 columns further)
    const int pc = kGated ? (c0 / 16) * 32 + c0 % 16 : c0;
    if (n >= a.Nout) continue;
    const int valid = a.Nout - n;
    float v[8], g[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = g[e] = 0.0f;
#pragma unroll 4
    for (int ww = 0; ww < NW; ++ww) {
      const float* row = red + (ww * BM + r) * S::kRowF32;
      const f32x4 p0 = *reinterpret_cast<const f32x4*>(row + pc);
      const f32x4 p1 = *reinterpret_cast<const f32x4*>(row + pc + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] += p0[e];
        v[4 + e] += p1[e];
      }
      if constexpr (kGated) {  // the up rows of the same columns, 16 rows further
        const f32x4 u0 = *reinterpret_cast<const f32x4*>(row + pc + 16);
        const f32x4 u1 = *reinterpret_cast<const f32x4*>(row + pc + 20);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          g[e] += u0[e];
          g[4 + e] += u1[e];
        }
      }
    }
    // (for gated epilogues v holds the gate sums and g the up sums)
    if constexpr (NORM != kNormNone) {
      const float r = kNormPre ? rs_pre : a.stats[2 * (int64_t)m + 1];
      const float mu = NORM == kNormLayer ? (kNormPre ? mu_pre : a.stats[2 * (int64_t)m]) : 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if constexpr (NORM == kNormLayer) {
          const int wn = min(n0 + pc + e, a.N - 1);  // weight row of the gate (or plain) column
          const float cs = kNormPre ? cs_pre[e] : a.colsum[wn];
          v[e] = r * (v[e] - mu * cs);
          if constexpr (kGated) g[e] = r * (g[e] - mu * a.colsum[min(wn + 16, a.N - 1)]);
        } else {
          v[e] *= r;
          if constexpr (kGated) g[e] *= r;
        }
      }
    }
    bf16x8 o;
    if constexpr (kGated) {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = to_bf16(epi_gate<E>(v[e], g[e]));
    } else {
      float b[8] = {0, 0, 0, 0, 0, 0, 0, 0}, r[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      if constexpr (kBiasPre) {
#pragma unroll
        for (int e = 0; e < 8; ++e) b[e] = to_f32(bias_pre[e]);
      } else if constexpr (epi_has_bias<E>()) {
        load8(a.bias + n, b, valid);
      }
      if constexpr (kResPre) {
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = to_f32(res_pre[e]);
      } else if constexpr (epi_has_resid<E>()) {
        load8(a.resid + (int64_t)m * a.ldr + n, r, valid);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = to_bf16(epi_apply<E>(v[e], b[e], r[e]));
    }
    store8(a.y + (int64_t)m * a.ldy + n, o, valid);
  }
}

}  // namespace sys1
