// Large-M projection GEMM for gfx950: y[M,N] = x[M,K] . w[N,K]^T on
// v_mfma_f32_32x32x16_bf16, LDS double-buffered, fused epilogue.
//
// Tile:   BM x BN output tile per workgroup, BK = 64, WM x WN waves, each wave
//         owns a (BM/WM) x (BN/WN) sub-tile made of 32x32 MFMA blocks.
// Operands: both x and w are K-contiguous ("NT" GEMM).  The MFMA is issued
//         with the weight block as the A operand and the activation block as
//         B, so each lane's accumulator holds 4 runs of 4 consecutive output
//         features of one token: the epilogue stores 8-byte runs of y rows.
// LDS:    per operand, 8 k-chunks of 8 bf16 (16 B) x rows, chunk-major with a
//         one-unit pad per chunk: [k0][row + pad] in 16-byte units.  MFMA
//         operand reads (32 consecutive rows of one chunk) are contiguous and
//         the global->LDS writes (8 chunks of one row) fall in distinct banks.
// Pipeline: global loads of tile kt+1 are in flight in registers while tile
//         kt is multiplied from LDS; one barrier per k-tile.
#pragma once

#include "common.hpp"

namespace sys1 {

__device__ __forceinline__ f32x16 mfma32(const i32x4& a, const i32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <int BM, int BN, int WM, int WN>
struct TileShape {
  static constexpr int kThreads = WM * WN * 64;
  static constexpr int BK = 64;
  static constexpr int TM = BM / WM;
  static constexpr int TN = BN / WN;
  static constexpr int FM = TM / 32;
  static constexpr int FN = TN / 32;
  static constexpr int XP = BM + 1;  // k-chunk pitch, 16-byte units
  static constexpr int WP = BN + 1;
  static constexpr int XL = BM * 8 / kThreads;  // 16-byte loads per thread per k-tile
  static constexpr int WL = BN * 8 / kThreads;
  static constexpr int kLdsUnits = 8 * XP + 8 * WP;  // one buffer
  static constexpr int kLdsBytes = 2 * kLdsUnits * 16;
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be whole 32x32 blocks");
  static_assert(XL >= 1 && WL >= 1 && BM * 8 % kThreads == 0 && BN * 8 % kThreads == 0,
                "tile rows must split evenly over the threads");
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget of one gfx950 CU");
};

template <int BM, int BN, int WM, int WN, int EPI>
__global__ __launch_bounds__(WM* WN * 64) void gemm_tile_kernel(GemmArgs a) {
  using S = TileShape<BM, BN, WM, WN>;
  constexpr int T = S::kThreads;
  __shared__ i32x4 lds[2][S::kLdsUnits];

  const int tiles_n = (a.N + BN - 1) / BN;
  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int m0 = (logical / tiles_n) * BM;
  const int n0 = (logical % tiles_n) * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN;
  const int wn = wave % WN;

  // Global -> LDS assignment: thread covers chunk c of rows r0 + p * (T/8).
  const int c = tid & 7;
  const int r0 = tid >> 3;
  const __bf16* xp[S::XL];
  const __bf16* wp[S::WL];
#pragma unroll
  for (int p = 0; p < S::XL; ++p) {
    const int row = min(m0 + r0 + p * (T / 8), a.M - 1);
    xp[p] = a.x + (int64_t)row * a.ldx + c * 8;
  }
#pragma unroll
  for (int p = 0; p < S::WL; ++p) {
    const int row = min(n0 + r0 + p * (T / 8), a.N - 1);
    wp[p] = a.w + (int64_t)row * a.ldw + c * 8;
  }

  i32x4 xr[S::XL], wr[S::WL];
  auto load_tile = [&](int kt) {
    const int k = kt * S::BK + c * 8;
    const bool ok = k < a.K;
#pragma unroll
    for (int p = 0; p < S::XL; ++p)
      xr[p] = ok ? *reinterpret_cast<const i32x4*>(xp[p] + kt * S::BK) : i32x4{0, 0, 0, 0};
#pragma unroll
    for (int p = 0; p < S::WL; ++p)
      wr[p] = ok ? *reinterpret_cast<const i32x4*>(wp[p] + kt * S::BK) : i32x4{0, 0, 0, 0};
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int p = 0; p < S::XL; ++p) lds[buf][c * S::XP + r0 + p * (T / 8)] = xr[p];
#pragma unroll
    for (int p = 0; p < S::WL; ++p) lds[buf][8 * S::XP + c * S::WP + r0 + p * (T / 8)] = wr[p];
  };

  f32x16 acc[S::FN][S::FM];
#pragma unroll
  for (int i = 0; i < S::FN; ++i)
#pragma unroll
    for (int j = 0; j < S::FM; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int kt_count = (a.K + S::BK - 1) / S::BK;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  const int lrow = lane & 31;
  const int lk = lane >> 5;
  for (int kt = 0; kt < kt_count; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < kt_count;
    if (more) load_tile(kt + 1);
    const i32x4* lx = lds[buf] + wm * S::TM + lrow;
    const i32x4* lw = lds[buf] + 8 * S::XP + wn * S::TN + lrow;
#pragma unroll
    for (int ks = 0; ks < S::BK / 16; ++ks) {
      const int k0 = ks * 2 + lk;
      i32x4 xf[S::FM], wf[S::FN];
#pragma unroll
      for (int i = 0; i < S::FM; ++i) xf[i] = lx[k0 * S::XP + i * 32];
#pragma unroll
      for (int i = 0; i < S::FN; ++i) wf[i] = lw[k0 * S::WP + i * 32];
#pragma unroll
      for (int i = 0; i < S::FN; ++i)
#pragma unroll
        for (int j = 0; j < S::FM; ++j) acc[i][j] = mfma32(wf[i], xf[j], acc[i][j]);
    }
    if (more) store_tile(buf ^ 1);
    __syncthreads();
  }

  // Epilogue.  Lane holds, for block (i, j): token m = lane%32 of the block,
  // features 8g + 4*(lane/32) + [0..3] for g = 0..3.
  const int nq = 4 * lk;
#pragma unroll
  for (int j = 0; j < S::FM; ++j) {
    const int m = m0 + wm * S::TM + j * 32 + lrow;
    if (m >= a.M) continue;
    __bf16* yrow = a.y + (int64_t)m * a.ldy;
    if constexpr (epi_gated(EPI)) {
#pragma unroll
      for (int i = 0; i < S::FN; i += 2) {
        // Packed rows n0 + wn*TN + i*32 .. +64 are 32 gate rows then 32 up rows
        // of output columns (that base)/2 .. +32.
        const int ob = (n0 + wn * S::TN + i * 32) / 2;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = ob + 8 * g + nq;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = epi_gate<EPI>(acc[i][j][4 * g + e], acc[i + 1][j][4 * g + e]);
          if (n < a.Nout) store4(yrow + n, v, a.Nout - n);
        }
      }
    } else {
      const __bf16* rrow = epi_has_resid<EPI>() ? a.resid + (int64_t)m * a.ldr : nullptr;
#pragma unroll
      for (int i = 0; i < S::FN; ++i) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0 + wn * S::TN + i * 32 + 8 * g + nq;
          if (n >= a.Nout) continue;
          const int valid = a.Nout - n;
          float b[4] = {0, 0, 0, 0}, r[4] = {0, 0, 0, 0}, v[4];
          if constexpr (epi_has_bias<EPI>()) load4(a.bias + n, b, valid);
          if constexpr (epi_has_resid<EPI>()) load4(rrow + n, r, valid);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = epi_apply<EPI>(acc[i][j][4 * g + e], b[e], r[e]);
          store4(yrow + n, v, valid);
        }
      }
    }
  }
}

}  // namespace sys1
