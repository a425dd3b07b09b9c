// Small-M projection GEMM for gfx950 (M <= 256): the weight-streaming regime,
// where the kernel is bound by HBM reads of w[N,K] rather than by MFMA.
//
// Work split: a workgroup (4 waves) owns 128 weight rows and one of `splits`
// contiguous K ranges.  Each wave owns 32 of those rows as two 16-row
// fragments (for a packed gated weight: the 16 gate rows and the matching 16
// up rows, which so meet in one lane) and streams them straight from HBM
// into registers in the v_mfma_f32_16x16x32_bf16 operand layout: the weight
// is read once and never staged.  The activations x[0:M, k-slab] are shared
// by the 4 waves through an LDS double buffer.
// Split-K: with splits > 1 every workgroup writes its f32 partial tile to the
// workspace slice of its split, and the last workgroup to finish a tile (an
// arrival counter per tile) sums the slices in split order -- deterministic
// -- applies the epilogue and re-arms the counter for the next call.
#pragma once

#include "common.hpp"

namespace sys1 {

__device__ __forceinline__ f32x4 mfma16(const i32x4& a, const i32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

constexpr int kSkinnyRows = 128;  // weight rows per workgroup
constexpr int kSkinnyThreads = 256;

template <int MB16>
struct SkinnyShape {
  static constexpr int Mp = 16 * MB16;        // padded token rows
  static constexpr int KS = MB16 >= 16 ? 64 : 128;  // k-slab per LDS stage
  static constexpr int KC = KS / 8;           // 16-byte chunks per row per slab
  static constexpr int KSTEPS = KS / 32;      // MFMA k-steps per slab
  static constexpr int XP = Mp + 1;           // chunk pitch in 16-byte units
  static constexpr int XL = Mp * KC / kSkinnyThreads;  // x loads per thread per slab
  static constexpr int kLdsUnits = KC * XP;
  static_assert(Mp * KC % kSkinnyThreads == 0, "x slab must split evenly");
  static_assert(2 * kLdsUnits * 16 <= 160 * 1024, "LDS budget");
};

template <int MB16, int EPI>
__global__ __launch_bounds__(kSkinnyThreads) void gemm_skinny_kernel(GemmArgs a) {
  using S = SkinnyShape<MB16>;
  __shared__ i32x4 lds[2][S::kLdsUnits];
  __shared__ int last_flag;

  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int tile = logical / a.splits;
  const int split = logical % a.splits;
  const int n0 = tile * kSkinnyRows;
  const int nslab = (a.K + S::KS - 1) / S::KS;
  const int s_begin = (int)((int64_t)split * nslab / a.splits);
  const int s_end = (int)((int64_t)(split + 1) * nslab / a.splits);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l16 = lane & 15;
  const int lk = lane >> 4;  // k-group of 8 within a 32-wide MFMA step
  // Wave rows: fragment f covers rows n0 + 32*wave + 16*f + [0,16).
  const int rbase = n0 + 32 * wave;
  const __bf16* wrow[2];
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    const int row = min(rbase + 16 * f + l16, a.N - 1);
    wrow[f] = a.w + (int64_t)row * a.ldw + lk * 8;
  }

  // x slab loads: thread covers chunk c of rows xr0 + p * (256 / KC).
  const int c = tid % S::KC;
  const int xr0 = tid / S::KC;
  const __bf16* xrow[S::XL];
#pragma unroll
  for (int p = 0; p < S::XL; ++p) {
    const int row = min(xr0 + p * (kSkinnyThreads / S::KC), a.M - 1);
    xrow[p] = a.x + (int64_t)row * a.ldx + c * 8;
  }

  i32x4 xr[S::XL];
  i32x4 wcur[2][S::KSTEPS], wnext[2][S::KSTEPS];
  auto load_x = [&](int slab) {
    const int k = slab * S::KS + c * 8;
    const bool ok = k < a.K;
#pragma unroll
    for (int p = 0; p < S::XL; ++p)
      xr[p] = ok ? *reinterpret_cast<const i32x4*>(xrow[p] + slab * S::KS) : i32x4{0, 0, 0, 0};
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int p = 0; p < S::XL; ++p) lds[buf][c * S::XP + xr0 + p * (kSkinnyThreads / S::KC)] = xr[p];
  };
  auto load_w = [&](i32x4 (&dst)[2][S::KSTEPS], int slab) {
#pragma unroll
    for (int ks = 0; ks < S::KSTEPS; ++ks) {
      const int k = slab * S::KS + ks * 32;
      const bool ok = k + lk * 8 < a.K;
#pragma unroll
      for (int f = 0; f < 2; ++f)
        dst[f][ks] = ok ? *reinterpret_cast<const i32x4*>(wrow[f] + k) : i32x4{0, 0, 0, 0};
    }
  };

  f32x4 acc[2][MB16];
#pragma unroll
  for (int f = 0; f < 2; ++f)
#pragma unroll
    for (int j = 0; j < MB16; ++j) acc[f][j] = f32x4{0, 0, 0, 0};

  if (s_begin < s_end) {
    load_x(s_begin);
    load_w(wcur, s_begin);
    store_x(0);
    __syncthreads();
    for (int slab = s_begin; slab < s_end; ++slab) {
      const int buf = (slab - s_begin) & 1;
      const bool more = slab + 1 < s_end;
      if (more) {
        load_x(slab + 1);
        load_w(wnext, slab + 1);
      }
      const i32x4* lx = lds[buf] + l16;
#pragma unroll
      for (int ks = 0; ks < S::KSTEPS; ++ks) {
        const int k0 = ks * 4 + lk;
#pragma unroll
        for (int j = 0; j < MB16; ++j) {
          const i32x4 xf = lx[k0 * S::XP + j * 16];
          acc[0][j] = mfma16(wcur[0][ks], xf, acc[0][j]);
          acc[1][j] = mfma16(wcur[1][ks], xf, acc[1][j]);
        }
      }
      if (more) {
        store_x(buf ^ 1);
#pragma unroll
        for (int f = 0; f < 2; ++f)
#pragma unroll
          for (int ks = 0; ks < S::KSTEPS; ++ks) wcur[f][ks] = wnext[f][ks];
      }
      __syncthreads();
    }
  }

  if (a.splits > 1) {
    // Partials in lane-native order: slice (split, tile), then (wave, f, j, lane).
    constexpr int kTileFloats4 = 4 * 2 * MB16 * 64;
    const int tiles = (a.N + kSkinnyRows - 1) / kSkinnyRows;
    f32x4* ws = reinterpret_cast<f32x4*>(a.ws);
    f32x4* mine = ws + ((int64_t)split * tiles + tile) * kTileFloats4 + wave * 2 * MB16 * 64 + lane;
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
      for (int j = 0; j < MB16; ++j) mine[(f * MB16 + j) * 64] = acc[f][j];
    __threadfence();
    __syncthreads();
    if (tid == 0) {
      const unsigned prev = __hip_atomic_fetch_add(a.counters + tile, 1u, __ATOMIC_ACQ_REL,
                                                   __HIP_MEMORY_SCOPE_AGENT);
      last_flag = prev == (unsigned)(a.splits - 1);
    }
    __syncthreads();
    if (!last_flag) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    const f32x4* base = ws + (int64_t)tile * kTileFloats4 + wave * 2 * MB16 * 64 + lane;
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
      for (int j = 0; j < MB16; ++j) {
        f32x4 s = f32x4{0, 0, 0, 0};
        for (int sp = 0; sp < a.splits; ++sp)
          s += __builtin_nontemporal_load(base + (int64_t)sp * tiles * kTileFloats4 + (f * MB16 + j) * 64);
        acc[f][j] = s;
      }
    if (tid == 0) __hip_atomic_store(a.counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // Epilogue.  Lane holds, per fragment f and token block j: token
  // m = 16j + lane%16, features rbase + 16f + 4*(lane/16) + [0..3].
  const int nq = 4 * lk;
#pragma unroll
  for (int j = 0; j < MB16; ++j) {
    const int m = j * 16 + l16;
    if (m >= a.M) continue;
    __bf16* yrow = a.y + (int64_t)m * a.ldy;
    if constexpr (epi_gated(EPI)) {
      // Fragment 0 holds gate rows, fragment 1 the matching up rows.
      const int n = rbase / 2 + nq;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = epi_gate<EPI>(acc[0][j][e], acc[1][j][e]);
      if (n < a.Nout) store4(yrow + n, v, a.Nout - n);
    } else {
      const __bf16* rrow = epi_has_resid<EPI>() ? a.resid + (int64_t)m * a.ldr : nullptr;
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const int n = rbase + 16 * f + nq;
        if (n >= a.Nout) continue;
        const int valid = a.Nout - n;
        float b[4] = {0, 0, 0, 0}, r[4] = {0, 0, 0, 0}, v[4];
        if constexpr (epi_has_bias<EPI>()) load4(a.bias + n, b, valid);
        if constexpr (epi_has_resid<EPI>()) load4(rrow + n, r, valid);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = epi_apply<EPI>(acc[f][j][e], b[e], r[e]);
        store4(yrow + n, v, valid);
      }
    }
  }
}

}  // namespace sys1
