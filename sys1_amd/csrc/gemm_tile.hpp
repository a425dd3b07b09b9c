// Large-M projection GEMM for gfx950: y[M,N] = x[M,K] . w[N,K]^T on
// v_mfma_f32_32x32x16_bf16, fused epilogue.
//
// Tile:    BM x BN output tile per workgroup, BK = 64, WM x WN waves, each wave
//          owns a (BM/WM) x (BN/WN) sub-tile made of 32x32 MFMA blocks.  The
//          MFMA takes the weight block as A and the activation block as B, so
//          a lane's accumulator holds runs of 4 consecutive output features of
//          one token: the epilogue stores 8-byte runs of y rows.
// Loads:   global -> LDS directly (global_load_lds_dwordx4, no VGPR staging).
//          One wave instruction fills 1 KB of LDS = 8 rows x 128 B; the 8
//          lanes of a row read its 128 B line (coalesced) in a permuted chunk
//          order that realises the LDS swizzle below.
// LDS:     per operand, row-major 128 B rows (64 bf16 of K); the 16-byte
//          chunk c of row r sits at position c ^ f(r), f(r) = (r ^ r/8) & 7.
//          With this f the MFMA operand reads (lanes 0-31: 32 rows of one
//          chunk, lanes 32-63: the next chunk) run without LDS bank conflicts
//          on gfx950 (SQ_LDS_BANK_CONFLICT = 0 measured; the plain r & 7 and
//          (r + r/8) & 7 swizzles measure 2-way), and the DMA writes are
//          contiguous by construction.
// Pipeline: STAGES LDS stages fed as one stream of k-tiles that runs across
//          the output tiles a persistent workgroup serves, so the next tile's
//          loads overlap the current tile's last k-tiles and its epilogue.
//          Fragments are double-buffered in registers across k-steps, and
//          the last k-step's MFMAs run after the barrier, overlapping the
//          next k-tile's first LDS reads.
#pragma once

#include "common.hpp"

namespace sys1 {

__device__ __forceinline__ f32x16 mfma32(const i32x4& a, const i32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

typedef __attribute__((address_space(3))) void lds_void;

// Raw buffer descriptor over [base, base + 2 GiB): offsets at or past
// kOutOfRange fall outside it and read as zeros.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr unsigned kOutOfRange = 0x80000000u;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7ffffff0,
                                           0x00020000);
}

// Asynchronous 16-byte-per-lane copy global -> LDS: lane i's 16 bytes (from
// byte offset `off` of the buffer) land at lds_base + 16 * i; lds_base is
// wave-uniform.
__device__ __forceinline__ void dma16(rsrc_t r, unsigned off, lds_void* lds_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds_base, 16, (int)off, 0, 0, 0);
}

// s_waitcnt vmcnt(N) with the LDS and export counters left unconstrained.
template <int N>
__device__ __forceinline__ void vm_wait() {
  __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15) | ((N >> 4) << 14));
}

// LDS row swizzle: chunk c of row r is stored at position c ^ swz(r).
template <int CPR>
__device__ __forceinline__ int lds_swz(int row) {
  constexpr int kShift = CPR == 8 ? 3 : 2;
  return (row ^ (row >> kShift)) & (CPR - 1);
}

template <int BM, int BN, int WM, int WN, int BK, int STAGES>
struct TileShape {
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int TM = BM / WM;
  static constexpr int TN = BN / WN;
  static constexpr int FM = TM / 32;
  static constexpr int FN = TN / 32;
  static constexpr int KS = BK / 16;                 // MFMA k-steps per k-tile
  static constexpr int CPR = BK / 8;                 // 16-byte chunks per row
  static constexpr int kRowBytes = BK * 2;
  static constexpr int RPI = 1024 / kRowBytes;       // rows per DMA instruction
  static constexpr int kXBytes = BM * kRowBytes;     // one stage of x
  static constexpr int kWBytes = BN * kRowBytes;
  static constexpr int kStageBytes = kXBytes + kWBytes;
  static constexpr int kStagesBytes = STAGES * kStageBytes;
  // Epilogue scratch, private to each wave: one 32-row block of its output
  // sub-tile in bf16 (TN columns; a gated tile stores TN/2).
  static constexpr int kEpiCols = TN;
  static constexpr int kEpiBytes = 32 * kEpiCols * 2;
  static constexpr int kLdsBytes = kStagesBytes + kWaves * kEpiBytes;
  static constexpr int XT = BM / RPI;                // DMA instructions per k-tile (x)
  static constexpr int WT = BN / RPI;                //                              (w)
  static constexpr int XI = (XT + kWaves - 1) / kWaves;  // per wave, rounded up
  static constexpr int WI = (WT + kWaves - 1) / kWaves;
  // When the instructions do not split evenly over the waves, the per-wave
  // outstanding-load counts differ and every wait is a full vmcnt(0).
  static constexpr bool kEven = XT % kWaves == 0 && WT % kWaves == 0;
  static constexpr int kDma = kEven ? XI + WI : 0;
  static_assert(BK == 32 || BK == 64, "k-tile of 32 or 64");
  static_assert(KS % 2 == 0, "fragment ping-pong needs an even k-step count");
  static_assert(STAGES >= 2, "at least double buffering");
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be whole 32x32 blocks");
  static_assert(BM % RPI == 0 && BN % RPI == 0, "whole DMA instructions per tile");
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget of one gfx950 CU");
  static_assert(kDma * (STAGES - 1) < 64, "vmcnt field");
};

// Persistent schedule: the grid holds at most (CUs x resident workgroups per
// CU) workgroups; workgroup b serves XCD b % 8 and walks that XCD's share
// of the tiles with stride (workgroups on the XCD).  Each XCD owns a
// contiguous range of tiles, rasterised in groups of kGroupM tile rows so the
// tiles in flight on one XCD share x row panels and w column panels in its
// L2.
struct TileWalk {
  int tiles, tiles_m, tiles_n;
  int first, count, stride;  // this workgroup's logical tiles: first + j * stride, j < count
  static constexpr int kGroupM = 4;

  __device__ TileWalk(int M, int N, int BM, int BN) {
    tiles_m = (M + BM - 1) / BM;
    tiles_n = (N + BN - 1) / BN;
    tiles = tiles_m * tiles_n;
    constexpr int kXcds = 8;
    const int grid = gridDim.x;
    const int xcd = blockIdx.x % kXcds;
    const int slot = blockIdx.x / kXcds;
    const int slots = grid / kXcds + (xcd < grid % kXcds ? 1 : 0);  // workgroups on this XCD
    const int per = tiles / kXcds, rem = tiles % kXcds;
    const int xbegin = xcd * per + min(xcd, rem);
    const int xcount = per + (xcd < rem ? 1 : 0);
    first = xbegin + slot;
    stride = slots;
    count = slot < xcount ? (xcount - slot + slots - 1) / slots : 0;
  }
  // Logical tile -> (tile row, tile column), grouped rasterisation.
  __device__ void coords(int t, int& tm, int& tn) const {
    const int group = t / (kGroupM * tiles_n);
    const int first_m = group * kGroupM;
    const int gm = min(kGroupM, tiles_m - first_m);
    const int in = t - group * kGroupM * tiles_n;
    tm = first_m + in % gm;
    tn = in / gm;
  }
};

template <int BM, int BN, int WM, int WN, int BK, int STAGES, int EPI>
__global__ __launch_bounds__(WM* WN * 64) void gemm_tile_kernel(GemmArgs a) {
  using S = TileShape<BM, BN, WM, WN, BK, STAGES>;
  __shared__ __attribute__((aligned(1024))) char lds[S::kLdsBytes];

  const TileWalk walk(a.M, a.N, BM, BN);
  if (walk.count == 0) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keep in SGPRs
  const int wm = wave / WN;
  const int wn = wave % WN;

  const int kt_count = (a.K + BK - 1) / BK;
  const int kt_full = a.K / BK;  // k-tiles with no K tail
  const int steps = walk.count * kt_count;

  // ---- DMA.  Step s of this workgroup is k-tile s % kt_count of its tile
  // s / kt_count.  Instruction i of this wave covers tile rows
  // r0 = (i * waves + wave) * RPI .. +RPI; lane -> row r0 + lane/CPR,
  // position lane%CPR, source chunk position ^ swz(row).  Loads are raw
  // buffer loads: a 32-bit per-lane offset from the tile's base (rows past M
  // / N clamp to the last row), and an offset past the buffer's range reads
  // zeros, which fills the chunks past K in a tail k-tile.
  const int lrow = lane / S::CPR, lpos = lane % S::CPR;
  auto issue = [&](int step, int stage) {
    const int j = step / kt_count;
    const int kt = step - j * kt_count;
    int tm, tn;
    walk.coords(walk.first + j * walk.stride, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    char* base = lds + stage * S::kStageBytes + wave * S::RPI * S::kRowBytes;
    const rsrc_t xr = make_rsrc(reinterpret_cast<const char*>(a.x + (int64_t)m0 * a.ldx) + kt * BK * 2);
    const rsrc_t wr = make_rsrc(reinterpret_cast<const char*>(a.w + (int64_t)n0 * a.ldw) + kt * BK * 2);
    const bool tail = kt >= kt_full;
    const int kleft = a.K - kt * BK;  // valid K elements in this tile
#pragma unroll
    for (int i = 0; i < S::XI; ++i) {
      if (!S::kEven && i * S::kWaves + wave >= S::XT) break;
      const int r = (i * S::kWaves + wave) * S::RPI + lrow;
      const int c = lpos ^ lds_swz<S::CPR>(r);
      unsigned off = (unsigned)(min(r, a.M - 1 - m0) * (int)a.ldx * 2 + c * 16);
      if (tail && c * 8 >= kleft) off = kOutOfRange;
      dma16(xr, off, (lds_void*)(base + i * S::kWaves * S::RPI * S::kRowBytes));
    }
#pragma unroll
    for (int i = 0; i < S::WI; ++i) {
      if (!S::kEven && i * S::kWaves + wave >= S::WT) break;
      const int r = (i * S::kWaves + wave) * S::RPI + lrow;
      const int c = lpos ^ lds_swz<S::CPR>(r);
      unsigned off = (unsigned)(min(r, a.N - 1 - n0) * (int)a.ldw * 2 + c * 16);
      if (tail && c * 8 >= kleft) off = kOutOfRange;
      dma16(wr, off, (lds_void*)(base + S::kXBytes + i * S::kWaves * S::RPI * S::kRowBytes));
    }
  };

  // ---- fragment addressing (byte offsets within a stage): lane reads row
  // (base + lane%32) of chunk 2*ks + lane/32.
  const int frow = lane & 31;
  const int fk = lane >> 5;
  int xrow_off[S::FM], xrow_swz[S::FM], wrow_off[S::FN], wrow_swz[S::FN];
#pragma unroll
  for (int j = 0; j < S::FM; ++j) {
    const int r = wm * S::TM + j * 32 + frow;
    xrow_off[j] = r * S::kRowBytes;
    xrow_swz[j] = lds_swz<S::CPR>(r);
  }
#pragma unroll
  for (int i = 0; i < S::FN; ++i) {
    const int r = wn * S::TN + i * 32 + frow;
    wrow_off[i] = S::kXBytes + r * S::kRowBytes;
    wrow_swz[i] = lds_swz<S::CPR>(r);
  }

  struct Frags {
    i32x4 x[S::FM];
    i32x4 w[S::FN];
  };
  auto read = [&](Frags& f, int stage, int ks) {
    const char* base = lds + stage * S::kStageBytes;
    const int c = ks * 2 + fk;
#pragma unroll
    for (int j = 0; j < S::FM; ++j)
      f.x[j] = *reinterpret_cast<const i32x4*>(base + xrow_off[j] + ((c ^ xrow_swz[j]) << 4));
#pragma unroll
    for (int i = 0; i < S::FN; ++i)
      f.w[i] = *reinterpret_cast<const i32x4*>(base + wrow_off[i] + ((c ^ wrow_swz[i]) << 4));
  };

  f32x16 acc[S::FN][S::FM];
  auto zero_acc = [&]() {
#pragma unroll
    for (int i = 0; i < S::FN; ++i)
#pragma unroll
      for (int j = 0; j < S::FM; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
  };
  zero_acc();

  auto mma = [&](const Frags& f) {
#pragma unroll
    for (int i = 0; i < S::FN; ++i)
#pragma unroll
      for (int j = 0; j < S::FM; ++j) acc[i][j] = mfma32(f.w[i], f.x[j], acc[i][j]);
  };

  // ---- epilogue of one tile, one 32-row block at a time.  Phase 1: the
  // lane's accumulators (token m = lane%32 of the block, features
  // 8g + 4*(lane/32) + [0..3]) get the register-side epilogue ops (bf16
  // rounding, bias, gelu, gating) and go to the wave's LDS scratch as bf16,
  // row-major with 16-byte chunks rotated by row.  Phase 2: 8 lanes per row
  // read back 16-byte chunks, add the residual from 16-byte loads and store
  // full 128-byte lines.
  constexpr int kOutCols = epi_gated(EPI) ? S::TN / 2 : S::TN;  // per wave
  constexpr int kC8 = kOutCols / 8;                             // 16-byte chunks per row
  static_assert(kOutCols % 8 == 0, "whole 16-byte chunks");
  char* scratch = lds + S::kStagesBytes + wave * S::kEpiBytes;
  auto sc_addr = [&](int row, int c8) -> char* {
    return scratch + row * (kOutCols * 2) + ((c8 + row) % kC8) * 16;
  };
  auto epilogue = [&](int m0, int n0) {
    const int nq = 4 * fk;
    const int out_n0 = (epi_gated(EPI) ? (n0 + wn * S::TN) / 2 : n0 + wn * S::TN);
#pragma unroll
    for (int j = 0; j < S::FM; ++j) {
      // phase 1: registers -> scratch
#pragma unroll
      for (int i = 0; i < S::FN; ++i) {
        if constexpr (epi_gated(EPI)) {
          // A 32-row block of the packed weight is 16 gate rows then the 16
          // up rows of the same 16 output columns: registers 4g+e (g = 0, 1)
          // hold gate rows, 4(g+2)+e the matching up rows.
#pragma unroll
          for (int g = 0; g < 2; ++g) {
            bf16x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              o[e] = to_bf16(epi_gate<EPI>(acc[i][j][4 * g + e], acc[i][j][4 * (g + 2) + e]));
            const int col = i * 16 + 8 * g + nq;
            *reinterpret_cast<bf16x4*>(sc_addr(frow, col / 8) + (col % 8) * 2) = o;
          }
        } else {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int col = i * 32 + 8 * g + nq;
            float b[4] = {0, 0, 0, 0};
            if constexpr (epi_has_bias<EPI>()) {
              const int n = n0 + wn * S::TN + col;
              load4(a.bias + n, b, a.Nout - n);
            }
            bf16x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = to_bf16(epi_pre<EPI>(acc[i][j][4 * g + e], b[e]));
            *reinterpret_cast<bf16x4*>(sc_addr(frow, col / 8) + (col % 8) * 2) = o;
          }
        }
      }
      // phase 2: scratch -> global, 16 bytes per lane
      const int mb = m0 + wm * S::TM + j * 32;
#pragma unroll
      for (int t = 0; t < (32 * kC8 + 63) / 64; ++t) {
        const int q = lane + 64 * t;
        if (32 * kC8 % 64 != 0 && q >= 32 * kC8) break;
        const int row = q / kC8, c8 = q % kC8;
        const int m = mb + row;
        const int n = out_n0 + c8 * 8;
        const i32x4 raw = *reinterpret_cast<const i32x4*>(sc_addr(row, c8));
        if (m < a.M && n < a.Nout) {
          const int valid = a.Nout - n;
          bf16x8 v = __builtin_bit_cast(bf16x8, raw);
          if constexpr (epi_has_resid<EPI>()) {
            float r[8];
            load8(a.resid + (int64_t)m * a.ldr + n, r, valid);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = to_bf16(to_f32(v[e]) + r[e]);
          }
          store8(a.y + (int64_t)m * a.ldy + n, v, valid);
        }
      }
    }
  };

  // ---- main loop over this workgroup's k-tile stream.  Step s lives in
  // stage s % STAGES.  The prologue requests steps 0..STAGES-1; after the
  // barrier that retires step s, step s + STAGES is requested into the stage
  // just freed -- across tile boundaries, so the next tile's first k-tiles
  // land while this tile finishes and stores.  Before that barrier step s+1
  // must have landed while s+2 .. s+STAGES-1 may still be in flight:
  // vmcnt((STAGES-2) * DMAs per step).  sched_barrier(0) pins the order
  // below: the next k-step's fragment reads are issued before the current
  // k-step's MFMAs, so LDS latency hides behind a full k-step of matrix work.
  for (int t = 0; t < STAGES; ++t)
    if (t < steps) issue(t, t);
  if (steps >= STAGES) vm_wait<(STAGES - 1) * S::kDma>();  // kDma = 0 when uneven
  else vm_wait<0>();
  __syncthreads();
  Frags f0, f1;
  read(f0, 0, 0);
  int stage = 0;
  int kt = 0, j = 0;
  for (int s = 0; s < steps; ++s) {
#pragma unroll
    for (int ks = 1; ks < S::KS; ks += 2) {
      read(f1, stage, ks);
      __builtin_amdgcn_sched_barrier(0);
      mma(f0);
      __builtin_amdgcn_sched_barrier(0);
      if (ks + 1 < S::KS) {
        read(f0, stage, ks + 1);
        __builtin_amdgcn_sched_barrier(0);
        mma(f1);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (s + 1 < steps) {
      if (s + STAGES - 1 < steps) vm_wait<(STAGES - 2) * S::kDma>();
      else vm_wait<0>();
    }
    __syncthreads();
    if (s + STAGES < steps) issue(s + STAGES, stage);
    stage = stage + 1 == STAGES ? 0 : stage + 1;
    if (s + 1 < steps) read(f0, stage, 0);
    __builtin_amdgcn_sched_barrier(0);
    mma(f1);
    __builtin_amdgcn_sched_barrier(0);
    if (++kt == kt_count) {
      int tm, tn;
      walk.coords(walk.first + j * walk.stride, tm, tn);
      epilogue(tm * BM, tn * BN);
      zero_acc();
      kt = 0;
      ++j;
    }
  }
}

}  // namespace sys1
