// Projection GEMM for gfx950: y[M,N] = epi(x[M,K] . w[N,K]^T) on
// v_mfma_f32_32x32x16_bf16.  One kernel template covers both regimes:
//   - large M: MFMA-bound output tiles, one k-stream per tile;
//   - small M (the weight-streaming regime): BM = the padded token count,
//     BN = 256, with K split over workgroups so that every CU streams weight.
//
// Tile:    BM x BN output tile, BK = 64 or 32, WM x WN waves, each wave owns a
//          (BM/WM) x (BN/WN) sub-tile of 32x32 MFMA blocks.  The MFMA takes the
//          weight block as A and the activation block as B, so a lane's
//          accumulator holds runs of 4 consecutive output features of one
//          token.
// Loads:   global -> LDS directly (buffer_load ... lds, no VGPR staging).  One
//          wave instruction fills 1 KB of LDS = 8 rows x 128 B (BK = 64) or
//          16 rows x 64 B (BK = 32); the lanes of a row read its line
//          (coalesced) in a permuted chunk order that realises the LDS swizzle
//          below.  The x and w instructions of a
//          k-tile form one list dealt round-robin to the waves, so every wave
//          issues the same count and vmcnt bookkeeping stays exact.
// LDS:     per operand, row-major rows of BK bf16; the 16-byte chunk c of
//          row r sits at position c ^ f(r), f(r) = (r ^ r/8) & 7 for 128 B
//          rows ((r ^ r/4) & 3 for 64 B rows).
//          With this f the MFMA operand reads (lanes 0-31: 32 rows of one
//          chunk, lanes 32-63: the next chunk) run without LDS bank conflicts
//          on gfx950 (SQ_LDS_BANK_CONFLICT = 0 measured; the plain r & 7 and
//          (r + r/8) & 7 swizzles measure 2-way).
// Pipeline: STAGES LDS stages fed as one stream of k-tiles that runs across
//          the work items a persistent workgroup serves, so the next item's
//          loads overlap the current item's last k-tiles and its epilogue.
//          Fragments are double-buffered in registers across k-steps, and the
//          last k-step's MFMAs run after the barrier, overlapping the next
//          k-tile's first LDS reads; the freed stage's refill is issued
//          behind them (spread between them with one workgroup per CU).
// Epilogue: straight from registers: lane pairs (l, l+32) exchange halves
//          with v_permlane32_swap so that every lane stores (and reads the
//          residual as) 16 contiguous bytes; no LDS, so all of it goes to
//          pipeline stages.
// Stream-K: the weight-streaming shapes split the flattened (tile, k-tile)
//          iteration space into one equal contiguous range per workgroup, so
//          every CU streams the same share of the weight (optionally after a
//          phase of whole tiles: the hybrid schedule of TileWalk).  A range covers at
//          most a partial head segment, whole tiles, and a partial tail
//          segment; a partial segment writes its f32 accumulators to the
//          workspace (head or tail slot of its workgroup), and, per wave
//          slice of the tile, the last owner to arrive (an arrival counter
//          per tile and wave) sums the slice's partials in workgroup order --
//          deterministic whatever the arrival order -- applies the epilogue
//          to it and re-arms the counter.
#pragma once
#define SYS1_GEMM_TILE_HPP

#include <type_traits>

#include "common.hpp"

namespace sys1 {

__device__ __forceinline__ f32x16 mfma32(const i32x4& a, const i32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// LDS row swizzle: chunk c of row r is stored at position c ^ swz(r).
// Measured conflict-free for the 32-lane fragment reads on gfx950: 128-byte
// rows (BK = 64, 8 chunks) use (r ^ r/8) & 7, 64-byte rows (BK = 32, 4
// chunks) use (r ^ r/4) & 3.
template <int BK>
__device__ __forceinline__ int lds_swz(int row) {
  if constexpr (BK == 64) return (row ^ (row >> 3)) & 7;
  else return (row ^ (row >> 2)) & 3;
}

template <int BM, int BN, int WM, int WN, int STAGES, int BK_>
struct TileShape {
  // (a blocked weight's k-tile is one 4 KB block per 32 tile rows)
  static_assert(BN % kBlkRows == 0 && BK_ == kBlkK, "tiles start on weight blocks of the blocked layout");
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int BK = BK_;
  static_assert(BK == 32 || BK == 64, "k-tile of 32 or 64");
  static constexpr int TM = BM / WM;
  static constexpr int TN = BN / WN;
  static constexpr int FM = TM / 32;
  static constexpr int FN = TN / 32;
  static constexpr int KS = BK / 16;                 // MFMA k-steps per k-tile
  static constexpr int kRowBytes = BK * 2;           // 128 or 64
  static constexpr int CPR = BK / 8;                 // 16-byte chunks per row
  static constexpr int RPI = 1024 / kRowBytes;       // rows per DMA instruction (1 KB)
  static constexpr int kXBytes = BM * kRowBytes;     // one stage of x
  static constexpr int kWBytes = BN * kRowBytes;
  static constexpr int kStageBytes = kXBytes + kWBytes;
  static constexpr int kStagesBytes = STAGES * kStageBytes;
  static constexpr int kLdsBytes = kStagesBytes;
  static constexpr int XT = BM / RPI;                // DMA instructions per k-tile: x
  static constexpr int DT = (BM + BN) / RPI;         // x and w together
  static constexpr int kDma = DT / kWaves;           // per wave per k-tile
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be whole 32x32 blocks");
  static_assert(BM % RPI == 0 && BN % RPI == 0, "whole DMA instructions per tile");
  static_assert(STAGES >= 2, "at least double buffering");
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget of one gfx950 CU");
  static_assert(kDma * (STAGES - 1) < 64, "vmcnt field");
};

// A segment of a workgroup's k-tile stream: k-tiles [kt0, kt1) of one tile.
struct Segment {
  int tm, tn;     // tile coordinates
  int kt0, kt1;   // k-tile range
  int pos;        // position in this workgroup's step sequence
  int st;         // stream-phase tile index (tile - dp_tiles), -1 in the tile phase
  int spos;       // stream-phase position of its first k-tile (st * kt_count + kt0)
};

// Persistent schedule over tiles rasterised in groups of group_m tile rows
// (tiles in flight together share x row panels and w column panels in L2).
// The grid holds at most (CUs x resident workgroups per CU) workgroups G.
//   Tile phase: tiles [0, dp_tiles), each a whole segment.  Workgroup b
//     serves XCD b % 8 and walks that XCD's contiguous share of these tiles
//     with stride (workgroups on the XCD).
//   Stream phase: the k-iterations of tiles [dp_tiles, tiles) flattened,
//     T = (tiles - dp_tiles) * kt_count; workgroup g < G' = min(G, T) owns
//     [start(g), start(g+1)), start(g) = g * T / G'.  A tile split over several
//     workgroups is summed by its last arriving owner.
// dp_tiles = tiles is the plain persistent tile schedule; dp_tiles = 0 is
// pure stream-K (the weight-streaming small-M shapes); in between is the
// hybrid that runs whole rounds of tiles and spreads the last, partial round
// over every CU.
struct TileWalk {
  int tiles_m, tiles_n, kt_count, tiles, dp_tiles;
  int step_m;  // rows between tile rows: BM, or BM - halo (tile rows overlap by the halo)
  // tile phase
  int first, count, stride;
  // stream phase
  int64_t total;
  int grid, sgrid, begin, end;  // sgrid: workgroups in the stream phase
  int dp_steps;

  int group_m;

  // halo > 0: tile row tm covers rows [tm (BM - halo), + BM), so the halo
  // rows before each tile row's outputs are computed in the same tile.
  __device__ TileWalk(int M, int N, int K, int BM, int BN, int BK, int dp, int group, int halo = 0) {
    group_m = max(1, group);
    step_m = BM - halo;
    tiles_m = M <= BM ? 1 : 1 + (M - BM + step_m - 1) / step_m;
    tiles_n = (N + BN - 1) / BN;
    kt_count = (K + BK - 1) / BK;
    tiles = tiles_m * tiles_n;
    dp_tiles = min(dp, tiles);
    grid = gridDim.x;
    // Workgroups are dispatched round-robin over the 8 XCDs; a grid smaller
    // than that deals the tiles over as many groups as it has workgroups.
    const int xcds = min(8, grid);
    const int xcd = blockIdx.x % xcds;
    const int slot = blockIdx.x / xcds;
    const int slots = grid / xcds + (xcd < grid % xcds ? 1 : 0);  // workgroups on this XCD
    const int per = dp_tiles / xcds, rem = dp_tiles % xcds;
    const int xbegin = xcd * per + min(xcd, rem);
    const int xcount = per + (xcd < rem ? 1 : 0);
    first = xbegin + slot;
    stride = slots;
    count = slot < xcount ? (xcount - slot + slots - 1) / slots : 0;
    dp_steps = count * kt_count;
    total = (int64_t)(tiles - dp_tiles) * kt_count;
    // At most one workgroup per iteration, so that every stream range is
    // non-empty (the arrival count of a split tile is its owner count).
    sgrid = (int)min<int64_t>(grid, total);
    begin = (int)blockIdx.x < sgrid ? start(blockIdx.x) : 0;
    end = (int)blockIdx.x < sgrid ? start(blockIdx.x + 1) : 0;
  }
  __device__ int start(int g) const { return (int)((int64_t)g * total / sgrid); }
  __device__ int row0(int tm) const { return tm * step_m; }

  // Tile index -> coordinates (grouped raster).
  __device__ void tile_coords(int t, int& tm, int& tn) const {
    const int group = t / (group_m * tiles_n);
    const int first_m = group * group_m;
    const int gm = min(group_m, tiles_m - first_m);
    const int in = t - group * group_m * tiles_n;
    tm = first_m + in % gm;
    tn = in / gm;
  }
  __device__ int steps() const { return dp_steps + (end - begin); }
  // The segment whose first k-tile is step `pos` of this workgroup.
  __device__ Segment segment_at(int pos) const {
    Segment sg;
    if (pos < dp_steps) {
      const int j = pos / kt_count;
      tile_coords(first + j * stride, sg.tm, sg.tn);
      sg.kt0 = 0;
      sg.kt1 = kt_count;
      sg.st = -1;
      sg.spos = 0;
    } else {
      const int sp = begin + (pos - dp_steps);
      const int t = sp / kt_count;
      tile_coords(dp_tiles + t, sg.tm, sg.tn);
      sg.kt0 = sp - t * kt_count;
      sg.kt1 = min(kt_count, sg.kt0 + (end - sp));
      sg.st = t;
      sg.spos = sp;
    }
    sg.pos = pos;
    return sg;
  }
  __device__ Segment first_segment() const { return segment_at(0); }
  __device__ Segment next_segment(const Segment& sg) const {
    return segment_at(sg.pos + (sg.kt1 - sg.kt0));
  }
  __device__ bool complete(const Segment& sg) const { return sg.kt0 == 0 && sg.kt1 == kt_count; }
  // Stream phase: the workgroups whose ranges overlap stream tile st, [g_lo, g_hi].
  __device__ void tile_owners(int st, int& g_lo, int& g_hi) const {
    const int64_t lo = (int64_t)st * kt_count, hi = lo + kt_count;  // [lo, hi)
    int g = (int)(lo * sgrid / total);
    while (g > 0 && start(g) > lo) --g;
    while (start(g + 1) <= lo) ++g;
    g_lo = g;
    g = (int)((hi - 1) * sgrid / total);
    while (g > 0 && start(g) > hi - 1) --g;
    while (start(g + 1) <= hi - 1) ++g;
    g_hi = g;
  }
};

// STREAMK: stream-K schedule (the weight-streaming shapes); the large-M
// shapes compile the tile schedule only.
// OCC: resident workgroups per CU the register allocation must allow.
// PW: producer waves.  0: every wave issues its share of the refills between
// its MFMAs.  PW > 0: PW extra waves issue all of them and do nothing else,
// so a refill instruction that stalls issue while the load path drains
// stalls no matrix work.  Under stream-K the compute waves then also wait
// for their partial stores (before the arrival counter) without draining
// the refills in flight: a wave's vmcnt covers every vector memory access
// it issued, and with producer waves those are its stores alone.
template <int BM, int BN, int WM, int WN, int STAGES, int BK_, int OCC, bool STREAMK, int EPI, int PW = 0>
__global__ __launch_bounds__((WM * WN + PW) * 64)
__attribute__((amdgpu_waves_per_eu(((WM * WN + PW) * OCC + 3) / 4))) void gemm_tile_kernel(GemmArgs a) {
  using S = TileShape<BM, BN, WM, WN, STAGES, BK_>;
  constexpr int BK = S::BK;
  // Residual epilogues of producer-wave tile kernels whose LDS budget has
  // room: the producers copy each tile's residual block into LDS while its
  // k-loop runs, so the epilogue does not wait on a read from HBM.
  constexpr bool kResLds = PW > 0 && !STREAMK && epi_has_resid<epi_base(EPI)>() &&
                           (S::kLdsBytes + BM * BN * 2) * OCC <= 160 * 1024 && (BM * BN * 2 / 1024) % PW == 0;
  constexpr int kResBytes = kResLds ? BM * BN * 2 : 0;
  __shared__ __attribute__((aligned(1024))) char lds[S::kLdsBytes + kResBytes];
  char* const res_lds = lds + S::kLdsBytes;
  // (every k-tile loop needs two k-steps per tile, so that a tile's copy,
  // issued after its first barrier, lands before its last)
  const bool res_in_lds = kResLds && a.K > BK_ && a.Nout >= 8 && a.Nout % 8 == 0 && a.ldr % 8 == 0 &&
                          (reinterpret_cast<uintptr_t>(a.resid) & 15) == 0 &&
                          (int64_t)a.M * a.ldr * 2 < 0x7ffffff0ll;

  constexpr bool kConv = epi_base(EPI) == kEpiConvSilu;
  static_assert(!kConv || WM == 1, "conv epilogue: one wave row per tile");
  static_assert(PW == 0 || !kConv, "producer waves: no conv epilogue");
  const TileWalk walk(a.M, a.N, a.K, BM, BN, BK, STREAMK ? a.dp_tiles : 1 << 30, a.group_m,
                      kConv ? kConvHalo : 0);
  if (walk.steps() == 0) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keep in SGPRs
  const int wm = wave / WN;
  const int wn = wave % WN;

  // ---- DMA.  The issue cursor walks the segments in stream order.
  // Instruction u = i * waves + wave of a k-tile: u < XT covers x rows
  // RPI*u .. RPI*u + RPI-1, else w rows RPI*(u-XT) ..; either way its 1 KB
  // lands at stage offset u * 1 KB.  Lane -> row + lane/CPR, position
  // lane%CPR, source chunk position ^ swz(row).  Rows past M / N clamp to
  // the last row; chunks past K read zeros through an out-of-range buffer
  // offset.
  const int lrow = lane / S::CPR, lpos = lane % S::CPR;
  // A wave's first kXDma instructions read x, the rest w.  Row, chunk and
  // swizzle of each instruction depend only on the lane, so the per-lane
  // source offsets (row clamp included) are computed when the issue cursor
  // enters a tile; a k-tile then costs only the scalar base advance, and the
  // K-tail test runs on a tile's last, partial k-tile only.
  constexpr int kDW = PW ? PW : S::kWaves;  // waves that issue refills
  constexpr int kDma = S::DT / kDW;          // refill instructions per issuing wave per k-tile
  static_assert(S::XT % kDW == 0 && S::DT % kDW == 0, "x and w instructions deal evenly over the waves");
  static_assert(kDma * (STAGES - 1) < 64, "vmcnt field");
  constexpr int kXDma = S::XT / kDW;
  const int dwave = PW ? wave - S::kWaves : wave;
  auto dma_row = [&](int i) {
    const int u = i * kDW + dwave;
    return (i < kXDma ? u : u - S::XT) * S::RPI + lrow;
  };
  unsigned src_off[kDma];
  auto set_offsets = [&](const Segment& sg) {
    const int x_left = a.M - 1 - walk.row0(sg.tm), w_left = a.N - 1 - sg.tn * BN;
#pragma unroll
    for (int i = 0; i < kDma; ++i) {
      const int r = dma_row(i);
      const int c = lpos ^ lds_swz<BK>(r);
      const int rw = min(r, w_left);  // (tile rows start on a 32-row block: BN % 32 == 0)
      src_off[i] = i < kXDma ? (unsigned)(min(r, x_left) * (int)a.ldx * 2 + c * 16)
                   : a.w_kt ? (unsigned)((rw / kBlkRows) * a.w_kt * kBlkBytes + (rw % kBlkRows) * (kBlkK * 2) + c * 16)
                            : (unsigned)(rw * (int)a.ldw * 2 + c * 16);
    }
  };
  Segment isg = walk.first_segment();
  int is_kt = isg.kt0;
  set_offsets(isg);
  // A refill of one stage from the cursor's k-tile, prepared once (scalar
  // descriptors, stage base, K-tail extent); dma_one(r, i) issues its
  // instruction i and issue_advance() then moves the cursor on, so that the
  // refill can be spread between MFMAs (mma_dma below).  A refill that is
  // not live gets descriptors of zero size: its instructions read zeros into
  // a stage that is never read again (the end of the stream), so the main
  // loop issues the same instruction sequence every k-tile.
  struct Refill {
    rsrc_t xr, wr;
    char* base;
    int kleft;  // valid K elements in the k-tile
  };
  auto refill_at = [&](int stage, bool live) {
    Refill r;
    const int m0 = walk.row0(isg.tm), n0 = isg.tn * BN;
    const int bytes = live ? 0x7ffffff0 : 0;
    r.base = lds + stage * S::kStageBytes;
    r.xr = make_rsrc_uniform(reinterpret_cast<const char*>(a.x + (int64_t)m0 * a.ldx) + is_kt * BK * 2, bytes);
    r.wr = make_rsrc_uniform(
        a.w_kt ? reinterpret_cast<const char*>(a.w) + ((int64_t)(n0 / kBlkRows) * a.w_kt + is_kt) * kBlkBytes
               : reinterpret_cast<const char*>(a.w + (int64_t)n0 * a.ldw) + is_kt * BK * 2,
        bytes);
    r.kleft = a.K - is_kt * BK;
    return r;
  };
  auto dma_one = [&](const Refill& r, int i) {
    unsigned off = src_off[i];
    if (r.kleft < BK && (lpos ^ lds_swz<BK>(dma_row(i))) * 8 >= r.kleft) off = kOutOfRange;
    // Stream-K reads each weight byte once per call: its weight loads are
    // non-temporal (nt), measured 4-8% faster on the weight streams than
    // the default policy.
    if (i < kXDma || !STREAMK) dma16(i < kXDma ? r.xr : r.wr, off, (lds_void*)(r.base + (i * kDW + dwave) * 1024));
    else dma16_pol<kCachePolicyNt>(r.wr, off, (lds_void*)(r.base + (i * kDW + dwave) * 1024));
  };
  auto issue_advance = [&]() {
    if (++is_kt == isg.kt1) {
      isg = walk.next_segment(isg);
      is_kt = isg.kt0;
      set_offsets(isg);
    }
  };
  auto issue = [&](int stage) {  // issue the cursor's k-tile, then advance the cursor
    const Refill r = refill_at(stage, true);
#pragma unroll
    for (int i = 0; i < kDma; ++i) dma_one(r, i);
    issue_advance();
  };

  // ---- producer waves: the prologue's requests, then per k-tile: wait for
  // the next k-tile's loads, the barrier that retires the current one (the
  // compute waves' barrier, one per k-tile on both sides), then the refill
  // of the stage it freed.
  if constexpr (PW > 0) {
    if (wave >= S::kWaves) {
      const int steps = walk.steps();
      // The residual copy of tile `sg`: instruction i fills LDS bytes
      // [1024 i, 1024 i + 1024) of the row-major [BM][BN] block.  Rows past
      // M and columns past Nout read clamped (their outputs are not stored).
      auto issue_res = [&](const Segment& sg) {
        if constexpr (kResLds) {
          const rsrc_t rr = make_rsrc_uniform(a.resid, 0x7ffffff0);
          const int m0 = walk.row0(sg.tm), n0 = sg.tn * BN;
#pragma unroll
          for (int q = 0; q < BM * BN * 2 / 1024 / PW; ++q) {
            const int i = q * PW + dwave;
            const int e = i * 512 + lane * 8;
            const int row = min(m0 + e / BN, a.M - 1), col = min(n0 + e % BN, a.Nout - 8);
            dma16(rr, (unsigned)(((int64_t)row * a.ldr + col) * 2), (lds_void*)(res_lds + i * 1024));
          }
        }
      };
      Segment psg = walk.first_segment();  // the tile of step s
      int pkt = psg.kt0;
      for (int t = 0; t < STAGES; ++t)
        if (t < steps) issue(t);
      if (steps >= STAGES) vm_wait<(STAGES - 1) * kDma>();
      else vm_wait<0>();
      if (res_in_lds) issue_res(psg);
      __syncthreads();
      int stage = 0;
      for (int s = 0; s < steps; ++s) {
        // Before the barrier after which the tile's epilogue runs, its
        // residual copy has landed too.
        const bool tile_end = kResLds && pkt + 1 == psg.kt1;
        if (res_in_lds && tile_end) {
          vm_wait<0>();
        } else if (s + 1 < steps) {
          if (s + STAGES - 1 < steps) vm_wait<(STAGES - 2) * kDma>();
          else vm_wait<0>();
        }
        __syncthreads();
        const int freed = stage;
        stage = stage + 1 == STAGES ? 0 : stage + 1;
        if (s + STAGES < steps) issue(freed);
        // A tile's copy goes out after its first barrier: the compute waves
        // have finished the previous tile's epilogue to get there.
        if constexpr (kResLds) {
          if (res_in_lds && s > 0 && pkt == psg.kt0) issue_res(psg);
          if (tile_end && s + 1 < steps) {
            psg = walk.next_segment(psg);
            pkt = psg.kt0;
          } else {
            ++pkt;
          }
        }
      }
      vm_wait<0>();
      return;
    }
  }

  // ---- fragment sets in registers (see the main loop):
  //   kDeep: one set per k-step of a k-tile;  otherwise two (ping-pong);
  //   kSingle: one, when two do not fit beside the accumulators in the
  //     register budget (the other compute wave on the SIMD covers the LDS
  //     latency that a single set exposes).
  constexpr int kReads = S::FM + S::FN;  // LDS reads per fragment set
  constexpr int kWavesPerSimd = ((S::kWaves + PW) * OCC + 3) / 4;  // register budget 512 / this
  constexpr bool kDeep = S::KS == 4 && kReads * 4 * 4 <= 64 && kWavesPerSimd <= 3;
  constexpr bool kSingle = !kDeep && S::FM * S::FN * 16 + 2 * kReads * 4 + 24 > 512 / kWavesPerSimd;

  // ---- fragment addressing (byte offsets within a stage): lane reads row
  // (base + lane%32) of chunk 2*ks + lane/32.
  const int frow = lane & 31;
  const int fk = lane >> 5;
  int xrow_off[S::FM], xrow_swz[S::FM], wrow_off[S::FN], wrow_swz[S::FN];
#pragma unroll
  for (int j = 0; j < S::FM; ++j) {
    const int r = wm * S::TM + j * 32 + frow;
    xrow_off[j] = r * S::kRowBytes;
    xrow_swz[j] = lds_swz<BK>(r);
  }
#pragma unroll
  for (int i = 0; i < S::FN; ++i) {
    const int r = wn * S::TN + i * 32 + frow;
    wrow_off[i] = S::kXBytes + r * S::kRowBytes;
    wrow_swz[i] = lds_swz<BK>(r);
  }

  // kSingle: chunk 2 ks + fk of a row sits at ((fk ^ swz) << 4) ^ (ks << 5),
  // so one base register per fragment row serves every k-step; the bases
  // are redefined (opaquely) each k-tile, so the compiler cannot hoist one
  // address per k-step out of the loop (which spills at this budget).
  int xaddr[S::FM], waddr[S::FN];
#pragma unroll
  for (int j = 0; j < S::FM; ++j) xaddr[j] = xrow_off[j] + ((fk ^ xrow_swz[j]) << 4);
#pragma unroll
  for (int i = 0; i < S::FN; ++i) waddr[i] = wrow_off[i] + ((fk ^ wrow_swz[i]) << 4);
  auto refresh_addr = [&]() {
#pragma unroll
    for (int j = 0; j < S::FM; ++j) asm volatile("" : "+v"(xaddr[j]));
#pragma unroll
    for (int i = 0; i < S::FN; ++i) asm volatile("" : "+v"(waddr[i]));
  };

  struct Frags {
    i32x4 x[S::FM];
    i32x4 w[S::FN];
  };
  auto read = [&](Frags& f, int stage, int ks) {
    const char* base = lds + stage * S::kStageBytes;
    if constexpr (kSingle) {
#pragma unroll
      for (int j = 0; j < S::FM; ++j) f.x[j] = *reinterpret_cast<const i32x4*>(base + (xaddr[j] ^ (ks << 5)));
#pragma unroll
      for (int i = 0; i < S::FN; ++i) f.w[i] = *reinterpret_cast<const i32x4*>(base + (waddr[i] ^ (ks << 5)));
      return;
    }
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
  // The same MFMAs with DMA instructions [I0, I0 + N) of refill `r` spread
  // evenly between them (after MFMA q go instructions I0 + q*N/Q ..
  // I0 + (q+1)*N/Q - 1, Q MFMAs in all), so that the load path drains while
  // the matrix unit works.
  auto mma_dma = [&](const Frags& f, const Refill& r, auto i0c, auto nc) {
    constexpr int I0 = decltype(i0c)::value, N = decltype(nc)::value;
    constexpr int Q = S::FN * S::FM;
#pragma unroll
    for (int i = 0; i < S::FN; ++i)
#pragma unroll
      for (int j = 0; j < S::FM; ++j) {
        const int q = i * S::FM + j;
        acc[i][j] = mfma32(f.w[i], f.x[j], acc[i][j]);
#pragma unroll
        for (int d = I0 + q * N / Q; d < I0 + (q + 1) * N / Q; ++d) dma_one(r, d);
        __builtin_amdgcn_sched_barrier(0);
      }
  };

  // ---- epilogue of one tile, straight from registers.  A lane's
  // accumulator block (i, j) holds token m = lane%32 and, in register
  // 4g + e, feature 8g + 4h + e (h = lane/32).  For a register-group pair
  // (g, g+1), lanes l and l+32 hold the two 8-byte halves of token l's
  // features 8g .. 8g+7 and 8(g+1) .. 8(g+1)+7 crosswise; one
  // v_permlane32_swap per dword turns that into 16 contiguous bytes per lane
  // (lane l: features 8g.., lane l+32: 8(g+1)..), stored with one 16-byte
  // store.  Rounding mirrors the unfused reference: the projection (or the
  // gated product) is rounded to bf16 in registers; bias, gelu and the
  // residual add then apply in f32 on the stored layout, each rounded.
  auto pair16 = [](bf16x4 lo, bf16x4 hi) -> bf16x8 {
    const i32x2 a = __builtin_bit_cast(i32x2, lo), b = __builtin_bit_cast(i32x2, hi);
    const auto s0 = __builtin_amdgcn_permlane32_swap((unsigned)a[0], (unsigned)b[0], false, false);
    const auto s1 = __builtin_amdgcn_permlane32_swap((unsigned)a[1], (unsigned)b[1], false, false);
    const i32x4 v = {(int)s0[0], (int)s1[0], (int)s0[1], (int)s1[1]};
    return __builtin_bit_cast(bf16x8, v);
  };
  // Pre-norm epilogues scale the accumulators of row m first: r_m (acc -
  // mu_m c_n) for LayerNorm, r_m acc for RMSNorm (the norm weight is folded
  // into w, c_n = sum_k of folded row n); then the base epilogue E runs.
  constexpr int E = epi_base(EPI);
  constexpr int NORM = epi_norm(EPI);
  // A tile's row statistics and column sums are all loaded before any of
  // them is used, so the epilogue waits for one round trip, not one per
  // block.
  auto normalize_tile = [&](int m0, int n0) {
    float rs[S::FM];
#pragma unroll
    for (int j = 0; j < S::FM; ++j) {
      const int m = min(m0 + wm * S::TM + j * 32 + frow, a.M - 1);
      rs[j] = a.stats[2 * (int64_t)m + 1];
    }
    if constexpr (NORM == kNormLayer) {
      // acc - mu_m c_n as one more MFMA per block: A holds c_n's bf16 split
      // (hi, hi, lo) and B -mu_m's (hi, lo, hi) in k = 0..2 (lanes 0-31;
      // zeros elsewhere), so the block gains c_hi mu_hi + c_hi mu_lo +
      // c_lo mu_hi, each product exact in f32 (relative error ~2^-16 of
      // mu c, the c_lo mu_lo term).  Two values per lane instead of the
      // block's 16 column sums.
      i32x4 ca[S::FN], mb[S::FM];
#pragma unroll
      for (int i = 0; i < S::FN; ++i) {
        const float c = a.colsum[min(n0 + wn * S::TN + i * 32 + frow, a.N - 1)];
        const __bf16 hi = to_bf16(c), lo = to_bf16(c - to_f32(hi));
        bf16x8 v = {};
        if (fk == 0) v[0] = hi, v[1] = hi, v[2] = lo;
        ca[i] = __builtin_bit_cast(i32x4, v);
      }
#pragma unroll
      for (int j = 0; j < S::FM; ++j) {
        const int m = min(m0 + wm * S::TM + j * 32 + frow, a.M - 1);
        const float nm = -a.stats[2 * (int64_t)m];
        const __bf16 hi = to_bf16(nm), lo = to_bf16(nm - to_f32(hi));
        bf16x8 v = {};
        if (fk == 0) v[0] = hi, v[1] = lo, v[2] = hi;
        mb[j] = __builtin_bit_cast(i32x4, v);
      }
#pragma unroll
      for (int i = 0; i < S::FN; ++i)
#pragma unroll
        for (int j = 0; j < S::FM; ++j) acc[i][j] = mfma32(ca[i], mb[j], acc[i][j]);
    }
#pragma unroll
    for (int i = 0; i < S::FN; ++i)
#pragma unroll
      for (int j = 0; j < S::FM; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] *= rs[j];
  };
  // DeltaNet causal conv + SiLU over the in_proj qkv columns
  // (src/archs/qwen35_text.rs:515-526,632-650; src/kernels/qwen35.cu:3-29):
  // out[r, n] = silu(sum over taps t = 3..0 of w[n, 3 - t] * p[r - t, n]),
  // p = the bf16-rounded projection, taps before the row's sequence start
  // (pos[r] < t) reading zeros; columns from conv_ch on are the plain
  // projection (z, b, a).  The taps accumulate in f32 and the SiLU uses the
  // hardware exp and reciprocal (as the SwiGLU epilogue), rounded once to
  // bf16: the reference rounds
  // every product and partial sum to bf16 instead, which costs three times
  // the VALU work in this epilogue and agrees to the projection tolerance.  The wave
  // holds all rows of the tile (WM = 1): row R = 32 j + lane % 32 of block
  // j, so row R - t is lane - t of block j, or lane + 32 - t of block j - 1.
  // One ds_bpermute per tap moves a bf16 pair: each lane offers block j's
  // value, or block j - 1's when it is among the last t lanes of its half.
  // Rows below `skip` are the tile's halo (computed, not stored).
  auto conv_epilogue = [&](int m0, int n0, int skip) {
    const int h = fk;
    int pos[S::FM];
#pragma unroll
    for (int j = 0; j < S::FM; ++j) {
      const int m = m0 + j * 32 + frow;
      pos[j] = m < a.M ? a.pos[m] : 0;
    }
#pragma unroll
    for (int i = 0; i < S::FN; ++i) {
      bf16x4 o[S::FM][4];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn * S::TN + i * 32 + 8 * g + 4 * h;  // features n .. n+3 (conv_ch % 4 == 0)
        float p[S::FM][4];
#pragma unroll
        for (int j = 0; j < S::FM; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) p[j][e] = round_bf16(acc[i][j][4 * g + e]);
        if (n < a.conv_ch) {
          // taps of features n .. n+3: 16 bf16, row-major [feature][tap]
          const bf16x8 w01 = *reinterpret_cast<const bf16x8*>(a.conv_w + (int64_t)n * kConvTaps);
          const bf16x8 w23 = *reinterpret_cast<const bf16x8*>(a.conv_w + (int64_t)n * kConvTaps + 8);
          float cw[4][kConvTaps];
#pragma unroll
          for (int q = 0; q < kConvTaps; ++q) {
            cw[0][q] = to_f32(w01[q]);
            cw[1][q] = to_f32(w01[4 + q]);
            cw[2][q] = to_f32(w23[q]);
            cw[3][q] = to_f32(w23[4 + q]);
          }
          // packed bf16 pairs of each block: (e0, e1), (e2, e3)
          unsigned pk[S::FM][2];
#pragma unroll
          for (int j = 0; j < S::FM; ++j)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              bf16x4 b4;
#pragma unroll
              for (int e = 0; e < 4; ++e) b4[e] = to_bf16(p[j][e]);
              pk[j][u] = __builtin_bit_cast(i32x2, b4)[u];
            }
          float val[S::FM][4];
#pragma unroll
          for (int j = 0; j < S::FM; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) val[j][e] = 0.0f;
#pragma unroll
          for (int t = kConvTaps - 1; t >= 0; --t) {  // oldest tap first, as the reference adds them
            float x[S::FM][4];
            if (t == 0) {
#pragma unroll
              for (int j = 0; j < S::FM; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) x[j][e] = p[j][e];
            } else {
              const int src = (lane & 32) | (((lane & 31) - t) & 31);
              const bool late = (lane & 31) >= 32 - t;  // offers the previous block's row
#pragma unroll
              for (int j = 0; j < S::FM; ++j)
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                  const unsigned prev = j > 0 ? pk[j > 0 ? j - 1 : 0][u] : 0u;
                  const unsigned offer = late ? prev : pk[j][u];
                  const unsigned got = (unsigned)__shfl((int)offer, src, 64);
                  const i32x2 g2 = {(int)(u == 0 ? got : 0), (int)(u == 1 ? got : 0)};
                  const bf16x4 b4 = __builtin_bit_cast(bf16x4, g2);
                  x[j][2 * u] = to_f32(b4[2 * u]);
                  x[j][2 * u + 1] = to_f32(b4[2 * u + 1]);
                }
            }
            const int tap = kConvTaps - 1 - t;
#pragma unroll
            for (int j = 0; j < S::FM; ++j) {
              const float keep = pos[j] >= t ? 1.0f : 0.0f;  // taps before the sequence start read zeros
#pragma unroll
              for (int e = 0; e < 4; ++e) val[j][e] = fmaf(x[j][e] * keep, cw[e][tap], val[j][e]);
            }
          }
#pragma unroll
          for (int j = 0; j < S::FM; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float v = val[j][e];
              o[j][g][e] = to_bf16(silu(v));
            }
        } else {
#pragma unroll
          for (int j = 0; j < S::FM; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) o[j][g][e] = to_bf16(p[j][e]);
        }
      }
#pragma unroll
      for (int j = 0; j < S::FM; ++j) {
        const int r = j * 32 + frow;
        const int m = m0 + r;
        const bool row_ok = m < a.M && r >= skip;
#pragma unroll
        for (int gp = 0; gp < 2; ++gp) {
          const bf16x8 v = pair16(o[j][2 * gp], o[j][2 * gp + 1]);
          const int n = n0 + wn * S::TN + i * 32 + 16 * gp + 8 * h;
          if (row_ok && n < a.Nout) store8(a.y + (int64_t)m * a.ldy + n, v, a.Nout - n);
        }
      }
    }
  };
  auto epilogue = [&](int m0, int n0, int skip) {
    if constexpr (NORM != kNormNone) normalize_tile(m0, n0);
    if constexpr (kConv) {
      conv_epilogue(m0, n0, skip);
      return;
    }
    const int h = fk;
    const int out_n0 = epi_gated(E) ? (n0 + wn * S::TN) / 2 : n0 + wn * S::TN;
    // The residual of every element this lane stores, loaded before any
    // store: y may alias it (the in-place update of the hidden state), and a
    // load behind a store to a possibly aliasing address would wait a whole
    // round trip each.  A lane reads exactly the elements it then writes, so
    // reading them all first is correct in place too.
    // (Only for wave tiles of at most three 32x32 blocks, or four with two
    // waves per SIMD (256 registers): the larger ones have no registers to
    // spare for the batch and would spill.)
    constexpr bool kResRegs = epi_has_resid<E>() && !epi_gated(E) && E != kEpiRopeQkv &&
                              (S::FM * S::FN <= 3 || (S::FM * S::FN <= 4 && kWavesPerSimd <= 2));
    bf16x8 rres[kResRegs ? S::FM : 1][kResRegs ? S::FN : 1][2];
    if constexpr (kResRegs) {
      if (!(kResLds && res_in_lds)) {
#pragma unroll
        for (int j = 0; j < S::FM; ++j) {
          const int m = m0 + wm * S::TM + j * 32 + frow;
#pragma unroll
          for (int i = 0; i < S::FN; ++i)
#pragma unroll
            for (int gp = 0; gp < 2; ++gp) {
              const int n = out_n0 + i * 32 + 16 * gp + 8 * h;
              rres[j][i][gp] = m < a.M && n < a.Nout ? load8_bf16(a.resid + (int64_t)m * a.ldr + n, a.Nout - n)
                                                     : bf16x8{};
            }
        }
      }
    }
    // The bias of every column this lane stores, likewise loaded before
    // any store (the bias does not depend on the row: FN x 2 vectors).
    // (Only where the accumulators and the batched vectors take at most half
    // of a wave's registers: beyond that the batch spills.)
    constexpr bool kBiasRegs = epi_has_bias<E>() && !epi_gated(E) && E != kEpiRopeQkv &&
                               S::FM * S::FN * 16 + S::FN * 8 + (kResRegs ? S::FM * S::FN * 8 : 0) <=
                                   512 / kWavesPerSimd / 2;
    bf16x8 rbias[kBiasRegs ? S::FN : 1][2];
    if constexpr (kBiasRegs) {
#pragma unroll
      for (int i = 0; i < S::FN; ++i)
#pragma unroll
        for (int gp = 0; gp < 2; ++gp) {
          const int n = out_n0 + i * 32 + 16 * gp + 8 * h;
          rbias[i][gp] = n < a.Nout ? load8_bf16(a.bias + n, a.Nout - n) : bf16x8{};
        }
    }
#pragma unroll
    for (int j = 0; j < S::FM; ++j) {
      const int m = m0 + wm * S::TM + j * 32 + frow;
      const bool row_ok = m < a.M;
#pragma unroll
      for (int i = 0; i < S::FN; ++i) {
        if constexpr (E == kEpiRopeQkv) {
          // Blocks i (even) and i+1 are the two halves of one 64-wide head
          // (the plan guarantees 64-wide, head-aligned wave columns), so a
          // lane holds columns c and c+32 of the same token: the rotation
          // of src/kernels/modernbert.cu:31-74 happens in registers on the
          // bf16-rounded projection, rounded once, and q, k and v go to
          // their planes.
          if (i % 2 == 0) {
            const int nw = out_n0 + i * 32;  // head start column in qkv
            const int H = a.Nout / 3;
            const int p = nw / H;
            const int col = nw - p * H;
            const int pos = row_ok ? min(max(a.pos[m], 0), a.rope_rows - 1) : 0;  // stay inside the tables
            bf16x4 lo[4], hi[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              float x0[4], x1[4];
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                x0[e] = round_bf16(acc[i][j][4 * g + e]);
                x1[e] = round_bf16(acc[i + 1][j][4 * g + e]);
              }
              if (p < 2) {
                const int c = 8 * g + 4 * h;  // column within the half head
                const f32x4 cs = *reinterpret_cast<const f32x4*>(a.rope_cos + (int64_t)pos * 32 + c);
                const f32x4 sn = *reinterpret_cast<const f32x4*>(a.rope_sin + (int64_t)pos * 32 + c);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  const float r0 = x0[e] * cs[e] - x1[e] * sn[e];
                  const float r1 = x0[e] * sn[e] + x1[e] * cs[e];
                  x0[e] = r0;
                  x1[e] = r1;
                }
              }
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                lo[g][e] = to_bf16(x0[e]);
                hi[g][e] = to_bf16(x1[e]);
              }
            }
            __bf16* dst = a.y + p * a.plane + (int64_t)m * a.ldy + col;
#pragma unroll
            for (int gp = 0; gp < 2; ++gp) {
              const bf16x8 vlo = pair16(lo[2 * gp], lo[2 * gp + 1]);
              const bf16x8 vhi = pair16(hi[2 * gp], hi[2 * gp + 1]);
              if (row_ok) {
                store8(dst + 16 * gp + 8 * h, vlo, 8);
                store8(dst + 32 + 16 * gp + 8 * h, vhi, 8);
              }
            }
          }
        } else if constexpr (epi_gated(E)) {
          // A 32-row block of the packed weight is 16 gate rows then the 16
          // up rows of the same 16 output columns: registers 4g+e (g = 0, 1)
          // hold gate rows, 4(g+2)+e the matching up rows.
          bf16x4 o[2];
#pragma unroll
          for (int g = 0; g < 2; ++g)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              o[g][e] = to_bf16(epi_gate<E>(acc[i][j][4 * g + e], acc[i][j][4 * (g + 2) + e]));
          const bf16x8 v = pair16(o[0], o[1]);
          const int n = out_n0 + i * 16 + 8 * h;
          if (row_ok && n < a.Nout) store8(a.y + (int64_t)m * a.ldy + n, v, a.Nout - n);
        } else {
#pragma unroll
          for (int gp = 0; gp < 2; ++gp) {
            bf16x4 p[2];
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
              for (int e = 0; e < 4; ++e) p[q][e] = to_bf16(acc[i][j][4 * (2 * gp + q) + e]);
            bf16x8 v = pair16(p[0], p[1]);
            const int n = out_n0 + i * 32 + 16 * gp + 8 * h;
            if (row_ok && n < a.Nout) {
              const int valid = a.Nout - n;
              if constexpr (E != kEpiNone) {
                float b[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                if constexpr (kBiasRegs) {
#pragma unroll
                  for (int e = 0; e < 8; ++e) b[e] = to_f32(rbias[i][gp][e]);
                } else if constexpr (epi_has_bias<E>()) {
                  load8(a.bias + n, b, valid);
                }
                float r[8];
                if constexpr (epi_has_resid<E>()) {
                  if (kResLds && res_in_lds) {
                    const bf16x8 rv = *reinterpret_cast<const bf16x8*>(
                        res_lds + ((m - m0) * BN + (n - n0)) * 2);
#pragma unroll
                    for (int e = 0; e < 8; ++e) r[e] = to_f32(rv[e]);
                  } else if constexpr (kResRegs) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) r[e] = to_f32(rres[j][i][gp][e]);
                  } else {
                    load8(a.resid + (int64_t)m * a.ldr + n, r, valid);
                  }
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                  float t = epi_pre<E>(to_f32(v[e]), b[e]);
                  if constexpr (epi_has_resid<E>()) t = round_bf16(t + r[e]);
                  v[e] = to_bf16(t);
                }
              }
              store8(a.y + (int64_t)m * a.ldy + n, v, valid);
            }
          }
        }
      }
    }
  };

  // ---- stream-K partials: f32 accumulators in lane-native order, two
  // slots (head, tail) per workgroup: [wave][block i][block j][4 x f32x4][64].
  // Each XCD has its own L2 and the L2s are not coherent with each other, so
  // a device-scope fence would write back and invalidate the whole L2 (and
  // with it the cached x panel every workgroup on the XCD is using).  The
  // partials instead move with the agent-coherent cache policy (sc1: stores
  // write through, loads bypass stale L2 lines): the writer waits for its
  // stores to be acknowledged before a relaxed agent-scope counter
  // increment, and the last arriving workgroup reads them back coherently.
  constexpr int kWaveF4 = S::FN * S::FM * 4 * 64;     // f32x4 per wave per slot
  constexpr int kTileF4 = S::kWaves * kWaveF4;        // f32x4 per slot
  constexpr int kCoherent = 16;                       // cache policy: sc1
  const rsrc_t wsr = make_rsrc(a.ws);
  auto slot_off = [&](int g, int slot) -> unsigned {  // byte offset of this lane's first f32x4
    return (unsigned)((((int64_t)g * 2 + slot) * kTileF4 + wave * kWaveF4 + lane) * 16);
  };
  // A partial segment: write this workgroup's partial; returns true when it
  // is the tile's last segment to arrive, with acc then holding the full sum
  // (the caller runs the epilogue).
  auto finish_partial = [&](const Segment& sg) -> bool {
    const int t = sg.st;
    const int slot = sg.spos == walk.begin ? 0 : 1;
    const unsigned mine = slot_off(blockIdx.x, slot);
    // (sched_barrier keeps the scheduler from hoisting the whole partial's
    // memory traffic together: that would raise the register peak of the
    // kernel, and with it cost occupancy in the main loop.)
#pragma unroll
    for (int i = 0; i < S::FN; ++i)
#pragma unroll
      for (int j = 0; j < S::FM; ++j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                           acc[i][j][4 * q + 3]};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v), wsr,
                                                 (int)(mine + ((i * S::FM + j) * 4 + q) * 64 * 16), 0,
                                                 kCoherent);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    int g_lo, g_hi;
    walk.tile_owners(t, g_lo, g_hi);
    // Each wave arrives on its own counter (tile, wave): its slice of the
    // tile (its accumulators, its epilogue) is independent of the other
    // waves', so the last owner of each slice sums and stores that slice
    // alone -- no barrier and no LDS.  Waves of one workgroup may disagree
    // about being last; every slice still has exactly one last owner.
    unsigned* counter = a.counters + (int64_t)t * S::kWaves + wave;
    __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores are acknowledged
    unsigned prev = 0;
    if (lane == 0) prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = __builtin_amdgcn_readfirstlane(prev);
    if (prev != (unsigned)(g_hi - g_lo)) return false;
    zero_acc();
    const int64_t tile_lo = (int64_t)t * walk.kt_count;
    for (int g = g_lo; g <= g_hi; ++g) {
      // g's segment in this tile is its head iff g's range starts inside the tile.
      const unsigned src = slot_off(g, walk.start(g) >= tile_lo ? 0 : 1);
      // All of one owner's loads are in flight together (these coherent
      // reads come from beyond the L2: one round trip per owner, not one
      // per block), then added in the same order as always.
      f32x4 v[S::FN][S::FM][4];
#pragma unroll
      for (int i = 0; i < S::FN; ++i)
#pragma unroll
        for (int j = 0; j < S::FM; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            v[i][j][q] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           wsr, (int)(src + ((i * S::FM + j) * 4 + q) * 64 * 16), 0, kCoherent));
#pragma unroll
      for (int i = 0; i < S::FN; ++i)
#pragma unroll
        for (int j = 0; j < S::FM; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] += v[i][j][q][e];
      __builtin_amdgcn_sched_barrier(0);
    }
    if (lane == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
  };

  // ---- main loop over this workgroup's k-tile stream.  Step s lives in
  // stage s % STAGES.  The prologue requests steps 0..STAGES-1; after the
  // barrier that retires step s, step s + STAGES is requested into the stage
  // just freed -- across item boundaries, so the next item's first k-tiles
  // land while this item finishes and stores.  Before that barrier step s+1
  // must have landed while s+2 .. s+STAGES-1 may still be in flight:
  // vmcnt((STAGES-2) * DMAs per step).  sched_barrier(0) pins the order
  // below: the next k-step's fragment reads are issued before the current
  // k-step's MFMAs, so LDS latency hides behind a full k-step of matrix work.
  const int steps = walk.steps();
  constexpr bool kIssue = PW == 0;  // this wave issues refills
  if constexpr (kIssue) {
    for (int t = 0; t < STAGES; ++t)
      if (t < steps) issue(t);
    if (steps >= STAGES) vm_wait<(STAGES - 1) * kDma>();
    else vm_wait<0>();
  }
  __syncthreads();

  Segment csg = walk.first_segment();  // compute cursor
  int ckt = csg.kt0;
  // Schedules of a k-tile's KS k-steps of MFMAs (fragment reads one k-step
  // ahead of their MFMAs in the first two; kSingle reads each k-step's set
  // behind the previous k-step's MFMAs and waits for it):
  //   kDeep (one fragment set per k-step, when they fit in registers): the
  //     barrier that frees the stage comes after the k-tile's last two
  //     fragment sets are in registers, so two k-steps of MFMAs run after it,
  //     covering the next stage's first fragment reads, with the freed
  //     stage's refill issued between them;
  //   otherwise (ping-pong sets): one k-step of MFMAs after the barrier.
  constexpr int kSets = kDeep ? 4 : kSingle ? 1 : 2;
  Frags fr[kSets];
  if (steps > 0) {
    read(fr[0], 0, 0);
    if constexpr (kDeep) read(fr[1], 0, 1);
  }
  int stage = 0;
  for (int s = 0; s < steps; ++s) {
    if constexpr (kSingle) refresh_addr();
    if constexpr (kDeep) {
      // fr[0] (and fr[1], one set later) of this k-tile were read after the
      // previous barrier.  Waiting for them explicitly keeps the compiler
      // from resolving its merged loop-header state with a full LDS wait
      // after the next reads.
      __builtin_amdgcn_s_waitcnt(0xc07f | (kReads << 8));  // lgkmcnt(kReads): fr[0] is in
      __builtin_amdgcn_sched_barrier(0);
      read(fr[2], stage, 2);
      __builtin_amdgcn_sched_barrier(0);
      mma(fr[0]);
      __builtin_amdgcn_sched_barrier(0);
      read(fr[3], stage, 3);
      __builtin_amdgcn_sched_barrier(0);
      mma(fr[1]);
      __builtin_amdgcn_sched_barrier(0);
    } else if constexpr (kSingle) {
      // Each k-step's fragments are waited for just before its MFMAs.
#pragma unroll
      for (int ks = 0; ks < S::KS; ++ks) {
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
        __builtin_amdgcn_sched_barrier(0);
        mma(fr[0]);
        __builtin_amdgcn_sched_barrier(0);
        if (ks + 1 < S::KS) read(fr[0], stage, ks + 1);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      // As above: the k-tile's first fragments are in.
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0), vmcnt/expcnt unconstrained
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int ks = 1; ks < S::KS; ++ks) {
        read(fr[ks % 2], stage, ks);
        __builtin_amdgcn_sched_barrier(0);
        mma(fr[(ks - 1) % 2]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (kIssue && s + 1 < steps) {
      if (s + STAGES - 1 < steps) vm_wait<(STAGES - 2) * kDma>();
      else vm_wait<0>();
    }
    __syncthreads();
    // Next k-tile's first fragments, this k-tile's last MFMAs, then the
    // refill of the stage just freed: the refill's load instructions can
    // stall issue while the load path drains, and issued behind the MFMAs
    // that stall overlaps matrix work instead of delaying it.
    const int freed = stage;
    stage = stage + 1 == STAGES ? 0 : stage + 1;
    // One workgroup per CU (OCC == 1): the refill's instructions go between
    // the MFMAs that follow the barrier.  With two workgroups per CU the
    // other workgroup's MFMAs cover the refill, and one burst after the
    // first MFMA group measured faster.
    using std::integral_constant;
    constexpr bool kSpread = OCC == 1 && kIssue;
    const Refill r = refill_at(freed, s + STAGES < steps);
    auto refill_all = [&]() {
#pragma unroll
      for (int i = 0; i < kDma; ++i) if constexpr (kIssue) dma_one(r, i);
    };
    if constexpr (kSingle) {
      if (s + 1 < steps) read(fr[0], stage, 0);
      __builtin_amdgcn_sched_barrier(0);
      refill_all();
    } else if constexpr (kDeep && kSpread) {
      constexpr int kHalf = kDma / 2;
      if (s + 1 < steps) {
        read(fr[0], stage, 0);
        read(fr[1], stage, 1);
      }
      __builtin_amdgcn_sched_barrier(0);
      mma_dma(fr[2], r, integral_constant<int, 0>(), integral_constant<int, kHalf>());
      mma_dma(fr[3], r, integral_constant<int, kHalf>(), integral_constant<int, kDma - kHalf>());
    } else if constexpr (kDeep) {
      if (s + 1 < steps) read(fr[0], stage, 0);
      __builtin_amdgcn_sched_barrier(0);
      mma(fr[2]);
      __builtin_amdgcn_sched_barrier(0);
      refill_all();
      __builtin_amdgcn_sched_barrier(0);
      if (s + 1 < steps) read(fr[1], stage, 1);
      __builtin_amdgcn_sched_barrier(0);
      mma(fr[3]);
    } else if constexpr (kSpread) {
      if (s + 1 < steps) read(fr[0], stage, 0);
      __builtin_amdgcn_sched_barrier(0);
      mma_dma(fr[(S::KS - 1) % 2], r, integral_constant<int, 0>(), integral_constant<int, kDma>());
    } else {
      if (s + 1 < steps) read(fr[0], stage, 0);
      __builtin_amdgcn_sched_barrier(0);
      mma(fr[(S::KS - 1) % 2]);
      __builtin_amdgcn_sched_barrier(0);
      refill_all();
    }
    if (kIssue && s + STAGES < steps) issue_advance();
    __builtin_amdgcn_sched_barrier(0);
    if (++ckt == csg.kt1) {
      if constexpr (STREAMK) {
        if (walk.complete(csg) || finish_partial(csg))
          epilogue(walk.row0(csg.tm), csg.tn * BN, csg.tm ? kConvHalo : 0);
      } else {
        epilogue(walk.row0(csg.tm), csg.tn * BN, csg.tm ? kConvHalo : 0);
      }
      zero_acc();
      if (s + 1 < steps) {
        csg = walk.next_segment(csg);
        ckt = csg.kt0;
      }
    }
  }
  vm_wait<0>();  // the zero-size refills of the last k-tiles write LDS too
}

}  // namespace sys1
