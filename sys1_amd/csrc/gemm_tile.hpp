// Projection GEMM for gfx950: y[M,N] = epi(x[M,K] . w[N,K]^T) on
// v_mfma_f32_32x32x16_bf16.  One kernel template covers both regimes:
//   - large M: MFMA-bound output tiles, one k-stream per tile;
//   - small M (the weight-streaming regime): BM = the padded token count,
//     BN = 256, with K split over workgroups so that every CU streams weight.
//
// Tile:    BM x BN output tile, BK = 64, WM x WN waves, each wave owns a
//          (BM/WM) x (BN/WN) sub-tile of 32x32 MFMA blocks.  The MFMA takes the
//          weight block as A and the activation block as B, so a lane's
//          accumulator holds runs of 4 consecutive output features of one
//          token.
// Loads:   global -> LDS directly (buffer_load ... lds, no VGPR staging).  One
//          wave instruction fills 1 KB of LDS = 8 rows x 128 B; the 8 lanes
//          of a row read its 128 B line (coalesced) in a permuted chunk order
//          that realises the LDS swizzle below.  The x and w instructions of a
//          k-tile form one list dealt round-robin to the waves, so every wave
//          issues the same count and vmcnt bookkeeping stays exact.
// LDS:     per operand, row-major 128 B rows (64 bf16 of K); the 16-byte
//          chunk c of row r sits at position c ^ f(r), f(r) = (r ^ r/8) & 7.
//          With this f the MFMA operand reads (lanes 0-31: 32 rows of one
//          chunk, lanes 32-63: the next chunk) run without LDS bank conflicts
//          on gfx950 (SQ_LDS_BANK_CONFLICT = 0 measured; the plain r & 7 and
//          (r + r/8) & 7 swizzles measure 2-way).
// Pipeline: STAGES LDS stages fed as one stream of k-tiles that runs across
//          the work items a persistent workgroup serves, so the next item's
//          loads overlap the current item's last k-tiles and its epilogue.
//          Fragments are double-buffered in registers across k-steps, and the
//          last k-step's MFMAs run after the barrier, overlapping the next
//          k-tile's first LDS reads.
// Epilogue: each wave transposes its output through a private LDS scratch
//          block so that stores (and residual loads) move full 128-byte lines
//          at 16 bytes per lane.
// Stream-K: the weight-streaming shapes split the flattened (tile, k-tile)
//          iteration space into one equal contiguous range per workgroup, so
//          every CU streams the same share of the weight.  A range covers at
//          most a partial head segment, whole tiles, and a partial tail
//          segment; a partial segment writes its f32 accumulators to the
//          workspace (head or tail slot of its workgroup), and the last
//          segment of a tile to arrive (an arrival counter per tile) sums the
//          tile's partials in workgroup order -- deterministic whatever the
//          arrival order -- applies the epilogue and re-arms the counter.
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
__device__ __forceinline__ int lds_swz(int row) { return (row ^ (row >> 3)) & 7; }

template <int BM, int BN, int WM, int WN, int STAGES>
struct TileShape {
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int BK = 64;
  static constexpr int TM = BM / WM;
  static constexpr int TN = BN / WN;
  static constexpr int FM = TM / 32;
  static constexpr int FN = TN / 32;
  static constexpr int KS = BK / 16;                 // MFMA k-steps per k-tile
  static constexpr int kRowBytes = BK * 2;           // 128
  static constexpr int RPI = 8;                      // rows per DMA instruction (1 KB)
  static constexpr int kXBytes = BM * kRowBytes;     // one stage of x
  static constexpr int kWBytes = BN * kRowBytes;
  static constexpr int kStageBytes = kXBytes + kWBytes;
  static constexpr int kStagesBytes = STAGES * kStageBytes;
  // Epilogue scratch, private to each wave: one 32-row block of its output
  // sub-tile in bf16.
  static constexpr int kEpiBytes = 32 * TN * 2;
  static constexpr int kLdsBytes = kStagesBytes + kWaves * kEpiBytes;
  static constexpr int XT = BM / RPI;                // DMA instructions per k-tile: x
  static constexpr int DT = (BM + BN) / RPI;         // x and w together
  static constexpr int kDma = DT / kWaves;           // per wave per k-tile
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be whole 32x32 blocks");
  static_assert(BM % RPI == 0 && BN % RPI == 0, "whole DMA instructions per tile");
  static_assert(DT % kWaves == 0, "DMA instructions deal evenly over the waves");
  static_assert(STAGES >= 2, "at least double buffering");
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget of one gfx950 CU");
  static_assert(kDma * (STAGES - 1) < 64, "vmcnt field");
};

// A segment of a workgroup's k-tile stream: k-tiles [kt0, kt1) of one tile.
struct Segment {
  int tm, tn;     // tile coordinates
  int kt0, kt1;   // k-tile range
  int pos;        // stream position of its first k-tile (tile * kt_count + kt0)
};

// Persistent schedule.  The grid holds at most (CUs x resident workgroups
// per CU) workgroups.
//   Tile mode (large M): each segment is a whole tile.  Workgroup b serves
//     XCD b % 8 and walks that XCD's contiguous share of the tiles with
//     stride (workgroups on the XCD); tiles are rasterised in groups of
//     kGroupM tile rows so the tiles in flight on one XCD share x row panels
//     and w column panels in its L2.
//   Stream mode (small M): workgroup g owns the flattened iterations
//     [start(g), start(g+1)), start(g) = g * T / G, T = tiles * kt_count.
struct TileWalk {
  int tiles_m, tiles_n, kt_count;
  bool stream;
  // tile mode
  int first, count, stride;
  // stream mode
  int64_t total;
  int grid, begin, end;

  static constexpr int kGroupM = 4;

  __device__ TileWalk(int M, int N, int K, int BM, int BN, int BK, bool streamk) {
    tiles_m = (M + BM - 1) / BM;
    tiles_n = (N + BN - 1) / BN;
    kt_count = (K + BK - 1) / BK;
    stream = streamk;
    grid = gridDim.x;
    const int tiles = tiles_m * tiles_n;
    if (stream) {
      total = (int64_t)tiles * kt_count;
      begin = start(blockIdx.x);
      end = start(blockIdx.x + 1);
      count = end > begin;
    } else {
      constexpr int kXcds = 8;
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
  }
  __device__ int start(int g) const { return (int)((int64_t)g * total / grid); }

  // Tile-mode tile index j of this workgroup -> coordinates (grouped raster).
  __device__ void tile_coords(int t, int& tm, int& tn) const {
    const int group = t / (kGroupM * tiles_n);
    const int first_m = group * kGroupM;
    const int gm = min(kGroupM, tiles_m - first_m);
    const int in = t - group * kGroupM * tiles_n;
    tm = first_m + in % gm;
    tn = in / gm;
  }
  __device__ int steps() const {
    return stream ? end - begin : count * kt_count;
  }
  // Segment starting at stream position `pos` (stream mode) or at tile-mode
  // index j = pos / kt_count.
  __device__ Segment segment_at(int pos) const {
    Segment sg;
    if (stream) {
      const int t = pos / kt_count;
      sg.tm = t / tiles_n;
      sg.tn = t - sg.tm * tiles_n;
      sg.kt0 = pos - t * kt_count;
      sg.kt1 = min(kt_count, sg.kt0 + (end - pos));
    } else {
      const int j = pos / kt_count;
      tile_coords(first + j * stride, sg.tm, sg.tn);
      sg.kt0 = 0;
      sg.kt1 = kt_count;
    }
    sg.pos = pos;
    return sg;
  }
  __device__ Segment first_segment() const { return segment_at(stream ? begin : 0); }
  __device__ Segment next_segment(const Segment& sg) const {
    return segment_at(sg.pos + (sg.kt1 - sg.kt0));
  }
  __device__ bool complete(const Segment& sg) const { return sg.kt0 == 0 && sg.kt1 == kt_count; }
  // Stream mode: the workgroups whose ranges overlap tile t, [g_lo, g_hi].
  __device__ void tile_owners(int t, int& g_lo, int& g_hi) const {
    const int64_t lo = (int64_t)t * kt_count, hi = lo + kt_count;  // [lo, hi)
    int g = (int)(lo * grid / total);
    while (g > 0 && start(g) > lo) --g;
    while (start(g + 1) <= lo) ++g;
    g_lo = g;
    g = (int)((hi - 1) * grid / total);
    while (g > 0 && start(g) > hi - 1) --g;
    while (start(g + 1) <= hi - 1) ++g;
    g_hi = g;
  }
};

// STREAMK: stream-K schedule (the weight-streaming shapes); the large-M
// shapes compile the tile schedule only.
template <int BM, int BN, int WM, int WN, int STAGES, bool STREAMK, int EPI>
__global__ __launch_bounds__(WM* WN * 64) void gemm_tile_kernel(GemmArgs a) {
  using S = TileShape<BM, BN, WM, WN, STAGES>;
  constexpr int BK = S::BK;
  __shared__ __attribute__((aligned(1024))) char lds[S::kLdsBytes];

  const TileWalk walk(a.M, a.N, a.K, BM, BN, BK, STREAMK);
  if (walk.count == 0) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keep in SGPRs
  const int wm = wave / WN;
  const int wn = wave % WN;

  // ---- DMA.  The issue cursor walks the segments in stream order.
  // Instruction u = i * waves + wave of a k-tile: u < XT covers x rows
  // 8u .. 8u+7, else w rows 8(u-XT) ..; either way its 1 KB lands at stage
  // offset u * 1 KB.  Lane -> row + lane/8, position lane%8, source chunk
  // position ^ swz(row).  Rows past M / N clamp to the last row; chunks past
  // K read zeros through an out-of-range buffer offset.
  const int lrow = lane >> 3, lpos = lane & 7;
  Segment isg = walk.first_segment();
  int is_kt = isg.kt0;
  auto issue = [&](int stage) {  // issue the cursor's k-tile, then advance the cursor
    const int m0 = isg.tm * BM, n0 = isg.tn * BN;
    char* base = lds + stage * S::kStageBytes;
    const rsrc_t xr = make_rsrc(reinterpret_cast<const char*>(a.x + (int64_t)m0 * a.ldx) + is_kt * BK * 2);
    const rsrc_t wr = make_rsrc(reinterpret_cast<const char*>(a.w + (int64_t)n0 * a.ldw) + is_kt * BK * 2);
    const int kleft = a.K - is_kt * BK;  // valid K elements in this k-tile
#pragma unroll
    for (int i = 0; i < S::kDma; ++i) {
      const int u = i * S::kWaves + wave;
      const bool is_x = u < S::XT;
      const int r = (is_x ? u : u - S::XT) * S::RPI + lrow;
      const int c = lpos ^ lds_swz(r);
      const int rows_left = is_x ? a.M - 1 - m0 : a.N - 1 - n0;
      const int ld = is_x ? (int)a.ldx : (int)a.ldw;
      unsigned off = (unsigned)(min(r, rows_left) * ld * 2 + c * 16);
      if (c * 8 >= kleft) off = kOutOfRange;
      dma16(is_x ? xr : wr, off, (lds_void*)(base + u * 1024));
    }
    if (++is_kt == isg.kt1) {
      isg = walk.next_segment(isg);
      is_kt = isg.kt0;
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
    xrow_swz[j] = lds_swz(r);
  }
#pragma unroll
  for (int i = 0; i < S::FN; ++i) {
    const int r = wn * S::TN + i * 32 + frow;
    wrow_off[i] = S::kXBytes + r * S::kRowBytes;
    wrow_swz[i] = lds_swz(r);
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
  // full 128-byte lines.  Scratch is written and read through int vectors
  // only, so type-based alias analysis cannot move one block's stores above
  // the previous block's loads.
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
            *reinterpret_cast<i32x2*>(sc_addr(frow, col / 8) + (col % 8) * 2) =
                __builtin_bit_cast(i32x2, o);
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
            *reinterpret_cast<i32x2*>(sc_addr(frow, col / 8) + (col % 8) * 2) =
                __builtin_bit_cast(i32x2, o);
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
    const int t = sg.tm * walk.tiles_n + sg.tn;
    const int slot = sg.pos == walk.begin ? 0 : 1;
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
    __builtin_amdgcn_s_waitcnt(0);  // every wave: its partial stores are acknowledged
    __syncthreads();
    // The arrival result goes through the first word of wave 0's epilogue
    // scratch (free here: every wave has finished its previous epilogue),
    // with a second barrier before anyone may overwrite it.
    volatile int* flag = reinterpret_cast<volatile int*>(lds + S::kStagesBytes);
    if (tid == 0) {
      const unsigned prev = __hip_atomic_fetch_add(a.counters + t, 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
      *flag = prev == (unsigned)(g_hi - g_lo);
    }
    __syncthreads();
    const bool last = *flag != 0;
    __syncthreads();
    if (!last) return false;
    zero_acc();
    const int64_t tile_lo = (int64_t)t * walk.kt_count;
    for (int g = g_lo; g <= g_hi; ++g) {
      // g's segment in this tile is its head iff g's range starts inside the tile.
      const unsigned src = slot_off(g, walk.start(g) >= tile_lo ? 0 : 1);
#pragma unroll
      for (int i = 0; i < S::FN; ++i)
#pragma unroll
        for (int j = 0; j < S::FM; ++j) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x4 v = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           wsr, (int)(src + ((i * S::FM + j) * 4 + q) * 64 * 16), 0, kCoherent));
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] += v[e];
          }
          __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (tid == 0)
      __hip_atomic_store(a.counters + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
  for (int t = 0; t < STAGES; ++t)
    if (t < steps) issue(t);
  if (steps >= STAGES) vm_wait<(STAGES - 1) * S::kDma>();
  else vm_wait<0>();
  __syncthreads();

  Segment csg = walk.first_segment();  // compute cursor
  int ckt = csg.kt0;
  Frags f0, f1;
  if (steps > 0) read(f0, 0, 0);
  int stage = 0;
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
    if (s + STAGES < steps) issue(stage);
    stage = stage + 1 == STAGES ? 0 : stage + 1;
    if (s + 1 < steps) read(f0, stage, 0);
    __builtin_amdgcn_sched_barrier(0);
    mma(f1);
    __builtin_amdgcn_sched_barrier(0);
    if (++ckt == csg.kt1) {
      if constexpr (STREAMK) {
        if (walk.complete(csg) || finish_partial(csg)) epilogue(csg.tm * BM, csg.tn * BN);
      } else {
        epilogue(csg.tm * BM, csg.tn * BN);
      }
      zero_acc();
      if (s + 1 < steps) {
        csg = walk.next_segment(csg);
        ckt = csg.kt0;
      }
    }
  }
}

}  // namespace sys1
