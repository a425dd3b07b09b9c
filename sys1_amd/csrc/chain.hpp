// Arguments of the projection-chain kernel (chain.hip): up to kChainMax
// row-local projections in one persistent launch, projection p reading rows
// that projections before it wrote.
#pragma once

#include "common.hpp"

namespace sys1 {

constexpr int kChainMax = 4;        // projections per launch
constexpr int kChainXcdMax = 8;     // queues (one per XCD)
constexpr int kChainHeader = 16;    // bank words before the dependency counters
constexpr int kChainMaxPanels = 1024;  // row panels per launch (BM = 128: 131072 tokens)
constexpr int kChainBankWords = kChainHeader + kChainMax * kChainMaxPanels;
// The weight-streaming chain's item counters, in the dependency words: per
// projection kStreamSlots counters, one 128-byte line each.
constexpr int kStreamSlots = 16;
constexpr int kStreamSlotStride = 32;
static_assert(kChainHeader + kChainMax * kStreamSlots * kStreamSlotStride <= kChainBankWords, "bank size");
// After the dependency words: kStreamSlots workgroup-exit counters (one
// line each), then the error word; kChainAllocWords in all.
constexpr int kChainExitWords = kChainBankWords;
constexpr int kChainErrWord = kChainExitWords + kStreamSlots * kStreamSlotStride;
constexpr int kChainAllocWords = kChainErrWord + 64;

// Error word bits (sys1hip_chain_status).
constexpr unsigned kChainErrTimeout = 1;    // a dependency wait expired
constexpr unsigned kChainErrUndrained = 2;  // an XCD's queue was not drained (no workgroup ran there)
constexpr unsigned kChainErrXcc = 4;        // a workgroup ran on an XCD id beyond nxcd

struct ChainProj {
  const __bf16* x;      // [M, K] ld ldx
  const __bf16* w;      // [N, K] ld ldw, or blocked (w_kt > 0)
  const __bf16* resid;  // [M, Nout] ld ldr (kEpiResidual), else null
  __bf16* y;            // [M, Nout] ld ldy
  int64_t ldx, ldw, ldr, ldy;
  int N, K, Nout;
  int epi;              // kEpiNone, kEpiResidual, kEpiGeglu or kEpiSwiglu
  int w_kt;             // blocked weight: 64-wide k-tiles per 32-row block; 0: row-major
  int tiles_n;          // column tiles (N / BN, rounded up)
  int kt_count;         // k-tiles (K / 64)
};

struct ChainArgs {
  ChainProj proj[kChainMax];
  unsigned* bank;       // [kChainBankWords]: queue heads, finished count, dependency counters
  unsigned* err;        // error word (kChainErr*), cleared by the host
  int nproj, M, row_panels, nxcd;
  int wait_us;          // real time a dependency wait may take before it gives up
  int dep_extra;        // added to every dependency target (test knob: forces the waits to expire)
  // Optional timeline (null: off): per workgroup, kChainTraceTiles records of
  // 4 x u64 {queue index | xcc << 32 | drained << 40, start, stores done,
  // projection | (epilogue start - start) << 8}, times on the 100 MHz
  // constant clock; the last record holds {~0, kernel entry, first k-tile
  // in LDS, 0}.
  unsigned long long* trace;
};
constexpr int kChainTraceTiles = 64;

// A tile of a queue: projection, row panel, column tile.
struct ChainTile {
  int p, rp, tn;
};

// The tile queue of one XCD: the row panels r with r % nxcd == xcc, every
// projection's tiles on them, projection-major and, inside a projection,
// row-panel-major (tile i of projection p: local panel i / tiles_n, column
// tile i % tiles_n).  A tile's dependencies -- the previous projection's
// tiles on its panel -- come earlier in the same queue.
struct XcdQueue {
  int xcc, nxcd, nproj, R, total;
  int count[kChainMax];    // tiles of each projection in this queue
  int tiles_n[kChainMax];

  __host__ __device__ XcdQueue(int xcc_, int nxcd_, int row_panels, int nproj_, const int* tn)
      : xcc(xcc_), nxcd(nxcd_), nproj(nproj_) {
    R = xcc < row_panels ? (row_panels - xcc + nxcd - 1) / nxcd : 0;
    total = 0;
    for (int p = 0; p < kChainMax; ++p) {
      tiles_n[p] = p < nproj ? tn[p] : 1;
      count[p] = p < nproj ? R * tn[p] : 0;
      total += count[p];
    }
  }
  // Tile i (0 <= i < total) of the queue.
  __host__ __device__ ChainTile decode(int i) const {
    ChainTile t{0, 0, 0};
    int base = 0;
    // the projection: the first p whose cumulative count exceeds i
    for (int p = 0; p + 1 < kChainMax; ++p) {
      if (t.p == p && p + 1 < nproj && i >= base + count[p]) {
        base += count[p];
        t.p = p + 1;
      }
    }
    const int j = i - base;
    const int rl = j / tiles_n[t.p];
    t.tn = j - rl * tiles_n[t.p];
    t.rp = xcc + nxcd * rl;
    return t;
  }
};

struct ChainKernel {
  const void* fn;
  int bm, bn;
  int stages;  // tile chain: LDS stages; weight-streaming chain: the largest K it takes
  int threads;
};
extern const ChainKernel kChainKernel;        // tile chain (128 x 192 tiles)
extern const ChainKernel kStreamChainKernel;  // weight-streaming chain (M <= 64)

}  // namespace sys1
