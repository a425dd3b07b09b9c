// C ABI of the gfx950 projection path (declared in include/sys1hip.h):
// context/stream management, argument validation, kernel table and the
// tile-choice heuristic keyed on the packed token count M.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.hpp"
#include "kernel_fns.hpp"
#include "norm.hpp"
#include "conv.hpp"
#include "chain.hpp"

using namespace sys1;

namespace {

constexpr int kVersion = 100;                        // 0.1.0
constexpr size_t kWorkspaceBytes = 64ull << 20;      // stream-K partials
constexpr int kCounterSlots = 1 << 16;               // stream-K arrival counters (tile x wave)
constexpr int64_t kNormRows = 1 << 20;               // rows of one pre-norm call (row statistics)

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

#define HIP_TRY(expr)                                                                     \
  do {                                                                                    \
    hipError_t e_ = (expr);                                                               \
    if (e_ != hipSuccess) return fail(SYS1HIP_EDEVICE, "%s: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

struct Plan {
  int kernel = 0;
  int64_t grid = 1;
  int64_t dp = 0;  // tiles run whole before the stream phase (stream-K kernels)
  double cost = 1e300;
};

struct PlanKey {
  int64_t M, N, K;
  int epi;
  bool head64, conv;
  bool wide_w;  // x or w spans 2 GiB or more (the skinny kernels' offsets would not reach: skinny_wide)
  bool operator==(const PlanKey& o) const {
    return M == o.M && N == o.N && K == o.K && epi == o.epi && head64 == o.head64 && conv == o.conv &&
           wide_w == o.wide_w;
  }
};

struct PlanKeyHash {
  size_t operator()(const PlanKey& k) const {
    uint64_t h = (uint64_t)k.M * 0x9E3779B97F4A7C15ull;
    h ^= ((uint64_t)k.N * 0xC2B2AE3D27D4EB4Full) + (h << 6) + (h >> 2);
    h ^= ((uint64_t)k.K * 0x165667B19E3779F9ull) + (h << 6) + (h >> 2);
    h ^= (uint64_t)(k.epi * 8 + k.wide_w * 4 + k.head64 * 2 + k.conv) + (h << 6) + (h >> 2);
    return (size_t)h;
  }
};

struct Context {
  int device = 0;
  hipStream_t own = nullptr;
  hipStream_t stream = nullptr;
  hipEvent_t order = nullptr;  // orders a new stream after the old one (sys1hip_set_stream)
  float* ws = nullptr;
  unsigned* counters = nullptr;
  float* stats = nullptr;  // pre-norm row statistics, kNormRows x (mean, 1/std)
  // Projection chains: the dependency bank (zero between launches: each
  // launch's last workgroup clears it) and the error word, one allocation.
  unsigned* chain = nullptr;
  int chain_wait_us = 20000;  // real time a dependency wait may take before it gives up
  int chain_extra = 0;
  int chain_occ = 0;         // resident chain workgroups per CU
  int stream_chain_occ = 0;  // the same for the weight-streaming chain
  unsigned long long* chain_trace = nullptr;  // optional timeline buffer (sys1hip_set_chain_trace)
  int64_t chain_trace_bytes = 0;
  int forced_kernel = -1;
  int forced_grid = 0;
  int forced_dp = -1;
  int cus = 256;
  // Resident workgroups per CU of each (kernel, epilogue) as the runtime
  // reports them (an epilogue that needs more registers can fit fewer).
  std::vector<int> occ;
  const int* occ_fixed = nullptr;  // the same table in static storage (the context-free entry point)
  // Chosen plans of unforced calls, keyed by shape and epilogue: pricing
  // every (kernel, grid) takes several microseconds of host time, more than
  // a small-M projection's kernel.
  std::mutex plan_mu;
  std::unordered_map<PlanKey, Plan, PlanKeyHash> plans;
};

struct KernelEntry {
  const char* name;
  int bm, bn, threads;
  int occupancy;        // resident workgroups per CU (LDS/register bound)
  bool streamk;         // stream-K schedule (weight-streaming shapes)
  float efficiency;     // measured MFMA efficiency of the shape, fitted to a sweep of the
                        // projection shapes (ModernBERT base/large, Qwen, square)
  int bk;               // k-tile depth
  int stages;           // LDS pipeline stages (stages - 1 k-tiles in flight)
  int tn;               // output columns per wave (the RoPE epilogue needs 64: one head)
  int wm;               // waves along M (the conv epilogue needs 1: a wave holds every row)
  int pw;               // producer waves (0: the compute waves issue the refills)
  float swiglu_efficiency;  // efficiency with a SwiGLU epilogue, when it differs (0: the same)
  float long_k_efficiency;  // efficiency for long K (model_cost), when it differs (0: the same)
  const KernelFn* fn;   // [kEpiCount]: the shape's kernel per epilogue (null: not built)
  bool skinny;          // skinny-M kernel (skinny.hpp): one workgroup per bm x bn tile, whole K
};

}  // namespace

// Each shape's kernels are compiled in a translation unit of their own.
#define SYS1_SHAPE(name, BM, BN, WM, WN, ST, BK, OCC, SK, PW, EFF, SWEFF, LKEFF) SYS1_DECLARE_SHAPE(name)
#define SYS1_SKINNY(name, FM, FN, NW, U) SYS1_DECLARE_SHAPE(name)
#include "shapes.def"
#undef SYS1_SHAPE
#undef SYS1_SKINNY

namespace {

// Output-tile shapes, in the order of shapes.def (the kernel ids).
const KernelEntry kKernels[] = {
#define SYS1_SHAPE(name, BM, BN, WM, WN, ST, BK, OCC, SK, PW, EFF, SWEFF, LKEFF) \
  KernelEntry{#name, BM, BN, (WM * WN + PW) * 64, OCC, SK, EFF, BK, ST, BN / WN, WM, PW, SWEFF, LKEFF, sys1::name##_fns, false},
// (skinny entries: tn 16 and wm 0 keep the RoPE and fused-conv calls off them)
#define SYS1_SKINNY(name, FM, FN, NW, U) \
  KernelEntry{#name, 16 * FM, 16 * FN, NW * 64, 1, false, 1.0f, 32, 0, 16, 0, 0, 0.0f, 0.0f, sys1::name##_fns, true},
#include "shapes.def"
#undef SYS1_SHAPE
#undef SYS1_SKINNY
};
constexpr int kNumKernels = sizeof(kKernels) / sizeof(kKernels[0]);

// (the weight-layout bit SYS1HIP_EPI_BLOCKED_W is not an epilogue)
int epi_id_from_flags(int32_t f) {
  switch (f & ~SYS1HIP_EPI_BLOCKED_W) {
    case SYS1HIP_EPI_NONE: return kEpiNone;
    case SYS1HIP_EPI_BIAS: return kEpiBias;
    case SYS1HIP_EPI_GEGLU: return kEpiGeglu;
    case SYS1HIP_EPI_SWIGLU: return kEpiSwiglu;
    case SYS1HIP_EPI_RESIDUAL: return kEpiResidual;
    case SYS1HIP_EPI_BIAS | SYS1HIP_EPI_GELU: return kEpiBiasGelu;
    case SYS1HIP_EPI_BIAS | SYS1HIP_EPI_GELU_TANH: return kEpiBiasGeluTanh;
    case SYS1HIP_EPI_BIAS | SYS1HIP_EPI_RESIDUAL: return kEpiBiasResidual;
    default: return -1;
  }
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Modelled time (in CU clocks) of a projection on kernel `e` launched on
// `grid` workgroups, of which the first `dp` tiles run whole (tile phase)
// and the rest are split over every workgroup (stream phase; stream-K
// kernels only).  A k-tile costs a workgroup the larger of
//   - its compute: MFMA cycles (derated by the shape's fitted efficiency) or
//     operand loads at kLoadBytesPerClk per CU, times the workgroups sharing
//     the CU, and
//   - the load latency spread over the k-tiles in flight (stages - 1).
// A split tile costs its last arriving owner the arrival latency plus
// reading every owner's f32 partial.  The call is bounded below by the
// weight bytes at a sustained HBM rate.  The constants and efficiencies are
// fitted to measured projection shapes (ModernBERT base/large in their
// chains, Qwen 27B at M = 128, square large GEMMs).
constexpr double kFlopPerClk = 4096.0;      // bf16 MFMA per CU per clock
constexpr double kLoadBytesPerClk = 48.0;   // L2 -> LDS per CU
constexpr double kStoreBytesPerClk = 64.0;
// A tile kernel's epilogue: output bytes at this rate, twice the time for an
// epilogue other than the plain store (operand reads, gating), half of it
// hidden when another workgroup on the CU runs MFMAs meanwhile.
constexpr double kTileStoreBytesPerClk = 32.0;
constexpr double kHbmBytesPerClk = 1500.0;  // whole chip, sustained by a weight stream
constexpr double kStreamCuFraction = 0.745;  // of the CUs, to draw the full weight-stream rate
constexpr int64_t kCachedWeightBytes = 32 << 20;  // weights up to this size stay in the caches
constexpr double kRereadShare = 0.25;  // of a streamed weight's re-walks charged at the HBM rate
constexpr double kRereadShareBig = 0.5;  // the same, for weights beyond half the MALL
constexpr double kRereadShareCached = 0.3;  // the same, in clocks of that rate, for weights the caches hold
constexpr int64_t kRereadWeightBytes = 128 << 20;  // half the 256 MB MALL
constexpr double kFixupClk = 2000.0;        // partial write + arrival
constexpr double kLatencyClk = 1500.0;      // load issue -> data in LDS
constexpr int64_t kLongK = 4096;            // see KernelEntry::long_k_efficiency
// From K > kMidK the same rate applies once the activations no longer fit
// one XCD's L2 (2 M K bytes above kXcdL2Bytes): the panels then stream from
// beyond the L2 as well.  Measured on the 256x192 two-stage shape, same box:
// Qwen3.5-small q_k_v at M = 8192 (K = 2048) 142 -> 124 us on 256x160 tiles,
// gate_up at M = 2048 / 3072 93 -> 83 / 136 -> 123 us on 256x128 / 256x160;
// at M = 1024 (x 4 MB, L2-resident) 256x192 stayed the faster (51.6 against
// 55.2 us on 256x256).
constexpr int64_t kMidK = 1536;
constexpr int64_t kXcdL2Bytes = 4 << 20;
// With producer waves a refill is issued as soon as its stage is freed, not
// behind the compute waves' MFMAs: a shorter effective latency (when every
// CU runs at least one workgroup).
constexpr double kProducerLatencyClk = 900.0;

int occupancy(const Context* c, int id, int epi) {
  const int n = c->occ_fixed ? c->occ_fixed[(size_t)id * kEpiCount + epi]
                : c->occ.empty() ? 0 : c->occ[(size_t)id * kEpiCount + epi];
  return n > 0 ? std::min(n, kKernels[id].occupancy) : kKernels[id].occupancy;
}

// A kernel whose epilogue variant fits fewer workgroups per CU than its
// shape was fitted with loses the overlap between them: 0.7 of the rate
// (measured: the 128x128 producer-wave shape with a LayerNorm epilogue at
// one workgroup per CU against the plain shape at two).
constexpr double kLowOccupancyRate = 0.7;

double model_cost(const Context* c, int id, int epi, int64_t M, int64_t N, int64_t K,
                  int64_t grid, int64_t dp) {
  const KernelEntry& e = kKernels[id];
  const int64_t tiles = cdiv(M, e.bm) * cdiv(N, e.bn);
  const int64_t kts = cdiv(K, e.bk);
  // Workgroups on the busiest CU: a grid between one and two per CU leaves
  // some CUs running two, and those set the launch's time.
  const double share = (double)std::max<int64_t>(1, cdiv(grid, c->cus));
  double base_eff =
      epi_base(epi) == kEpiSwiglu && e.swiglu_efficiency > 0.0f ? e.swiglu_efficiency : e.efficiency;
  const bool long_k = K > kLongK || (K > kMidK && 2 * M * K > kXcdL2Bytes);
  if (long_k && e.long_k_efficiency > 0.0f) base_eff = e.long_k_efficiency;
  const double eff = base_eff * (occupancy(c, id, epi) < e.occupancy ? kLowOccupancyRate : 1.0);
  const double mfma = 2.0 * e.bm * e.bn * e.bk / kFlopPerClk / eff;
  const double load = (double)(e.bm + e.bn) * e.bk * 2.0 / kLoadBytesPerClk;
  // (A grid below one workgroup per CU leaves each workgroup's load latency
  // exposed: measured ~2200 cycles per k-tile for one 128x128 producer-wave
  // workgroup per CU streaming a cold weight.)
  // A shape fitted for two workgroups per CU, alone on its CU (grid at most
  // the CU count), is priced the same way: measured ~2160 cycles per k-tile
  // for the 128x128 producer-wave shape on 256 tiles of 1024x2624.
  const bool lone_pair = occupancy(c, id, epi) >= 2 && grid <= c->cus;
  const double latency = e.pw && grid >= c->cus && !lone_pair ? kProducerLatencyClk : kLatencyClk;
  const double per_kt = std::max(share * std::max(mfma, load), latency / (e.stages - 1));
  const double store =
      e.streamk ? share * 2.0 * e.bm * e.bn / kStoreBytesPerClk
                : share * 2.0 * e.bm * e.bn / kTileStoreBytesPerClk * (epi == kEpiNone ? 1.0 : 2.0) *
                      (occupancy(c, id, epi) >= 2 ? 0.5 : 1.0);
  // The weight stream's floor.  Up to 128 tokens in one tile row,
  // fewer than ~3/4 of the CUs cannot draw the chip's rate: measured on
  // Qwen3.5-27B gate_up at M = 128 (one round of whole tiles), 182 CUs
  // streamed 4.64 TB/s and 218 CUs 4.86 TB/s.  (Applied at M = 129-256 the
  // same rule chose narrower tiles that ran slower: the 27B and
  // Qwen3.5-small stacks at M = 256 lost 6-7%.)
  const double active = (double)std::min<int64_t>(grid, c->cus);
  const double cu_floor = M <= 128 && cdiv(M, e.bm) == 1 ? std::max(1.0, kStreamCuFraction * c->cus / active) : 1.0;
  // A stream-K weight beyond the caches is walked once per row panel, and
  // part of each walk after the first comes from HBM again: measured on
  // the 27B out_proj (63 MB) at M = 272, 102.8 us on nine 32-row panels
  // against 60.9 us on three 128-row panels.  Beyond half the MALL the
  // share is larger: the 27B down (178 MB) at M = 512 / 768 ran 145.7 /
  // 211.8 us on 128-row panels against 112.8 / 155.9 on 256-row ones
  // (~17 us per extra walk, against ~1 us for out_proj at M = 512).  A
  // weight the caches hold still pays for its walks in clocks: the
  // Qwen3.5-small out_proj (16 MB) at M = 960 ran 65.9 us on thirty 32-row
  // panels against 38.5 us on eight 128-row ones, its down (24 MB) at
  // M = 576 59.0 against 40.1 us.
  const double reread_share = 2 * N * K > kRereadWeightBytes   ? kRereadShareBig
                              : 2 * N * K > kCachedWeightBytes ? kRereadShare
                                                               : kRereadShareCached;
  const double rereads = e.streamk ? 1.0 + reread_share * (double)(cdiv(M, e.bm) - 1) : 1.0;
  const double hbm = 2.0 * (double)N * K / kHbmBytesPerClk * cu_floor * rereads;
  double t = (double)cdiv(dp, grid) * (kts * per_kt + store);
  const int64_t st = tiles - dp;
  if (st > 0) {
    const int64_t total = st * kts;
    const int64_t sg = std::min(grid, total);  // workgroups in the stream phase
    t += (double)cdiv(total, sg) * per_kt + ((double)cdiv(st, sg) + 1.0) * store;
    if (total % sg != 0 || sg > st) {
      const double owners = std::min<double>((double)sg, (double)sg / st + 1.0);
      t += kFixupClk + owners * e.bm * e.bn * 4.0 / kLoadBytesPerClk;
      t += 2.0 * 2.0 * sg * e.bm * e.bn * 4.0 / kHbmBytesPerClk;  // partial traffic
    }
  }
  return std::max(t, hbm);
}

int64_t max_grid(const Context* c, int id, int epi, int64_t M, int64_t N, int64_t K) {
  const KernelEntry& e = kKernels[id];
  if (e.skinny) return cdiv(M, e.bm) * cdiv(N, e.bn);  // one workgroup per tile
  const int64_t tiles = cdiv(M, e.bm) * cdiv(N, e.bn);
  int64_t g = (int64_t)c->cus * occupancy(c, id, epi);
  if (!e.streamk) return std::min(g, tiles);
  g = std::min(g, tiles * cdiv(K, e.bk));
  while (g > 1 && 2 * g * e.bm * e.bn * 4 > (int64_t)kWorkspaceBytes) --g;
  return g;
}

// Between two stream-K plans the model prices the same (both at the weight
// stream's HBM floor), whether plan (id, dp) is to be preferred to `best`:
// the shorter tile height that still covers M (fewer padded rows, less x
// and partial traffic), then producer waves, then more tiles run whole
// before the stream phase (fewer split tiles).  Measured on the Qwen3.5-27B
// weights: at M = 16 the 32-row shape ran down / q_k_v / in_proj 5-12%
// faster than the 64-row one; at M = 128 the gate/up projection ran
// 86.7 us on 128x128 producer-wave tiles with one whole round of tiles
// first, against 88.7 us on 128x256 tiles and 90.0 us in pure stream-K.
bool stream_preferred(int id, int64_t dp, const Plan& best, int64_t M) {
  const KernelEntry& a = kKernels[id];
  const KernelEntry& b = kKernels[best.kernel];
  if (!a.streamk || !b.streamk) return false;
  const bool afit = a.bm >= M, bfit = b.bm >= M;
  if (afit != bfit) return afit;
  if (a.bm != b.bm) return afit ? a.bm < b.bm : a.bm > b.bm;
  if ((a.pw > 0) != (b.pw > 0)) return a.pw > 0;
  return id == best.kernel && dp > best.dp;
}

// Prices kernel `id` on `grid` workgroups and keeps it in *best when it is
// cheaper.  Tile kernels run every tile whole.  Stream-K kernels try: pure
// stream-K, the hybrid whose stream phase is the last partial round of
// tiles, and the hybrid whose stream phase also takes one full round (more
// iterations per workgroup, fewer owners per split tile).
void consider(const Context* c, int id, int epi, int64_t M, int64_t N, int64_t K, int64_t grid, Plan* best) {
  const KernelEntry& e = kKernels[id];
  const int64_t tiles = cdiv(M, e.bm) * cdiv(N, e.bn);
  int64_t cand[3] = {tiles, -1, -1};
  if (e.streamk && c->forced_dp >= 0) {
    cand[0] = std::min<int64_t>(c->forced_dp, tiles);
  } else if (e.streamk) {
    const int64_t whole = tiles / grid * grid;
    cand[0] = 0;
    if (whole > 0 && whole < tiles) cand[1] = whole;
    if (whole > grid && whole < tiles) cand[2] = whole - grid;
    if (whole == tiles) cand[1] = tiles;
  }
  for (int64_t dp : cand) {
    if (dp < 0 || (tiles - dp) * (e.threads / 64) > kCounterSlots) continue;
    const double cost = model_cost(c, id, epi, M, N, K, grid, dp);
    const bool tie = best->kernel >= 0 && cost <= best->cost * 1.001 && cost >= best->cost * 0.999;
    if (cost < best->cost * 0.999 || (tie && stream_preferred(id, dp, *best, M))) {
      best->kernel = id, best->grid = grid, best->dp = dp, best->cost = cost;
    }
  }
}

// Plan of a call: the cheapest modelled (kernel, grid, dp) over the shapes
// allowed for M (stream-K shapes where M fits their tile height or their
// tiles cannot fill the CUs, tile shapes above 128 tokens), or over the
// forced kernel, grid and/or dp.  Stream-K grids from a quarter of
// the slots up to all of them are tried.
// Rows a kernel computes for M outputs when its tile rows overlap by `halo`
// (the conv epilogue): whole tile rows, as the tile schedule counts them.
int64_t halo_rows(const KernelEntry& e, int64_t M, int halo) {
  if (halo == 0 || M <= e.bm) return M;
  return (1 + cdiv(M - e.bm, e.bm - halo)) * e.bm;
}

// conv: only shapes with a conv epilogue (waves spanning every row), priced
// on the rows their overlapping tile rows compute.

// The skinny-M kernel for a call, or -1.  A skinny workgroup reads its BN
// weight rows and its BM rows of x over the whole K, and one round of
// tiles (at most one workgroup per CU) is allowed, so each CU moves
//   (BM + BN) * K * 2 bytes
// through its load path; the one-round shape with the fewest such bytes is
// taken (ties: the first listed), and the skinny kernels win while that
// stays within kSkinnyCuBytes.  Measured over the ModernBERT-base/large and
// Qwen3.5-small projections at M = 16..4096: one round at up to ~420 KB per
// CU ran 1.1-1.9x faster than the stream-K and tile kernels.  Between 576
// and 704 KB the one-round skinny plans still won, same box (Qwen3.5 vision
// fc2 at M = 128 on 32x32 tiles 28.6 -> 21.8 us, Qwen3.5-small down at
// M = 64 26.3 -> 24.5, ModernBERT-large mlp.Wo at M = 1024 on 64x64 tiles
// 27.5 -> 25.9); from 768 KB up they lost (Qwen3.5-small down at M = 128
// 28.2 -> 31.1 us, ModernBERT-large mlp.Wo at M = 2048 36.5 -> 38.9).
// Shapes needing two or more rounds lost (the Qwen3.5-small
// q/k/v at M = 64 on 288 16-wide tiles: 26 against 23 us; ModernBERT-base
// Wqkv at M = 1024 on three rounds of 64x48 tiles: 24 against 15 us).
// Above kSkinnyWeightBytes the weight is streamed from HBM and needs the
// stream-K schedule's spread of K over every CU.
constexpr int64_t kSkinnyMaxM = 4096;
constexpr int64_t kSkinnyWeightBytes = 32 << 20;
constexpr int64_t kSkinnyCuBytes = 704 << 10;

// The skinny kernels address x and w through one buffer descriptor each,
// based at row 0, with 32-bit byte offsets: a call whose operands span 2 GiB
// or more from there (a strided x view, a huge weight) cannot run on them.
bool skinny_wide(int64_t M, int64_t K, int64_t ldx, int64_t N, int64_t ldw) {
  return 2 * (M - 1) * ldx + 2 * K >= 0x7ffffff0ll || 2 * N * ldw >= 0x7ffffff0ll;
}

int skinny_pick(const Context* c, int64_t M, int64_t N, int64_t K, bool wide, int epi) {
  if (M > kSkinnyMaxM || 2 * N * K > kSkinnyWeightBytes || wide) return -1;
  int best = -1;
  int64_t best_bytes = 0;
  for (int id = 0; id < kNumKernels; ++id) {
    const KernelEntry& e = kKernels[id];
    if (!e.skinny || !e.fn[epi]) continue;
    if (cdiv(M, e.bm) * cdiv(N, e.bn) > c->cus) continue;  // one round
    const int64_t bytes = (e.bm + e.bn) * K * 2;
    if (best < 0 || bytes < best_bytes) best = id, best_bytes = bytes;
  }
  return best >= 0 && best_bytes <= kSkinnyCuBytes ? best : -1;
}

Plan price_plans(const Context* c, int64_t M0, int64_t N, int64_t K, bool wide, int epi, bool head64,
                 bool conv) {
  Plan best;
  // (a forced grid or split asks for a persistent kernel: no skinny pick)
  if (c->forced_kernel < 0 && c->forced_grid <= 0 && c->forced_dp < 0 && !head64 && !conv) {
    const int id = skinny_pick(c, M0, N, K, wide, epi);
    if (id >= 0) {
      best.kernel = id, best.grid = cdiv(M0, kKernels[id].bm) * cdiv(N, kKernels[id].bn), best.dp = 0,
      best.cost = 0.0;
      return best;
    }
  }
  for (int id = 0; id < kNumKernels; ++id) {
    if (c->forced_kernel >= 0 && id != c->forced_kernel) continue;
    const KernelEntry& e = kKernels[id];
    if (!e.fn[epi]) continue;
    if (e.skinny) {
      // (only when forced: the automatic choice is skinny_pick's; the grid
      // is one workgroup per tile, whatever grid is forced)
      if (c->forced_kernel != id || head64 || conv || wide) continue;
      best.kernel = id, best.grid = cdiv(M0, e.bm) * cdiv(N, e.bn), best.dp = 0, best.cost = 0.0;
      continue;
    }
    if (head64 && e.tn != 64) continue;
    if (conv && e.wm != 1) continue;
    const int64_t M = conv ? halo_rows(e, M0, kConvHalo) : M0;
    if (c->forced_kernel < 0) {
      // Measured in the projection chains: the large-M hybrid loses to the
      // plain tile schedule (every split tile moves two f32 partials across
      // the fabric), so stream-K is offered where M fits one tile row, or,
      // above 256 tokens, where the tiles cannot fill the CUs (few tiles,
      // deep K).  Up to 256 tokens the weight stream dominates, and a tile
      // shorter than M would stream the weight from HBM once per tile row;
      // a weight of at most kCachedWeightBytes is re-read from L2 and MALL
      // instead (measured: ModernBERT-large's mlp.Wo, 256x1024x2624, 17.8 us
      // on 64-row stream tiles against 24.9 us on the best tile plan).
      // Up to kRereadWeightBytes, two tile rows (one re-read, from MALL)
      // still pay: the 27B out_proj at M = 256 (63 MB) ran 41.8 us on
      // 128-row stream tiles against 77 us on the best tile plan.
      const bool reread_ok = 2 * N * K <= kCachedWeightBytes ||
                             (2 * N * K <= kRereadWeightBytes && cdiv(M, e.bm) <= 2);
      if (e.streamk && M > e.bm && ((M <= 256 && !reread_ok) || cdiv(M, e.bm) * cdiv(N, e.bn) >= c->cus))
        continue;
      // Tile shapes up to 128 tokens only above 64 tokens (a 128-row tile at
      // least half used) and as one round of whole tiles over at least two
      // thirds of the CUs: the weight then streams with no
      // split tile to fix up (measured: Qwen3.5-27B gate_up at M = 128,
      // 182 tiles of 128x192, 76.0 us against 81.6-84.1 us on the stream-K
      // hybrid whose 16 split tiles are summed after the stream).
      const int64_t whole = cdiv(M, e.bm) * cdiv(N, e.bn);
      if (!e.streamk && M <= 128 &&
          !(M > 64 && cdiv(M, e.bm) == 1 && whole <= (int64_t)c->cus && 3 * whole >= 2 * (int64_t)c->cus))
        continue;
    }
    const int64_t gmax = max_grid(c, id, epi, M, N, K);
    if (c->forced_grid > 0) {
      consider(c, id, epi, M, N, K, std::min<int64_t>(c->forced_grid, gmax), &best);
      continue;
    }
    // A weight streamed from HBM (above kCachedWeightBytes) takes every CU:
    // measured on the 27B projections at M = 128 and 256, the full stream-K
    // grid was the fastest or within 3% of it, where the model's smaller
    // grids (a quarter to a half of the CUs) ran up to 34% slower.  Small
    // weights with short K keep the search (fewer owners per split tile).
    const int64_t gmin = e.streamk && M <= e.bm && 2 * N * K <= kCachedWeightBytes
                             ? std::max<int64_t>(1, gmax / 4)
                             : gmax;
    for (int64_t g = gmax; g >= gmin; g -= std::max<int64_t>(1, gmax / 16))
      consider(c, id, epi, M, N, K, g, &best);
  }
  if (best.cost == 1e300) best.kernel = -1;  // (a forced kernel that cannot run the call)
  return best;
}

// The plan for a call: priced once per (M, N, K, epilogue, head64, conv)
// and kept in the context, unless a kernel, grid or split is forced.  The
// cache is cleared when it reaches kPlanCacheMax entries (ragged serving
// sees many distinct M).
constexpr size_t kPlanCacheMax = 1 << 14;

Plan resolve(Context* c, int64_t M0, int64_t N, int64_t K, bool wide, int epi, bool head64 = false,
             bool conv = false) {
  if (c->forced_kernel >= 0 || c->forced_grid > 0 || c->forced_dp >= 0)
    return price_plans(c, M0, N, K, wide, epi, head64, conv);
  const PlanKey key{M0, N, K, epi, head64, conv, wide};
  std::lock_guard<std::mutex> lock(c->plan_mu);
  auto it = c->plans.find(key);
  if (it != c->plans.end()) return it->second;
  if (c->plans.size() >= kPlanCacheMax) c->plans.clear();
  const Plan p = price_plans(c, M0, N, K, wide, epi, head64, conv);
  c->plans.emplace(key, p);
  return p;
}

// Tile rows per raster group (tiles in flight together share x row panels
// and w column panels in L2).  Measured over the projection chains: 3 is
// best to within noise for K up to 6144 (2-6% above 4 on ModernBERT-base and
// Qwen3.5-small), 4 for the deep-K projections (Qwen3.5-27B down, K = 17408).
int raster_group(int64_t K) { return K > 8192 ? 4 : 3; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Bytes of a weight [N, K] in the blocked layout (see GemmArgs::w_kt).
int64_t blocked_bytes(int64_t N, int64_t K) { return cdiv(N, kBlkRows) * cdiv(K, kBlkK) * kBlkBytes; }

// Row-major [N, ldw] -> blocked layout, 16 bytes per thread; rows past N
// and k past K are zeros.
__global__ void pack_blocked_kernel(const __bf16* __restrict__ w, int64_t ldw, i32x4* __restrict__ out, int64_t N,
                                    int64_t K, int64_t kt_count, int64_t total) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // 16-byte unit of the output
  if (idx >= total) return;
  const int64_t blk = idx / (kBlkBytes / 16), in = idx % (kBlkBytes / 16);
  const int64_t rb = blk / kt_count, kt = blk % kt_count;
  const int64_t n = rb * kBlkRows + in / (kBlkK / 8), k = kt * kBlkK + (in % (kBlkK / 8)) * 8;
  i32x4 v = {0, 0, 0, 0};
  if (n < N && k < K) v = *reinterpret_cast<const i32x4*>(w + n * ldw + k);  // (K % 8 == 0: whole chunks)
  out[idx] = v;
}

__global__ void pack_gated_kernel(const i32x4* __restrict__ w, i32x4* __restrict__ out,
                                  int64_t N, int64_t kv) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= N * kv) return;
  const int64_t p = idx / kv;
  const int64_t k = idx % kv;
  const int64_t I = N / 2;
  const int64_t g = p / (2 * SYS1HIP_GATE_GROUP);
  const int64_t r = p % (2 * SYS1HIP_GATE_GROUP);
  const int64_t src = r < SYS1HIP_GATE_GROUP ? g * SYS1HIP_GATE_GROUP + r
                                             : I + g * SYS1HIP_GATE_GROUP + (r - SYS1HIP_GATE_GROUP);
  out[p * kv + k] = w[src * kv + k];
}

int use_device(Context* c) {
  int cur = -1;
  HIP_TRY(hipGetDevice(&cur));
  if (cur != c->device) HIP_TRY(hipSetDevice(c->device));
  return SYS1HIP_OK;
}

// Argument checks of sys1hip_linear_bf16 (and its context-free variant).
int check_linear(const char* who, const uint16_t* x, int64_t ldx, const uint16_t* w, int64_t ldw,
                 const uint16_t* bias, const uint16_t* residual, int64_t ldr, uint16_t* y, int64_t ldy,
                 int64_t M, int64_t N, int64_t K, int32_t epilogue) {
  const int epi = epi_id_from_flags(epilogue);
  if (epi < 0) return fail(SYS1HIP_EINVAL, "%s: unsupported epilogue flags %d", who, epilogue);
  if (M < 0 || N <= 0 || K <= 0)
    return fail(SYS1HIP_EINVAL, "%s: bad shape M=%lld N=%lld K=%lld", who, (long long)M, (long long)N,
                (long long)K);
  const bool gated = epi_gated(epi);
  if (gated && (N % (2 * SYS1HIP_GATE_GROUP)) != 0)
    return fail(SYS1HIP_EINVAL, "%s: gated epilogue needs N %% 32 == 0 (N=%lld)", who, (long long)N);
  const int64_t nout = gated ? N / 2 : N;
  if (M == 0) return SYS1HIP_OK;
  if (!x || !w || !y) return fail(SYS1HIP_EINVAL, "%s: null x, w or y", who);
  const bool want_bias = epilogue & SYS1HIP_EPI_BIAS;
  const bool want_res = epilogue & SYS1HIP_EPI_RESIDUAL;
  if (want_bias != (bias != nullptr))
    return fail(SYS1HIP_EINVAL, "%s: bias pointer %s but epilogue flags %d", who, bias ? "given" : "missing",
                epilogue);
  if (want_res != (residual != nullptr))
    return fail(SYS1HIP_EINVAL, "%s: residual pointer %s but epilogue flags %d", who,
                residual ? "given" : "missing", epilogue);
  const bool blocked = epilogue & SYS1HIP_EPI_BLOCKED_W;  // (ldw unused: the blocked layout has none)
  if (ldx < K || (!blocked && ldw < K) || ldy < nout || (want_res && ldr < nout))
    return fail(SYS1HIP_EINVAL, "%s: leading dimension too small (ldx=%lld ldw=%lld ldy=%lld ldr=%lld)", who,
                (long long)ldx, (long long)ldw, (long long)ldy, (long long)ldr);
  if (K % 8 || ldx % 8 || (!blocked && ldw % 8))
    return fail(SYS1HIP_EALIGN, "%s: K, ldx and ldw must be multiples of 8", who);
  if (!aligned16(x) || !aligned16(w)) return fail(SYS1HIP_EALIGN, "%s: x and w must be 16-byte aligned", who);
  if (M > (1ll << 30) || N > (1ll << 30) || K > (1ll << 30))
    return fail(SYS1HIP_ERANGE, "%s: dimension above 2^30", who);
  if (blocked && blocked_bytes(N, K) > 0x7ffffff0ll)
    return fail(SYS1HIP_ERANGE, "%s: blocked weight above 2 GiB", who);
  return SYS1HIP_OK;
}

// The row length the plan's 2 GiB offset check sees: the caller's ldw, or
// for a blocked weight the padded row of its layout (same total bytes).
int64_t plan_ldw(int64_t ldw, int64_t K, int32_t epilogue) {
  return (epilogue & SYS1HIP_EPI_BLOCKED_W) ? cdiv(K, kBlkK) * kBlkK : ldw;
}

// Launch a checked projection on `plan` with the given stream-K workspace
// (kWorkspaceBytes of partials, kCounterSlots arrival counters).
int launch_linear(const char* who, const Context* c, const Plan& p, hipStream_t stream, float* ws,
                  unsigned* counters, const uint16_t* x, int64_t ldx, const uint16_t* w, int64_t ldw,
                  const uint16_t* bias, const uint16_t* residual, int64_t ldr, uint16_t* y, int64_t ldy,
                  int64_t M, int64_t N, int64_t K, int epi, bool blocked) {
  (void)c;
  if (p.kernel < 0) return fail(SYS1HIP_EINVAL, "%s: the forced kernel does not fit this call", who);
  const KernelEntry& e = kKernels[p.kernel];
  const int64_t grid = p.grid;
  if (e.streamk && (cdiv(M, e.bm) * cdiv(N, e.bn) - p.dp) * (e.threads / 64) > kCounterSlots)
    return fail(SYS1HIP_ERANGE, "%s: more split tiles than stream-K counters", who);
  GemmArgs a = {};
  a.x = reinterpret_cast<const __bf16*>(x);
  a.w = reinterpret_cast<const __bf16*>(w);
  a.bias = reinterpret_cast<const __bf16*>(bias);
  a.resid = reinterpret_cast<const __bf16*>(residual);
  a.y = reinterpret_cast<__bf16*>(y);
  a.ws = ws;
  a.counters = counters;
  a.ldx = ldx, a.ldw = ldw, a.ldr = ldr, a.ldy = ldy;
  a.M = (int)M, a.N = (int)N, a.K = (int)K, a.Nout = (int)(epi_gated(epi) ? N / 2 : N);
  a.dp_tiles = (int)std::min<int64_t>(p.dp, 1 << 30);
  a.group_m = raster_group(K);
  a.w_kt = blocked ? (int)cdiv(K, kBlkK) : 0;
  if (grid <= 0 || grid > 0x7fffffff) return fail(SYS1HIP_ERANGE, "%s: grid of %lld workgroups", who, (long long)grid);
  hipLaunchKernelGGL(e.fn[epi], dim3((unsigned)grid), dim3(e.threads), 0, stream, a);
  HIP_TRY(hipGetLastError());
  return SYS1HIP_OK;
}

}  // namespace

extern "C" {

int sys1hip_version(void) { return kVersion; }

int sys1hip_kernel_count(void) { return kNumKernels; }

const char* sys1hip_kernel_name(int32_t id) {
  return (id >= 0 && id < kNumKernels) ? kKernels[id].name : nullptr;
}

const char* sys1hip_last_error(void* ctx) {
  (void)ctx;
  return g_last_error.c_str();
}

int sys1hip_init(int device, void** out) {
  if (!out) return fail(SYS1HIP_EINVAL, "sys1hip_init: null output pointer");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= 0)
    return fail(SYS1HIP_EDEVICE, "sys1hip_init: no HIP device (%s)", hipGetErrorString(e));
  if (device < 0 || device >= n)
    return fail(SYS1HIP_EINVAL, "sys1hip_init: device %d out of range (0..%d)", device, n - 1);
  HIP_TRY(hipSetDevice(device));
  Context* c = new Context();
  c->device = device;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) == hipSuccess && prop.multiProcessorCount > 0)
    c->cus = prop.multiProcessorCount;
  if (hipStreamCreateWithFlags(&c->own, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreateWithFlags(&c->order, hipEventDisableTiming) != hipSuccess ||
      hipMalloc(&c->ws, kWorkspaceBytes) != hipSuccess ||
      hipMalloc(&c->counters, kCounterSlots * sizeof(unsigned)) != hipSuccess ||
      hipMalloc(&c->stats, kNormRows * 2 * sizeof(float)) != hipSuccess ||
      hipMalloc(&c->chain, kChainAllocWords * sizeof(unsigned)) != hipSuccess ||
      hipMemsetAsync(c->counters, 0, kCounterSlots * sizeof(unsigned), c->own) != hipSuccess ||
      hipMemsetAsync(c->chain, 0, kChainAllocWords * sizeof(unsigned), c->own) != hipSuccess ||
      hipStreamSynchronize(c->own) != hipSuccess) {
    const char* msg = hipGetErrorString(hipGetLastError());
    if (c->chain) (void)hipFree(c->chain);
    if (c->stats) (void)hipFree(c->stats);
    if (c->counters) (void)hipFree(c->counters);
    if (c->ws) (void)hipFree(c->ws);
    if (c->order) (void)hipEventDestroy(c->order);
    if (c->own) (void)hipStreamDestroy(c->own);
    delete c;
    return fail(SYS1HIP_EDEVICE, "sys1hip_init: device set-up failed (%s)", msg);
  }
  c->stream = c->own;
  c->occ.assign((size_t)kNumKernels * kEpiCount, 0);
  for (int id = 0; id < kNumKernels; ++id)
    for (int epi = 0; epi < kEpiCount; ++epi) {
      int n = 0;
      const KernelFn fn = kKernels[id].fn[epi];
      if (fn && hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(fn),
                                                             kKernels[id].threads, 0) == hipSuccess)
        c->occ[(size_t)id * kEpiCount + epi] = n;
    }
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&c->chain_occ, kChainKernel.fn, kChainKernel.threads, 0) !=
      hipSuccess)
    c->chain_occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&c->stream_chain_occ, kStreamChainKernel.fn,
                                                   kStreamChainKernel.threads, 0) != hipSuccess)
    c->stream_chain_occ = 0;
  (void)hipGetLastError();
  *out = c;
  return SYS1HIP_OK;
}

int sys1hip_destroy(void* ctx) {
  if (!ctx) return fail(SYS1HIP_EINVAL, "sys1hip_destroy: null context");
  Context* c = static_cast<Context*>(ctx);
  int rc = use_device(c);
  if (rc) return rc;
  HIP_TRY(hipStreamSynchronize(c->stream));
  (void)hipFree(c->chain);
  (void)hipFree(c->stats);
  (void)hipFree(c->counters);
  (void)hipFree(c->ws);
  (void)hipEventDestroy(c->order);
  (void)hipStreamDestroy(c->own);
  delete c;
  return SYS1HIP_OK;
}

int sys1hip_set_stream(void* ctx, void* stream) {
  if (!ctx) return fail(SYS1HIP_EINVAL, "sys1hip_set_stream: null context");
  Context* c = static_cast<Context*>(ctx);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (s == c->stream) return SYS1HIP_OK;
  int rc = use_device(c);
  if (rc) return rc;
  // The context's workspace, counters and row statistics are shared by all
  // its calls: work enqueued after the switch waits for work enqueued
  // before it.  (Not while a graph is being captured on either stream: a
  // wait on an event from outside the capture is not capturable.)
  hipStreamCaptureStatus old_st = hipStreamCaptureStatusNone, new_st = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(c->stream, &old_st));
  HIP_TRY(hipStreamIsCapturing(s, &new_st));
  if (old_st == hipStreamCaptureStatusNone && new_st == hipStreamCaptureStatusNone) {
    HIP_TRY(hipEventRecord(c->order, c->stream));
    HIP_TRY(hipStreamWaitEvent(s, c->order, 0));
  }
  c->stream = s;
  return SYS1HIP_OK;
}

int sys1hip_sync(void* ctx) {
  if (!ctx) return fail(SYS1HIP_EINVAL, "sys1hip_sync: null context");
  Context* c = static_cast<Context*>(ctx);
  int rc = use_device(c);
  if (rc) return rc;
  HIP_TRY(hipStreamSynchronize(c->stream));
  return SYS1HIP_OK;
}

// The query above without a device: the fitted occupancies stand in for the
// runtime's (the same numbers unless an epilogue variant spills).
int sys1hip_plan_kernel(int32_t cus, int64_t M, int64_t N, int64_t K, int32_t epilogue, int64_t* grid,
                        char* name, int64_t cap) {
  return sys1hip_plan_kernel_strided(cus, M, N, K, K, K, epilogue, grid, name, cap);
}

int sys1hip_plan_kernel_strided(int32_t cus, int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldw,
                                int32_t epilogue, int64_t* grid, char* name, int64_t cap) {
  if (ldx < K || ldw < K) return fail(SYS1HIP_EINVAL, "sys1hip_plan_kernel: ldx/ldw below K");
  if (cus <= 0) return fail(SYS1HIP_EINVAL, "sys1hip_plan_kernel: %d CUs", (int)cus);
  if (epi_id_from_flags(epilogue) < 0)
    return fail(SYS1HIP_EINVAL, "sys1hip_plan_kernel: unsupported epilogue flags %d", epilogue);
  if (M <= 0 || N <= 0 || K <= 0) return fail(SYS1HIP_EINVAL, "sys1hip_plan_kernel: bad shape");
  const int epi = epi_id_from_flags(epilogue);
  if (epi_gated(epi) && N % (2 * SYS1HIP_GATE_GROUP) != 0)
    return fail(SYS1HIP_EINVAL, "sys1hip_plan_kernel: gated N must be a multiple of %d", 2 * SYS1HIP_GATE_GROUP);
  Context c;  // no device: cus and the fitted occupancies only
  c.cus = cus;
  const Plan p = price_plans(&c, M, N, K, skinny_wide(M, K, ldx, N, plan_ldw(ldw, K, epilogue)), epi, false, false);
  if (p.kernel < 0) return fail(SYS1HIP_EINVAL, "sys1hip_plan_kernel: no kernel fits this call");
  if (grid) *grid = p.grid;
  if (name && cap > 0) {
    std::string s = kKernels[p.kernel].name;
    s += "_g" + std::to_string(p.grid);
    const int64_t tiles = cdiv(M, kKernels[p.kernel].bm) * cdiv(N, kKernels[p.kernel].bn);
    if (kKernels[p.kernel].streamk && p.dp > 0 && p.dp < tiles) s += "_dp" + std::to_string(p.dp);
    snprintf(name, (size_t)cap, "%s", s.c_str());
  }
  return p.kernel;
}

int sys1hip_set_kernel(void* ctx, int32_t id) {
  if (!ctx) return fail(SYS1HIP_EINVAL, "sys1hip_set_kernel: null context");
  if (id < -1 || id >= kNumKernels)
    return fail(SYS1HIP_EINVAL, "sys1hip_set_kernel: kernel id %d out of range", id);
  static_cast<Context*>(ctx)->forced_kernel = id;
  return SYS1HIP_OK;
}

int sys1hip_set_grid(void* ctx, int32_t workgroups) {
  if (!ctx) return fail(SYS1HIP_EINVAL, "sys1hip_set_grid: null context");
  if (workgroups < 0) return fail(SYS1HIP_EINVAL, "sys1hip_set_grid: negative grid %d", workgroups);
  static_cast<Context*>(ctx)->forced_grid = workgroups;
  return SYS1HIP_OK;
}

int sys1hip_set_dp_tiles(void* ctx, int32_t tiles) {
  if (!ctx) return fail(SYS1HIP_EINVAL, "sys1hip_set_dp_tiles: null context");
  if (tiles < -1) return fail(SYS1HIP_EINVAL, "sys1hip_set_dp_tiles: %d below -1", tiles);
  static_cast<Context*>(ctx)->forced_dp = tiles;
  return SYS1HIP_OK;
}

int sys1hip_query_kernel(void* ctx, int64_t M, int64_t N, int64_t K, int32_t epilogue, char* name,
                         int64_t cap) {
  if (!ctx) return fail(SYS1HIP_EINVAL, "sys1hip_query_kernel: null context");
  if (epi_id_from_flags(epilogue) < 0)
    return fail(SYS1HIP_EINVAL, "sys1hip_query_kernel: unsupported epilogue flags %d", epilogue);
  Context* c = static_cast<Context*>(ctx);
  if (M <= 0 || N <= 0 || K <= 0)
    return fail(SYS1HIP_EINVAL, "sys1hip_query_kernel: bad shape");
  const Plan p = resolve(c, M, N, K, skinny_wide(M, K, K, N, K), epi_id_from_flags(epilogue));
  const int id = p.kernel;
  if (id < 0) return fail(SYS1HIP_EINVAL, "sys1hip_query_kernel: the forced kernel does not fit this call");
  if (name && cap > 0) {
    std::string s = kKernels[id].name;
    s += "_g" + std::to_string(p.grid);
    const int64_t tiles = cdiv(M, kKernels[id].bm) * cdiv(N, kKernels[id].bn);
    if (kKernels[id].streamk && p.dp > 0 && p.dp < tiles) s += "_dp" + std::to_string(p.dp);
    snprintf(name, (size_t)cap, "%s", s.c_str());
  }
  return id;
}

int sys1hip_linear_bf16(void* ctx, const uint16_t* x, int64_t ldx, const uint16_t* w, int64_t ldw,
                        const uint16_t* bias, const uint16_t* residual, int64_t ldr, uint16_t* y,
                        int64_t ldy, int64_t M, int64_t N, int64_t K, int32_t epilogue) {
  if (!ctx) return fail(SYS1HIP_EINVAL, "sys1hip_linear_bf16: null context");
  Context* c = static_cast<Context*>(ctx);
  int rc = check_linear("sys1hip_linear_bf16", x, ldx, w, ldw, bias, residual, ldr, y, ldy, M, N, K, epilogue);
  if (rc || M == 0) return rc;
  rc = use_device(c);
  if (rc) return rc;
  const int epi = epi_id_from_flags(epilogue);
  return launch_linear("sys1hip_linear_bf16", c, resolve(c, M, N, K, skinny_wide(M, K, ldx, N, plan_ldw(ldw, K, epilogue)), epi), c->stream,
                       c->ws, c->counters, x, ldx, w, ldw, bias, residual, ldr, y, ldy, M, N, K, epi,
                       epilogue & SYS1HIP_EPI_BLOCKED_W);
}

}  // extern "C"

namespace {

// ---- The context-free entry point that allocates nothing
// (sys1hip_linear_bf16_noalloc).  Its stream-K workspace is `scratch`, a
// static device array: each GPU the library runs on holds one copy, at its
// own address, from the module's load to the end of the process.  Host code
// must not use the array's name as a device address (it is a host-side
// stand-in); each device's address comes from hipGetSymbolAddress, taken
// once per device with that device current, and only that address is
// passed to kernels.
constexpr int kMaxStaticDevices = 64;
constexpr size_t kScratchBytes = kWorkspaceBytes + (size_t)kCounterSlots * sizeof(unsigned);
__device__ __align__(256) char scratch[kScratchBytes];

__global__ void clear_words_kernel(unsigned* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Per device: the scratch address and the plan inputs (CU count and the
// kernels' occupancy), all in static storage.
struct StaticDevice {
  std::mutex mu;      // guards the set-up; `ready` is set only when it succeeded,
  std::atomic<bool> ready{false};  // so a failed set-up is retried by the next call
  int rc = SYS1HIP_OK;
  char* ptr = nullptr;
  Context plan_ctx;  // only cus and occ_fixed are used (price_plans)
  int occ[kNumKernels * kEpiCount] = {};
};
StaticDevice g_static[kMaxStaticDevices];

int setup_static(StaticDevice& d, int dev, hipStream_t stream) {
  HIP_TRY(hipGetSymbolAddress(reinterpret_cast<void**>(&d.ptr), HIP_SYMBOL(scratch)));
  if (!d.ptr) return fail(SYS1HIP_EDEVICE, "sys1hip_linear_bf16_noalloc: no scratch address on device %d", dev);
  int cus = 0;
  HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  d.plan_ctx.cus = cus > 0 ? cus : 256;
  for (int id = 0; id < kNumKernels; ++id)
    for (int epi = 0; epi < kEpiCount; ++epi) {
      int n = 0;
      const KernelFn fn = kKernels[id].fn[epi];
      if (fn && hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(fn),
                                                             kKernels[id].threads, 0) == hipSuccess)
        d.occ[id * kEpiCount + epi] = n;
    }
  (void)hipGetLastError();
  d.plan_ctx.occ_fixed = d.occ;
  // The arrival counters must start at zero (device globals are zeroed at
  // load; each stream-K call's last arriving waves re-arm theirs).  When
  // the first call is not being captured, they are also cleared explicitly,
  // with a kernel on the caller's stream (ordered before the call).
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(stream, &st));
  if (st == hipStreamCaptureStatusNone) {
    hipLaunchKernelGGL(clear_words_kernel, dim3((unsigned)cdiv(kCounterSlots, 256)), dim3(256), 0, stream,
                       reinterpret_cast<unsigned*>(d.ptr + kWorkspaceBytes), (int64_t)kCounterSlots);
    HIP_TRY(hipGetLastError());
  }
  return SYS1HIP_OK;
}

}  // namespace

extern "C" {

int sys1hip_linear_bf16_noalloc(void* stream, const uint16_t* x, int64_t ldx, const uint16_t* w, int64_t ldw,
                                const uint16_t* bias, const uint16_t* residual, int64_t ldr, uint16_t* y,
                                int64_t ldy, int64_t M, int64_t N, int64_t K, int32_t epilogue) {
  static const char* who = "sys1hip_linear_bf16_noalloc";
  int rc = check_linear(who, x, ldx, w, ldw, bias, residual, ldr, y, ldy, M, N, K, epilogue);
  if (rc || M == 0) return rc;
  int dev = -1;
  HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxStaticDevices)
    return fail(SYS1HIP_EDEVICE, "%s: device %d beyond the %d this entry point serves", who, dev, kMaxStaticDevices);
  StaticDevice& d = g_static[dev];
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (!d.ready.load(std::memory_order_acquire)) {
    std::lock_guard<std::mutex> lock(d.mu);
    if (!d.ready.load(std::memory_order_relaxed)) {
      d.rc = setup_static(d, dev, s);
      if (d.rc) return fail(d.rc, "%s: set-up on device %d failed (retried on the next call): %s", who, dev,
                            g_last_error.c_str());
      d.ready.store(true, std::memory_order_release);
    }
  }
  // The plan is priced on every call (no cache: a cache insert would
  // allocate host memory).
  const int epi = epi_id_from_flags(epilogue);
  const Plan p = price_plans(&d.plan_ctx, M, N, K, skinny_wide(M, K, ldx, N, plan_ldw(ldw, K, epilogue)), epi,
                             false, false);
  return launch_linear(who, &d.plan_ctx, p, s, reinterpret_cast<float*>(d.ptr),
                       reinterpret_cast<unsigned*>(d.ptr + kWorkspaceBytes), x, ldx, w, ldw, bias, residual, ldr,
                       y, ldy, M, N, K, epi, epilogue & SYS1HIP_EPI_BLOCKED_W);
}

int sys1hip_linear_rope_qkv_bf16(void* ctx, const uint16_t* x, int64_t ldx, const uint16_t* w,
                                 int64_t ldw, const float* rope_cos, const float* rope_sin,
                                 int64_t rope_rows, const int32_t* positions, uint16_t* qkv,
                                 int64_t M, int64_t heads, int64_t head_dim, int64_t K) {
  if (!ctx) return fail(SYS1HIP_EINVAL, "sys1hip_linear_rope_qkv_bf16: null context");
  Context* c = static_cast<Context*>(ctx);
  if (M < 0 || heads <= 0 || K <= 0 || rope_rows <= 0 || rope_rows > (1ll << 30))
    return fail(SYS1HIP_EINVAL,
                "sys1hip_linear_rope_qkv_bf16: bad shape M=%lld heads=%lld K=%lld rope_rows=%lld",
                (long long)M, (long long)heads, (long long)K, (long long)rope_rows);
  if (head_dim != 64)
    return fail(SYS1HIP_EINVAL, "sys1hip_linear_rope_qkv_bf16: head_dim %lld unsupported (64 only)",
                (long long)head_dim);
  if (M == 0) return SYS1HIP_OK;
  if (!x || !w || !qkv || !rope_cos || !rope_sin || !positions)
    return fail(SYS1HIP_EINVAL, "sys1hip_linear_rope_qkv_bf16: null pointer");
  if (ldx < K || ldw < K)
    return fail(SYS1HIP_EINVAL, "sys1hip_linear_rope_qkv_bf16: leading dimension below K");
  if (K % 8 || ldx % 8 || ldw % 8)
    return fail(SYS1HIP_EALIGN, "sys1hip_linear_rope_qkv_bf16: K, ldx and ldw must be multiples of 8");
  if (!aligned16(x) || !aligned16(w) || !aligned16(rope_cos) || !aligned16(rope_sin))
    return fail(SYS1HIP_EALIGN, "sys1hip_linear_rope_qkv_bf16: x, w, cos and sin must be 16-byte aligned");
  const int64_t H = heads * head_dim, N = 3 * H;
  if (M > (1ll << 30) || N > (1ll << 30) || K > (1ll << 30) || M * H > (1ll << 40))
    return fail(SYS1HIP_ERANGE, "sys1hip_linear_rope_qkv_bf16: dimension above 2^30");
  int rc = use_device(c);
  if (rc) return rc;
  if (c->forced_kernel >= 0 && kKernels[c->forced_kernel].tn != 64)
    return fail(SYS1HIP_EINVAL, "sys1hip_linear_rope_qkv_bf16: forced kernel %s is not head-aligned",
                kKernels[c->forced_kernel].name);
  const Plan p = resolve(c, M, N, K, skinny_wide(M, K, ldx, N, ldw), kEpiRopeQkv, true);
  if (p.kernel < 0) return fail(SYS1HIP_EINVAL, "sys1hip_linear_rope_qkv_bf16: the forced kernel does not fit this call");
  const KernelEntry& e = kKernels[p.kernel];
  if (e.streamk && (cdiv(M, e.bm) * cdiv(N, e.bn) - p.dp) * (e.threads / 64) > kCounterSlots)
    return fail(SYS1HIP_ERANGE, "sys1hip_linear_rope_qkv_bf16: more split tiles than stream-K counters");
  GemmArgs a = {};
  a.x = reinterpret_cast<const __bf16*>(x);
  a.w = reinterpret_cast<const __bf16*>(w);
  a.y = reinterpret_cast<__bf16*>(qkv);
  a.ws = c->ws;
  a.counters = c->counters;
  a.ldx = ldx, a.ldw = ldw, a.ldr = 0, a.ldy = H;
  a.M = (int)M, a.N = (int)N, a.K = (int)K, a.Nout = (int)N;
  a.dp_tiles = (int)std::min<int64_t>(p.dp, 1 << 30);
  a.group_m = raster_group(K);
  a.rope_cos = rope_cos;
  a.rope_sin = rope_sin;
  a.pos = positions;
  a.rope_rows = (int)rope_rows;
  a.plane = M * H;
  hipLaunchKernelGGL(e.fn[kEpiRopeQkv], dim3((unsigned)p.grid), dim3(e.threads), 0, c->stream, a);
  HIP_TRY(hipGetLastError());
  return SYS1HIP_OK;
}

}  // extern "C"

namespace {
// Per-row (mean, 1/std) of x into the context's statistics buffer.
int launch_row_stats(Context* c, const __bf16* x, int64_t ldx, int64_t M, int64_t K, int32_t norm,
                     float eps) {
  using StatsFn = void (*)(const __bf16*, int64_t, int, int, float, float*);
  static constexpr StatsFn kStats[2][4] = {
      {row_stats_kernel<kNormLayer, 2>, row_stats_kernel<kNormLayer, 4>, row_stats_kernel<kNormLayer, 8>,
       row_stats_kernel<kNormLayer, 16>},
      {row_stats_kernel<kNormRms, 2>, row_stats_kernel<kNormRms, 4>, row_stats_kernel<kNormRms, 8>,
       row_stats_kernel<kNormRms, 16>}};
  const int ch = K <= 1024 ? 0 : K <= 2048 ? 1 : K <= 4096 ? 2 : 3;  // register row of 2..16 x 512
  hipLaunchKernelGGL(kStats[norm == SYS1HIP_NORM_LAYER ? 0 : 1][ch], dim3((unsigned)cdiv(M, 4)), dim3(256), 0,
                     c->stream, x, ldx, (int)M, (int)K, eps, c->stats);
  HIP_TRY(hipGetLastError());
  return SYS1HIP_OK;
}
}  // namespace

extern "C" {

int sys1hip_fold_norm_weight(void* ctx, const uint16_t* w, const float* gamma, int32_t norm,
                             uint16_t* w_folded, float* colsum, int64_t N, int64_t K) {
  if (!ctx) return fail(SYS1HIP_EINVAL, "sys1hip_fold_norm_weight: null context");
  Context* c = static_cast<Context*>(ctx);
  if (norm != SYS1HIP_NORM_LAYER && norm != SYS1HIP_NORM_RMS)
    return fail(SYS1HIP_EINVAL, "sys1hip_fold_norm_weight: unknown norm %d", norm);
  if (N <= 0 || K <= 0)
    return fail(SYS1HIP_EINVAL, "sys1hip_fold_norm_weight: bad shape N=%lld K=%lld", (long long)N,
                (long long)K);
  if (!w || !gamma || !w_folded || (norm == SYS1HIP_NORM_LAYER && !colsum))
    return fail(SYS1HIP_EINVAL, "sys1hip_fold_norm_weight: null pointer");
  if (K % 8) return fail(SYS1HIP_EALIGN, "sys1hip_fold_norm_weight: K must be a multiple of 8");
  if (!aligned16(w) || !aligned16(w_folded) || !aligned16(gamma))
    return fail(SYS1HIP_EALIGN, "sys1hip_fold_norm_weight: w, w_folded and gamma must be 16-byte aligned");
  if (N > (1ll << 30) || K > (1ll << 30))
    return fail(SYS1HIP_ERANGE, "sys1hip_fold_norm_weight: dimension above 2^30");
  int rc = use_device(c);
  if (rc) return rc;
  const unsigned blocks = (unsigned)cdiv(N, 4);
  const auto* wb = reinterpret_cast<const __bf16*>(w);
  auto* ob = reinterpret_cast<__bf16*>(w_folded);
  if (norm == SYS1HIP_NORM_LAYER)
    hipLaunchKernelGGL(fold_norm_kernel<kNormLayer>, dim3(blocks), dim3(256), 0, c->stream, wb, gamma, ob,
                       colsum, (int)N, (int)K);
  else
    hipLaunchKernelGGL(fold_norm_kernel<kNormRms>, dim3(blocks), dim3(256), 0, c->stream, wb, gamma, ob,
                       colsum, (int)N, (int)K);
  HIP_TRY(hipGetLastError());
  return SYS1HIP_OK;
}

int sys1hip_norm_linear_bf16(void* ctx, const uint16_t* x, int64_t ldx, const uint16_t* w_folded,
                             int64_t ldw, const float* colsum, int32_t norm, float eps, uint16_t* y,
                             int64_t ldy, int64_t M, int64_t N, int64_t K, int32_t epilogue) {
  if (!ctx) return fail(SYS1HIP_EINVAL, "sys1hip_norm_linear_bf16: null context");
  Context* c = static_cast<Context*>(ctx);
  int epi = -1;
  const bool blocked = epilogue & SYS1HIP_EPI_BLOCKED_W;
  const int32_t base = epilogue & ~SYS1HIP_EPI_BLOCKED_W;
  if (norm == SYS1HIP_NORM_LAYER && base == SYS1HIP_EPI_NONE) epi = kEpiNormLn;
  if (norm == SYS1HIP_NORM_LAYER && base == SYS1HIP_EPI_GEGLU) epi = kEpiNormLnGeglu;
  if (norm == SYS1HIP_NORM_RMS && base == SYS1HIP_EPI_NONE) epi = kEpiNormRms;
  if (norm == SYS1HIP_NORM_RMS && base == SYS1HIP_EPI_SWIGLU) epi = kEpiNormRmsSwiglu;
  if (epi < 0)
    return fail(SYS1HIP_EINVAL, "sys1hip_norm_linear_bf16: unsupported norm %d with epilogue flags %d",
                norm, epilogue);
  if (M < 0 || N <= 0 || K <= 0 || !(eps >= 0.0f))
    return fail(SYS1HIP_EINVAL, "sys1hip_norm_linear_bf16: bad shape M=%lld N=%lld K=%lld or eps",
                (long long)M, (long long)N, (long long)K);
  const bool gated = epi_gated(epi);
  if (gated && (N % (2 * SYS1HIP_GATE_GROUP)) != 0)
    return fail(SYS1HIP_EINVAL, "sys1hip_norm_linear_bf16: gated epilogue needs N %% 32 == 0 (N=%lld)",
                (long long)N);
  const int64_t nout = gated ? N / 2 : N;
  if (M == 0) return SYS1HIP_OK;
  if (!x || !w_folded || !y || (norm == SYS1HIP_NORM_LAYER && !colsum))
    return fail(SYS1HIP_EINVAL, "sys1hip_norm_linear_bf16: null pointer");
  if (ldx < K || (!blocked && ldw < K) || ldy < nout)
    return fail(SYS1HIP_EINVAL, "sys1hip_norm_linear_bf16: leading dimension too small");
  if (K % 8 || ldx % 8 || (!blocked && ldw % 8))
    return fail(SYS1HIP_EALIGN, "sys1hip_norm_linear_bf16: K, ldx and ldw must be multiples of 8");
  if (blocked && blocked_bytes(N, K) > 0x7ffffff0ll)
    return fail(SYS1HIP_ERANGE, "sys1hip_norm_linear_bf16: blocked weight above 2 GiB");
  if (!aligned16(x) || !aligned16(w_folded) || (colsum && !aligned16(colsum)))
    return fail(SYS1HIP_EALIGN, "sys1hip_norm_linear_bf16: x, w_folded and colsum must be 16-byte aligned");
  if (M > kNormRows)
    return fail(SYS1HIP_ERANGE, "sys1hip_norm_linear_bf16: M=%lld above the %lld rows of one call",
                (long long)M, (long long)kNormRows);
  if (N > (1ll << 30) || K > (1ll << 30))
    return fail(SYS1HIP_ERANGE, "sys1hip_norm_linear_bf16: dimension above 2^30");
  int rc = use_device(c);
  if (rc) return rc;
  const Plan p = resolve(c, M, N, K, skinny_wide(M, K, ldx, N, plan_ldw(ldw, K, epilogue)), epi);
  if (p.kernel < 0) return fail(SYS1HIP_EINVAL, "sys1hip_norm_linear_bf16: the forced kernel does not fit this call");
  const KernelEntry& e = kKernels[p.kernel];
  if (e.streamk && (cdiv(M, e.bm) * cdiv(N, e.bn) - p.dp) * (e.threads / 64) > kCounterSlots)
    return fail(SYS1HIP_ERANGE, "sys1hip_norm_linear_bf16: more split tiles than stream-K counters");
  const auto* xb = reinterpret_cast<const __bf16*>(x);
  rc = launch_row_stats(c, xb, ldx, M, K, norm, eps);
  if (rc) return rc;
  GemmArgs a = {};
  a.x = xb;
  a.w = reinterpret_cast<const __bf16*>(w_folded);
  a.y = reinterpret_cast<__bf16*>(y);
  a.ws = c->ws;
  a.counters = c->counters;
  a.ldx = ldx, a.ldw = ldw, a.ldr = 0, a.ldy = ldy;
  a.M = (int)M, a.N = (int)N, a.K = (int)K, a.Nout = (int)nout;
  a.dp_tiles = (int)std::min<int64_t>(p.dp, 1 << 30);
  a.group_m = raster_group(K);
  a.stats = c->stats;
  a.colsum = colsum;
  a.w_kt = blocked ? (int)cdiv(K, kBlkK) : 0;
  hipLaunchKernelGGL(e.fn[epi], dim3((unsigned)p.grid), dim3(e.threads), 0, c->stream, a);
  HIP_TRY(hipGetLastError());
  return SYS1HIP_OK;
}

int sys1hip_linear_conv_silu_bf16(void* ctx, const uint16_t* x, int64_t ldx, const uint16_t* w, int64_t ldw,
                                  int32_t norm, float eps, const uint16_t* conv_w, int64_t conv_ch,
                                  const int32_t* positions, uint16_t* y, int64_t ldy, int64_t M, int64_t N,
                                  int64_t K) {
  if (!ctx) return fail(SYS1HIP_EINVAL, "sys1hip_linear_conv_silu_bf16: null context");
  Context* c = static_cast<Context*>(ctx);
  if (norm != 0 && norm != SYS1HIP_NORM_RMS)
    return fail(SYS1HIP_EINVAL, "sys1hip_linear_conv_silu_bf16: norm %d (0 or SYS1HIP_NORM_RMS)", norm);
  if (M < 0 || N <= 0 || K <= 0 || conv_ch <= 0 || conv_ch > N || conv_ch % 8 || !(eps >= 0.0f))
    return fail(SYS1HIP_EINVAL,
                "sys1hip_linear_conv_silu_bf16: bad shape M=%lld N=%lld K=%lld conv_ch=%lld (multiple of 8, "
                "at most N) or eps",
                (long long)M, (long long)N, (long long)K, (long long)conv_ch);
  if (M == 0) return SYS1HIP_OK;
  if (!x || !w || !y || !conv_w || !positions)
    return fail(SYS1HIP_EINVAL, "sys1hip_linear_conv_silu_bf16: null pointer");
  if (ldx < K || ldw < K || ldy < N)
    return fail(SYS1HIP_EINVAL, "sys1hip_linear_conv_silu_bf16: leading dimension too small");
  if (K % 8 || ldx % 8 || ldw % 8)
    return fail(SYS1HIP_EALIGN, "sys1hip_linear_conv_silu_bf16: K, ldx and ldw must be multiples of 8");
  if (!aligned16(x) || !aligned16(w) || !aligned16(conv_w))
    return fail(SYS1HIP_EALIGN, "sys1hip_linear_conv_silu_bf16: x, w and conv_w must be 16-byte aligned");
  if (M > kNormRows)
    return fail(SYS1HIP_ERANGE, "sys1hip_linear_conv_silu_bf16: M=%lld above the %lld rows of one call",
                (long long)M, (long long)kNormRows);
  if (N > (1ll << 30) || K > (1ll << 30))
    return fail(SYS1HIP_ERANGE, "sys1hip_linear_conv_silu_bf16: dimension above 2^30");
  if (ldy % 8 || !aligned16(y))
    return fail(SYS1HIP_EALIGN, "sys1hip_linear_conv_silu_bf16: y must be 16-byte aligned, ldy a multiple of 8");
  int rc = use_device(c);
  if (rc) return rc;
  const auto* xb = reinterpret_cast<const __bf16*>(x);
  GemmArgs a = {};
  a.x = xb;
  a.w = reinterpret_cast<const __bf16*>(w);
  a.y = reinterpret_cast<__bf16*>(y);
  a.ws = c->ws;
  a.counters = c->counters;
  a.ldx = ldx, a.ldw = ldw, a.ldr = 0, a.ldy = ldy;
  a.M = (int)M, a.N = (int)N, a.K = (int)K, a.Nout = (int)N;
  a.stats = c->stats;
  a.pos = positions;
  a.conv_w = reinterpret_cast<const __bf16*>(conv_w);
  a.conv_ch = (int)conv_ch;
  // Two forms.  Fused: the conv in the GEMM epilogue, on the shapes whose
  // waves span every row of a tile (chosen when such a kernel is forced).
  // Two-pass (the default): the projection on the best kernel for the
  // shape, then the conv in place over segments of rows.  On MI355X the
  // two-pass form measured faster at M = 128 and 8192: the wave-spanning
  // shapes lose more in the GEMM than the fused form saves in traffic.
  const bool fused = c->forced_kernel >= 0 && kKernels[c->forced_kernel].wm == 1;
  const int epi = fused ? (norm ? kEpiNormRmsConvSilu : kEpiConvSilu) : (norm ? kEpiNormRms : kEpiNone);
  const Plan p = resolve(c, M, N, K, skinny_wide(M, K, ldx, N, ldw), epi, false, fused);
  if (p.kernel < 0) return fail(SYS1HIP_EINVAL, "sys1hip_linear_conv_silu_bf16: the forced kernel does not fit this call");
  const KernelEntry& e = kKernels[p.kernel];
  if (!e.fn[epi])
    return fail(SYS1HIP_EINVAL, "sys1hip_linear_conv_silu_bf16: kernel %s has no conv epilogue", e.name);
  const int64_t rows = fused ? halo_rows(e, M, kConvHalo) : M;
  if (e.streamk && (cdiv(rows, e.bm) * cdiv(N, e.bn) - p.dp) * (e.threads / 64) > kCounterSlots)
    return fail(SYS1HIP_ERANGE, "sys1hip_linear_conv_silu_bf16: more split tiles than stream-K counters");
  if (norm) {
    rc = launch_row_stats(c, xb, ldx, M, K, norm, eps);
    if (rc) return rc;
  }
  a.dp_tiles = (int)std::min<int64_t>(p.dp, 1 << 30);
  a.group_m = raster_group(K);
  hipLaunchKernelGGL(e.fn[epi], dim3((unsigned)p.grid), dim3(e.threads), 0, c->stream, a);
  HIP_TRY(hipGetLastError());
  if (fused) return SYS1HIP_OK;
  // Segments of S rows: one chunk (kConvChunk rows) each, for the most
  // threads in flight, except from kConvLongRows rows on, where four chunks
  // per segment still leave 2^17 threads or more (one per segment and 8
  // channels) and save three quarters of the halo rows (3 per segment);
  // longer only when the halos (kConvHalo rows of conv_ch bf16 per
  // segment) would not fit the workspace.  Measured, same box: Qwen3.5-small
  // in_proj + conv at 8192 tokens (8192 conv channels) 389.4 us at 16-row
  // segments, 382.4 at 32, 379.0 at 64; the 27B in_proj + conv at 4096
  // tokens 565 us at 16 rows and 568 at 32.
  constexpr int64_t kConvLongRows = 8192;
  const int64_t vecs = conv_ch / kConvVec;
  const int64_t halo_row_bytes = (int64_t)kConvHalo * conv_ch * 2;
  const int64_t max_segs = std::max<int64_t>(1, (int64_t)kWorkspaceBytes / halo_row_bytes);
  const int64_t chunks = M >= kConvLongRows && (M / (4 * kConvChunk)) * vecs >= (1 << 17) ? 4 : 1;
  const int64_t S = std::max<int64_t>(chunks * kConvChunk, cdiv(cdiv(M, max_segs), kConvChunk) * kConvChunk);
  const int64_t segs = cdiv(M, S);
  auto* halo = reinterpret_cast<__bf16*>(c->ws);
  if (segs > 1) {
    const int64_t n = (segs - 1) * kConvHalo * vecs;
    hipLaunchKernelGGL(conv_halo_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, c->stream, a.y, ldy, (int)M,
                       (int)conv_ch, (int)S, halo);
    HIP_TRY(hipGetLastError());
  }
  hipLaunchKernelGGL(conv_silu_inplace_kernel, dim3((unsigned)cdiv(segs * vecs, 256)), dim3(256), 0, c->stream,
                     a.y, ldy, (int)M, (int)conv_ch, (int)S, halo, a.conv_w, positions);
  HIP_TRY(hipGetLastError());
  return SYS1HIP_OK;
}

int64_t sys1hip_blocked_weight_bytes(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0 || N > (1ll << 30) || K > (1ll << 30)) return -1;
  return blocked_bytes(N, K);
}

int sys1hip_pack_blocked_weight(void* ctx, const uint16_t* w, int64_t ldw, uint16_t* packed, int64_t N,
                                int64_t K) {
  if (!ctx) return fail(SYS1HIP_EINVAL, "sys1hip_pack_blocked_weight: null context");
  if (!w || !packed) return fail(SYS1HIP_EINVAL, "sys1hip_pack_blocked_weight: null pointer");
  if (w == packed) return fail(SYS1HIP_EINVAL, "sys1hip_pack_blocked_weight: packed aliases w");
  if (N <= 0 || K <= 0 || ldw < K || N > (1ll << 30) || K > (1ll << 30))
    return fail(SYS1HIP_EINVAL, "sys1hip_pack_blocked_weight: bad shape N=%lld K=%lld ldw=%lld", (long long)N,
                (long long)K, (long long)ldw);
  if (K % 8 || ldw % 8) return fail(SYS1HIP_EALIGN, "sys1hip_pack_blocked_weight: K and ldw must be multiples of 8");
  if (!aligned16(w) || !aligned16(packed))
    return fail(SYS1HIP_EALIGN, "sys1hip_pack_blocked_weight: pointers must be 16-byte aligned");
  if (blocked_bytes(N, K) > 0x7ffffff0ll)
    return fail(SYS1HIP_ERANGE, "sys1hip_pack_blocked_weight: blocked weight above 2 GiB");
  Context* c = static_cast<Context*>(ctx);
  int rc = use_device(c);
  if (rc) return rc;
  const int64_t total = blocked_bytes(N, K) / 16;
  hipLaunchKernelGGL(pack_blocked_kernel, dim3((unsigned)cdiv(total, 256)), dim3(256), 0, c->stream,
                     reinterpret_cast<const __bf16*>(w), ldw, reinterpret_cast<i32x4*>(packed), N, K, cdiv(K, kBlkK),
                     total);
  HIP_TRY(hipGetLastError());
  return SYS1HIP_OK;
}

int sys1hip_pack_gated_weight(void* ctx, const uint16_t* w, uint16_t* packed, int64_t N, int64_t K) {
  if (!ctx) return fail(SYS1HIP_EINVAL, "sys1hip_pack_gated_weight: null context");
  if (!w || !packed) return fail(SYS1HIP_EINVAL, "sys1hip_pack_gated_weight: null pointer");
  if (w == packed) return fail(SYS1HIP_EINVAL, "sys1hip_pack_gated_weight: packed aliases w");
  if (N <= 0 || K <= 0 || N % (2 * SYS1HIP_GATE_GROUP))
    return fail(SYS1HIP_EINVAL, "sys1hip_pack_gated_weight: need N %% 32 == 0 and K > 0 (N=%lld K=%lld)",
                (long long)N, (long long)K);
  if (K % 8) return fail(SYS1HIP_EALIGN, "sys1hip_pack_gated_weight: K must be a multiple of 8");
  if (!aligned16(w) || !aligned16(packed))
    return fail(SYS1HIP_EALIGN, "sys1hip_pack_gated_weight: pointers must be 16-byte aligned");
  Context* c = static_cast<Context*>(ctx);
  int rc = use_device(c);
  if (rc) return rc;
  const int64_t kv = K / 8;
  const int64_t total = N * kv;
  const int64_t blocks = cdiv(total, 256);
  if (blocks > 0x7fffffff) return fail(SYS1HIP_ERANGE, "sys1hip_pack_gated_weight: too large");
  hipLaunchKernelGGL(pack_gated_kernel, dim3((unsigned)blocks), dim3(256), 0, c->stream,
                     reinterpret_cast<const i32x4*>(w), reinterpret_cast<i32x4*>(packed), N, kv);
  HIP_TRY(hipGetLastError());
  return SYS1HIP_OK;
}

// ---- projection chains (chain.hip)

// Whether a chain runs as a weight stream: up to kStreamChainKernel.bm
// tokens, every K within its reach.
bool stream_chain_fits(const sys1hip_chain_proj* proj, int count, int64_t M) {
  if (M > kStreamChainKernel.bm) return false;
  for (int p = 0; p < count; ++p)
    if (proj[p].K > kStreamChainKernel.stages) return false;
  return true;
}

int sys1hip_linear_chain_bf16(void* ctx, const sys1hip_chain_proj* proj, int32_t count, int64_t M) {
  static const char* who = "sys1hip_linear_chain_bf16";
  if (!ctx) return fail(SYS1HIP_EINVAL, "%s: null context", who);
  if (!proj || count < 1 || count > kChainMax)
    return fail(SYS1HIP_EINVAL, "%s: %d projections (1..%d)", who, (int)count, kChainMax);
  if (M < 0) return fail(SYS1HIP_EINVAL, "%s: M=%lld", who, (long long)M);
  Context* c = static_cast<Context*>(ctx);
  // Up to 64 tokens the chain is a weight stream (stream_chain_kernel: 32-
  // column items over the whole K, every CU); above, 128 x 192 tiles on row
  // panels (chain_kernel).
  const bool stream = stream_chain_fits(proj, count, M);
  const ChainKernel& ck = stream ? kStreamChainKernel : kChainKernel;
  const int64_t panels = stream ? 1 : cdiv(M, ck.bm);
  if (panels > kChainMaxPanels)
    return fail(SYS1HIP_ERANGE, "%s: M=%lld above %lld tokens", who, (long long)M, (long long)kChainMaxPanels * ck.bm);
  ChainArgs a{};
  for (int p = 0; p < count; ++p) {
    const sys1hip_chain_proj& q = proj[p];
    int rc = check_linear(who, q.x, q.ldx, q.w, q.ldw, nullptr, q.residual, q.ldr, q.y, q.ldy, M, q.N, q.K,
                          q.epilogue);
    if (rc) return rc;
    const int epi = epi_id_from_flags(q.epilogue);
    if (epi != kEpiNone && epi != kEpiResidual && epi != kEpiGeglu && epi != kEpiSwiglu)
      return fail(SYS1HIP_EINVAL, "%s: projection %d: epilogue flags %d (none, residual, GeGLU or SwiGLU)", who, p,
                  q.epilogue);
    if (!stream && (q.K % kBlkK || q.K / kBlkK < ck.stages))
      return fail(SYS1HIP_EINVAL, "%s: projection %d: K=%lld must be a multiple of %d and at least %d", who, p,
                  (long long)q.K, kBlkK, kBlkK * ck.stages);
    const int64_t nout = epi_gated(epi) ? q.N / 2 : q.N;
    if (epi == kEpiResidual &&
        (nout % 8 || q.ldr % 8 || !aligned16(q.residual) || 2 * (M * q.ldr + nout) >= 0x7ffffff0ll))
      return fail(SYS1HIP_EALIGN, "%s: projection %d: the residual needs Nout and ldr multiples of 8, 16-byte "
                  "alignment and fewer than 2 GiB of rows", who, p);
    if (stream && (nout % 8 || q.ldy % 8 || !aligned16(q.y) || 2 * (M * q.ldy + nout) >= 0x7ffffff0ll ||
                   2 * (M * q.ldx + q.K) >= 0x7ffffff0ll ||
                   (q.epilogue & SYS1HIP_EPI_BLOCKED_W ? blocked_bytes(q.N, q.K) : 2 * q.N * q.ldw) >= 0x7ffffff0ll))
      return fail(SYS1HIP_EALIGN, "%s: projection %d: a chain of up to %d tokens needs Nout and ldy multiples of 8, "
                  "16-byte aligned y and operands below 2 GiB", who, p, kStreamChainKernel.bm);
    if (!stream && (2 * (int64_t)ck.bm * q.ldx + 2 * q.K >= 0x7ffffff0ll ||
                    (!(q.epilogue & SYS1HIP_EPI_BLOCKED_W) && 2 * (int64_t)ck.bn * q.ldw >= 0x7ffffff0ll)))
      return fail(SYS1HIP_ERANGE, "%s: projection %d: leading dimension too large", who, p);
    ChainProj& P = a.proj[p];
    P.x = reinterpret_cast<const __bf16*>(q.x);
    P.w = reinterpret_cast<const __bf16*>(q.w);
    P.resid = reinterpret_cast<const __bf16*>(q.residual);
    P.y = reinterpret_cast<__bf16*>(q.y);
    P.ldx = q.ldx, P.ldw = q.ldw, P.ldr = q.ldr, P.ldy = q.ldy;
    P.N = (int)q.N, P.K = (int)q.K, P.Nout = (int)nout, P.epi = epi;
    P.w_kt = (q.epilogue & SYS1HIP_EPI_BLOCKED_W) ? (int)cdiv(q.K, kBlkK) : 0;
    P.tiles_n = (int)cdiv(q.N, ck.bn);
    P.kt_count = (int)(q.K / kBlkK);
  }
  if (M == 0) return SYS1HIP_OK;
  int rc = use_device(c);
  if (rc) return rc;
  const int occ = stream ? c->stream_chain_occ : c->chain_occ;
  if (occ < 1) return fail(SYS1HIP_EDEVICE, "%s: the chain kernel cannot be resident on this device", who);
  a.bank = c->chain;
  a.err = c->chain + kChainErrWord;
  a.nproj = count;
  a.M = (int)M;
  a.row_panels = (int)panels;
  a.nxcd = kChainXcdMax;
  a.wait_us = c->chain_wait_us;
  a.dep_extra = c->chain_extra;
  const int grid = c->cus * occ;
  a.trace = c->chain_trace && c->chain_trace_bytes >= (int64_t)grid * kChainTraceTiles * 32
                ? c->chain_trace : nullptr;
  hipLaunchKernelGGL(reinterpret_cast<void (*)(ChainArgs)>(const_cast<void*>(ck.fn)), dim3((unsigned)grid),
                     dim3(ck.threads), 0, c->stream, a);
  HIP_TRY(hipGetLastError());
  return SYS1HIP_OK;
}

int sys1hip_chain_queue(int32_t xcc, int64_t M, int32_t count, const int64_t* N, int32_t* tiles, int64_t cap) {
  if (count < 1 || count > kChainMax || !N || xcc < 0 || xcc >= kChainXcdMax || M < 0)
    return fail(SYS1HIP_EINVAL, "sys1hip_chain_queue: bad arguments");
  const int64_t panels = cdiv(M, kChainKernel.bm);
  if (panels > kChainMaxPanels) return fail(SYS1HIP_ERANGE, "sys1hip_chain_queue: M=%lld", (long long)M);
  int tn[kChainMax] = {};
  for (int p = 0; p < count; ++p) {
    if (N[p] <= 0) return fail(SYS1HIP_EINVAL, "sys1hip_chain_queue: N[%d]=%lld", p, (long long)N[p]);
    tn[p] = (int)cdiv(N[p], kChainKernel.bn);
  }
  const XcdQueue q(xcc, kChainXcdMax, (int)panels, count, tn);
  for (int i = 0; i < q.total && tiles && 3 * (int64_t)i + 2 < cap; ++i) {
    const ChainTile t = q.decode(i);
    tiles[3 * i] = t.p, tiles[3 * i + 1] = t.rp, tiles[3 * i + 2] = t.tn;
  }
  return q.total;
}

int sys1hip_chain_status(void* ctx, int32_t* flags) {
  if (!ctx || !flags) return fail(SYS1HIP_EINVAL, "sys1hip_chain_status: null argument");
  Context* c = static_cast<Context*>(ctx);
  int rc = use_device(c);
  if (rc) return rc;
  unsigned v = 0;
  HIP_TRY(hipStreamSynchronize(c->stream));
  HIP_TRY(hipMemcpy(&v, c->chain + kChainErrWord, sizeof(v), hipMemcpyDeviceToHost));
  if (v) HIP_TRY(hipMemset(c->chain + kChainErrWord, 0, sizeof(v)));
  *flags = (int32_t)v;
  return SYS1HIP_OK;
}

int sys1hip_set_chain_trace(void* ctx, void* buffer, int64_t bytes) {
  if (!ctx) return fail(SYS1HIP_EINVAL, "sys1hip_set_chain_trace: null context");
  Context* c = static_cast<Context*>(ctx);
  c->chain_trace = static_cast<unsigned long long*>(buffer);
  c->chain_trace_bytes = buffer ? bytes : 0;
  return SYS1HIP_OK;
}

int sys1hip_set_chain_wait(void* ctx, int32_t wait_us, int32_t extra) {
  if (!ctx) return fail(SYS1HIP_EINVAL, "sys1hip_set_chain_wait: null context");
  if (wait_us < 1 || wait_us > 1000000 || extra < 0)
    return fail(SYS1HIP_EINVAL, "sys1hip_set_chain_wait: wait_us %d (1..1000000), extra %d", (int)wait_us,
                (int)extra);
  Context* c = static_cast<Context*>(ctx);
  c->chain_wait_us = wait_us;
  c->chain_extra = extra;
  return SYS1HIP_OK;
}

}  // extern "C"
