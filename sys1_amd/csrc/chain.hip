// Several row-local projections in one persistent launch (the projection
// chain of one transformer layer between two attention calls):
//   attn.Wo (+residual) -> Wi (+GeGLU) -> mlp.Wo (+residual) -> next Wqkv
// (src/archs/modernbert.rs:857-887), or the Qwen3.5 out_proj / o_proj ->
// gate_up (+SwiGLU) -> down (+residual) -> next in_proj (:932-940).
//
// Projection p reads rows that projections before it wrote, at the same
// rows only (every projection is row-independent), so its tile on row panel
// r can start as soon as every tile of projection p-1 on that panel is done.
// One launch then replaces the per-projection launches: no launch gaps, and
// the tail of one projection overlaps the head of the next.
//
// Schedule.  Row panel r (BM token rows) belongs to XCD r % nxcd for every
// projection of the chain, so a panel's producer and consumers share that
// XCD's L2: the consumer reads what the producer wrote through the same L2
// (loads bypass the per-CU L1 with the sc0 policy), and the panel is still
// in the L2 when the next projection reads it.  Each XCD keeps a queue of its
// tiles, projection-major and row-panel-major inside a projection; a
// workgroup reads its XCD id from the hardware (HW_REG_XCC_ID) and takes
// tiles from that queue with an atomic counter, one tile ahead of the one it
// computes.  Taking tiles in queue order makes the launch deadlock-free
// whatever the residency: a tile waits only for tiles earlier in the queue,
// which are held by running workgroups.
//
// Dependencies.  A compute wave that has stored its part of a tile waits for
// its stores (vmcnt 0) and adds 1 to the tile's (projection, row panel)
// counter; the panel is complete for projection p when the counter reaches
// tiles_n(p) x compute waves.  Counters live in the context's bank, zeroed
// at the end of every launch by its last workgroup, so a launch (and a graph
// replay of it) always starts from zeros without a memset.
//
// Pipeline.  The tile loop is the producer-wave loop of gemm_tile_kernel
// (four producer waves issue the direct-to-LDS refills, STAGES stages, the
// k-tile stream runs across tiles).  The next tile's loads are issued
// STAGES - 1 k-tiles before the current tile ends; compute wave 0 takes
// that tile when the current one starts and publishes, just before then,
// whether its dependency is met.  If it is, the
// stream runs on; if not, the producers stop issuing, and after the current
// tile's last barrier the compute waves finish the tile (epilogue and
// counter) while the producers wait for the dependency, issue the next
// tile's first k-tiles and meet them at one extra barrier (a drain).  A
// producer never waits while its own compute waves have work left, so a
// tile that depends on the workgroup's own current tile cannot deadlock.
//
// Every wait is bounded (wait_us of real time, and no waiting at all once
// one wait of the launch has expired); one that expires sets bit 1 of the
// error word and goes on, so the launch always finishes; the caller reads
// the word with sys1hip_chain_status.
#include "chain.hpp"
#include "gemm_tile.hpp"
#include "skinny.hpp"

namespace sys1 {

namespace {

constexpr int kPolicySc0 = 1;  // buffer cache policy: sc0 (miss in the CU's L1, read the L2)
#ifndef SYS1_X_POLICY
#define SYS1_X_POLICY kPolicySc0
#endif
#ifndef SYS1_RES_POLICY
#define SYS1_RES_POLICY kPolicySc0
#endif

__device__ __forceinline__ int hw_xcc_id() {
  int v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xf;
}

__device__ __forceinline__ unsigned atomic_load_agent(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The kernel's arguments, read in place from the kernarg segment (constant
// address space): a projection's fields are scalar loads at a wave-uniform
// offset, and nothing is copied to private memory.
typedef const ChainArgs __attribute__((address_space(4)))* KArgs;

#define CHAIN_FIELD(a, p, f) ((a)->proj[(p)].f)

__device__ __forceinline__ ChainProj proj_at(KArgs a, int p) {
  ChainProj P;
  P.x = a->proj[p].x;
  P.w = a->proj[p].w;
  P.resid = a->proj[p].resid;
  P.y = a->proj[p].y;
  P.ldx = a->proj[p].ldx;
  P.ldw = a->proj[p].ldw;
  P.ldr = a->proj[p].ldr;
  P.ldy = a->proj[p].ldy;
  P.N = a->proj[p].N;
  P.K = a->proj[p].K;
  P.Nout = a->proj[p].Nout;
  P.epi = a->proj[p].epi;
  P.w_kt = a->proj[p].w_kt;
  P.tiles_n = a->proj[p].tiles_n;
  P.kt_count = a->proj[p].kt_count;
  return P;
}

}  // namespace

// Whether this workgroup is the launch's last to exit (wave 0 calls it; the
// result is wave-uniform).  Exits are counted in two levels, per slot of
// kStreamSlots workgroups and then per slot: same-address atomics serialise
// (some 40 ns each, measured), and one counter for 256 exiting workgroups
// would add microseconds to the launch's tail.  The last one clears the
// exit counters; the caller clears the rest of the bank.
__device__ bool chain_exit_last(unsigned* bank, int lane) {
  unsigned* const exits = bank + kChainExitWords;
  unsigned* const done = bank + kChainXcdMax;
  const int es = (int)(blockIdx.x % kStreamSlots);
  const unsigned members = (gridDim.x - es + kStreamSlots - 1) / kStreamSlots;
  const unsigned groups = min(gridDim.x, (unsigned)kStreamSlots);
  unsigned last = 0;
  if (lane == 0) {
    const unsigned prev =
        __hip_atomic_fetch_add(exits + es * kStreamSlotStride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == members - 1)
      last = __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1 == groups;
  }
  last = __builtin_amdgcn_readfirstlane(last);
  if (last && lane < kStreamSlots)
    __hip_atomic_store(exits + lane * kStreamSlotStride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return last != 0;
}

template <int BM, int BN, int WM, int WN, int STAGES, int PW>
__global__ __launch_bounds__((WM * WN + PW) * 64)
__attribute__((amdgpu_waves_per_eu(((WM * WN + PW) + 3) / 4))) void chain_kernel(ChainArgs) {
  const KArgs a = (KArgs)__builtin_amdgcn_kernarg_segment_ptr();
  using S = TileShape<BM, BN, WM, WN, STAGES, 64>;
  constexpr int BK = 64;
  constexpr int kWaves = S::kWaves;
  static_assert(PW > 0, "the chain schedule runs on producer waves");
  constexpr int kDW = PW;
  constexpr int kDma = S::DT / kDW;
  constexpr int kXDma = S::XT / kDW;
  static_assert(S::XT % kDW == 0 && S::DT % kDW == 0, "x and w instructions deal evenly over the producers");
  static_assert(kDma * (STAGES - 1) < 64, "vmcnt field");
  constexpr int kReads = S::FM + S::FN;
  static_assert(S::KS == 4 && kReads * 16 <= 64, "four fragment sets per k-tile (kDeep schedule)");

  __shared__ __attribute__((aligned(1024))) char lds[S::kLdsBytes];
  __shared__ int slot_id[4];     // queue index of tile n (n % 4), -1 past the end
  __shared__ int slot_ready[4];  // its dependency was met when it was taken
  __shared__ int drain_met;      // tile sequence number whose deferred dependency producer 0 saw met

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  const uint64_t t_entry = a->trace ? wall_clock64() : 0;
  const int xcc = hw_xcc_id();
  const bool active = xcc < a->nxcd;
  int tiles_n[kChainMax];
#pragma unroll
  for (int p = 0; p < kChainMax; ++p) tiles_n[p] = p < a->nproj ? CHAIN_FIELD(a, p, tiles_n) : 0;
  const XcdQueue q(active ? xcc : 0, a->nxcd, a->row_panels, a->nproj, tiles_n);
  unsigned* const heads = a->bank;                 // [kChainXcdMax] queue heads
  unsigned* const aborted = a->bank + kChainXcdMax + 1;  // a wait of this launch expired
  unsigned* const deps = a->bank + kChainHeader;   // [nproj][row_panels]

  auto dep_met = [&](const ChainTile& t) -> bool {
    if (t.p == 0) return true;
    const unsigned need = (unsigned)(CHAIN_FIELD(a, t.p - 1, tiles_n) * kWaves + a->dep_extra);
    return atomic_load_agent(deps + (t.p - 1) * a->row_panels + t.rp) >= need;
  };
  // Bounded wait for a tile's dependency: at most wait_us of real time (the
  // 100 MHz constant clock), and none at all once any wait of this launch
  // has expired.  An expired wait is reported and passed: the launch still
  // finishes, and its results are then not to be used.  One wave per
  // workgroup polls, backing off to about a microsecond between polls: the
  // counters of a row panel are polled by every workgroup that waits for
  // it, and faster polling floods the memory channel that holds them.
  auto wait_dep = [&](const ChainTile& t) {
    if (dep_met(t)) return;
    if (atomic_load_agent(aborted)) return;
    const uint64_t t0 = wall_clock64();
    const uint64_t budget = (uint64_t)a->wait_us * 100;
    for (int n = 1; !dep_met(t); ++n) {
      if (wall_clock64() - t0 > budget || ((n & 15) == 0 && atomic_load_agent(aborted))) {
        if (lane == 0) {
          __hip_atomic_store(aborted, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_fetch_or(a->err, kChainErrTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
      }
      if (n < 4) __builtin_amdgcn_s_sleep(8);
      else __builtin_amdgcn_s_sleep(32);
    }
  };
  // Compute wave 0 takes the tiles: the next one is taken (one atomic) when
  // the current one starts, its dependency is polled one k-tile before the
  // decision and published with it (slot n % 4) before the barrier after
  // which the producers would issue its first k-tile.  Compute waves have no
  // loads in flight, so these round trips overlap their MFMAs instead of
  // draining the refills.
  auto grab = [&]() -> unsigned {
    unsigned i = 0xffffffffu;
    if (lane == 0) i = __hip_atomic_fetch_add(heads + q.xcc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return i;
  };
  auto id_of = [&](unsigned raw) -> int {
    const int i = (int)__builtin_amdgcn_readfirstlane(raw);
    return i >= 0 && i < q.total ? i : -1;
  };
  auto publish = [&](int n, int id, int ready) {
    if (lane == 0) {
      slot_id[n & 3] = id;
      slot_ready[n & 3] = ready;
    }
  };
  const bool producer = wave >= kWaves;
  if (tid == 0) drain_met = 0;
  if (active && wave == 0) {
    const int id = id_of(grab());
    if (id >= 0) wait_dep(q.decode(id));
    publish(0, id, 1);
  }
  __syncthreads();  // B_init
  const int first = active ? __builtin_amdgcn_readfirstlane(slot_id[0]) : -1;

  if (first >= 0 && producer) {
    // ---------------------------------------------------------------- producers
    const int dwave = wave - kWaves;
    const int lrow = lane / S::CPR, lpos = lane % S::CPR;
    auto dma_row = [&](int i) {
      const int u = i * kDW + dwave;
      return (i < kXDma ? u : u - S::XT) * S::RPI + lrow;
    };
    // issue cursor: tile, its projection's operands, k-tile
    ChainTile it = q.decode(first);
    int ikt = 0, ikc = CHAIN_FIELD(a, it.p, kt_count);
    unsigned src_off[kDma];
    rsrc_t xr, wr;
    auto enter = [&](const ChainTile& t) {
      const ChainProj P = proj_at(a, t.p);
      const int m0 = t.rp * BM, n0 = t.tn * BN;
      const int x_left = a->M - 1 - m0, w_left = P.N - 1 - n0;
#pragma unroll
      for (int i = 0; i < kDma; ++i) {
        const int r = dma_row(i);
        const int c = lpos ^ lds_swz<BK>(r);
        const int rw = min(r, w_left);
        src_off[i] = i < kXDma ? (unsigned)(min(r, x_left) * (int)P.ldx * 2 + c * 16)
                     : P.w_kt ? (unsigned)((rw / kBlkRows) * P.w_kt * kBlkBytes + (rw % kBlkRows) * (kBlkK * 2) + c * 16)
                              : (unsigned)(rw * (int)P.ldw * 2 + c * 16);
      }
      xr = make_rsrc_uniform(reinterpret_cast<const char*>(P.x + (int64_t)m0 * P.ldx), 0x7ffffff0);
      wr = make_rsrc_uniform(P.w_kt ? reinterpret_cast<const char*>(P.w) + (int64_t)(n0 / kBlkRows) * P.w_kt * kBlkBytes
                                    : reinterpret_cast<const char*>(P.w + (int64_t)n0 * P.ldw),
                             0x7ffffff0);
      ikc = P.kt_count;
      ikt = 0;
    };
    int w_kt_cur = CHAIN_FIELD(a, it.p, w_kt);
    enter(it);
    auto issue = [&](int stage) {  // the cursor's k-tile into `stage`
      char* const base = lds + stage * S::kStageBytes;
      const int xk = ikt * BK * 2;
      const int wk = w_kt_cur ? ikt * kBlkBytes : ikt * BK * 2;
#pragma unroll
      for (int i = 0; i < kDma; ++i) {
        lds_void* dst = (lds_void*)(base + (i * kDW + dwave) * 1024);
        if (i < kXDma)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, dst, 16, (int)src_off[i], xk, 0, SYS1_X_POLICY);
        else
          __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, dst, 16, (int)src_off[i], wk, 0, 0);
      }
      ++ikt;
    };

    int n = 0;             // tile sequence number of the issue cursor
    int F_next = ikc;      // first step of tile n + 1
    int issued = 0;        // steps [0, issued) issued
    int last_step = -1;    // the end: steps stop after this barrier
    int drain_at = -1;     // the deferred next tile is met after this barrier
    int next_id = -1;
    for (int t = 0; t < STAGES; ++t) issue(t);
    issued = STAGES;
    vm_wait<(STAGES - 1) * kDma>();
    __syncthreads();  // B_start
    for (int s = 0;; ++s) {
      if (issued >= s + STAGES) vm_wait<(STAGES - 2) * kDma>();
      else vm_wait<0>();
      __syncthreads();  // barrier(s)
      if (s + STAGES == F_next && last_step < 0 && drain_at < 0) {
        next_id = __builtin_amdgcn_readfirstlane(slot_id[(n + 1) & 3]);
        if (next_id < 0) last_step = F_next - 1;
        else if (!__builtin_amdgcn_readfirstlane(slot_ready[(n + 1) & 3])) drain_at = F_next - 1;
        else {
          ++n;
          it = q.decode(next_id);
          w_kt_cur = CHAIN_FIELD(a, it.p, w_kt);
          enter(it);
          F_next += ikc;
        }
      }
      if (s == last_step) break;
      if (s == drain_at) {
        const ChainTile nt = q.decode(next_id);
        if (dwave == 0) {
          wait_dep(nt);
          if (lane == 0) __hip_atomic_store(&drain_met, n + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        } else {
          while (__hip_atomic_load(&drain_met, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) != n + 1)
            __builtin_amdgcn_s_sleep(2);
        }
        ++n;
        it = nt;
        w_kt_cur = CHAIN_FIELD(a, it.p, w_kt);
        enter(it);
        F_next += ikc;
        const int stage0 = (s + 1) % STAGES;
        for (int t = 0; t < STAGES; ++t) issue((stage0 + t) % STAGES);
        issued = s + 1 + STAGES;
        vm_wait<(STAGES - 1) * kDma>();
        drain_at = -1;
        __syncthreads();  // barrier(D)
        continue;
      }
      const int qs = s + STAGES;  // the step issued into the stage just freed
      if (qs < F_next && issued == qs) {
        issue(s % STAGES);
        issued = qs + 1;
      }
    }
    vm_wait<0>();
  } else if (first >= 0) {
    // ------------------------------------------------------------ compute waves
    const int wm = wave / WN;
    const int wn = wave % WN;
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
    auto mma = [&](const Frags& f) {
#pragma unroll
      for (int i = 0; i < S::FN; ++i)
#pragma unroll
        for (int j = 0; j < S::FM; ++j) acc[i][j] = mfma32(f.w[i], f.x[j], acc[i][j]);
    };
    auto pair16 = [](bf16x4 lo, bf16x4 hi) -> bf16x8 {
      const i32x2 u = __builtin_bit_cast(i32x2, lo), v = __builtin_bit_cast(i32x2, hi);
      const auto s0 = __builtin_amdgcn_permlane32_swap((unsigned)u[0], (unsigned)v[0], false, false);
      const auto s1 = __builtin_amdgcn_permlane32_swap((unsigned)u[1], (unsigned)v[1], false, false);
      const i32x4 r = {(int)s0[0], (int)s1[0], (int)s0[1], (int)s1[1]};
      return __builtin_bit_cast(bf16x8, r);
    };
    // Epilogue of tile t straight from registers (the layout and rounding of
    // gemm_tile_kernel's): lanes l and l+32 swap halves so every lane stores
    // 16 contiguous bytes; residual reads bypass the L1 (sc0), since another
    // CU of this XCD may have written those rows during this launch.
    auto epilogue_as = [&](const ChainTile& t, auto ec) {
      constexpr int E = decltype(ec)::value;
      const ChainProj P = proj_at(a, t.p);
      const int m0 = t.rp * BM, n0 = t.tn * BN;
      constexpr bool kGated = E == kEpiGeglu || E == kEpiSwiglu;
      const int out_n0 = kGated ? (n0 + wn * S::TN) / 2 : n0 + wn * S::TN;
      // The residual of every element this lane stores is loaded first, all
      // loads in flight together: y may alias the residual (the in-place
      // update of the hidden state), so a load issued after a store could
      // not be moved ahead of it, and each would wait a full round trip.
      // Each lane reads exactly the elements it then writes, so reading all
      // of them first is correct for an in-place update too.
      bf16x8 res[S::FM][S::FN][2];
      if constexpr (E == kEpiResidual) {
        const rsrc_t rr = make_rsrc_uniform(P.resid, 0x7ffffff0);
#pragma unroll
        for (int j = 0; j < S::FM; ++j) {
          const int m = m0 + wm * S::TM + j * 32 + frow;
#pragma unroll
          for (int i = 0; i < S::FN; ++i)
#pragma unroll
            for (int gp = 0; gp < 2; ++gp) {
              const int nn = out_n0 + i * 32 + 16 * gp + 8 * fk;
              // (Nout % 8 == 0, 16-byte aligned rows, M ldr 2 < 2 GiB: checked
              // by the host; rows past M and columns past Nout read zeros)
              const unsigned off = m < a->M && nn < P.Nout ? (unsigned)(((int64_t)m * P.ldr + nn) * 2) : kOutOfRange;
#ifdef SYS1_RES_NOLOAD
              res[j][i][gp] = bf16x8{};
              (void)off;
#else
              res[j][i][gp] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rr, (int)off, 0, SYS1_RES_POLICY));
#endif
            }
        }
      }
#pragma unroll
      for (int j = 0; j < S::FM; ++j) {
        const int m = m0 + wm * S::TM + j * 32 + frow;
        const bool row_ok = m < a->M;
#pragma unroll
        for (int i = 0; i < S::FN; ++i) {
          if constexpr (kGated) {
            bf16x4 o[2];
#pragma unroll
            for (int g = 0; g < 2; ++g)
#pragma unroll
              for (int e = 0; e < 4; ++e) o[g][e] = to_bf16(epi_gate<E>(acc[i][j][4 * g + e], acc[i][j][4 * (g + 2) + e]));
            const bf16x8 v = pair16(o[0], o[1]);
            const int nn = out_n0 + i * 16 + 8 * fk;
            if (row_ok && nn < P.Nout) store8(P.y + (int64_t)m * P.ldy + nn, v, P.Nout - nn);
          } else {
#pragma unroll
            for (int gp = 0; gp < 2; ++gp) {
              bf16x4 pv[2];
#pragma unroll
              for (int qq = 0; qq < 2; ++qq)
#pragma unroll
                for (int e = 0; e < 4; ++e) pv[qq][e] = to_bf16(acc[i][j][4 * (2 * gp + qq) + e]);
              bf16x8 v = pair16(pv[0], pv[1]);
              const int nn = out_n0 + i * 32 + 16 * gp + 8 * fk;
              if (row_ok && nn < P.Nout) {
                if constexpr (E == kEpiResidual) {
#pragma unroll
                  for (int e = 0; e < 8; ++e) v[e] = to_bf16(round_bf16(to_f32(v[e]) + to_f32(res[j][i][gp][e])));
                }
                store8(P.y + (int64_t)m * P.ldy + nn, v, P.Nout - nn);
              }
            }
          }
        }
      }
    };
    // Epilogue of tile t straight from registers (the layout and rounding of
    // gemm_tile_kernel's): lanes l and l+32 swap halves so every lane stores
    // 16 contiguous bytes; residual reads bypass the L1 (sc0), since another
    // CU of this XCD may have written those rows during this launch.
    auto epilogue = [&](const ChainTile& t) {
      using std::integral_constant;
      switch (CHAIN_FIELD(a, t.p, epi)) {
        case kEpiResidual: epilogue_as(t, integral_constant<int, kEpiResidual>()); break;
        case kEpiGeglu: epilogue_as(t, integral_constant<int, kEpiGeglu>()); break;
        case kEpiSwiglu: epilogue_as(t, integral_constant<int, kEpiSwiglu>()); break;
        default: epilogue_as(t, integral_constant<int, kEpiNone>()); break;
      }
    };
    // This wave's part of tile t is counted once its stores are done.  When
    // the next tile streams in, that happens a k-step into it (the MFMAs go
    // on while the stores drain); before a drain or the end, at once (the
    // next tile may depend on this one).
    auto release = [&](const ChainTile& t) {
      vm_wait<0>();
      if (lane == 0)
        __hip_atomic_fetch_add(deps + t.p * a->row_panels + t.rp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    bool pending = false;
    ChainTile pend_tile{0, 0, 0};

    ChainTile ct = q.decode(first);
    int kc = CHAIN_FIELD(a, ct.p, kt_count);
    int ckt = 0;
    int n = 0;
    int cur_id = first;
    uint64_t t_start = 0, t_epi = 0;
    bool drained = false;
    unsigned long long* const trace = a->trace;
    auto record = [&]() {
      if (trace && wave == 0 && lane == 0 && n < kChainTraceTiles - 1) {
        unsigned long long* r = trace + ((size_t)blockIdx.x * kChainTraceTiles + n) * 4;
        r[0] = (unsigned long long)cur_id | ((unsigned long long)q.xcc << 32) | ((unsigned long long)drained << 40);
        r[1] = t_start;
        r[2] = wall_clock64();
        r[3] = (unsigned long long)ct.p | ((unsigned long long)(t_epi - t_start) << 8);
      }
    };
    zero_acc();
    Frags fr[4];
    unsigned next_raw = 0xffffffffu, poll_raw = 0;
    int next_id = -1;
    ChainTile next_tile{0, 0, 0};
    __syncthreads();  // B_start
    if (trace) {
      t_start = wall_clock64();
      if (wave == 0 && lane == 0) {  // the last record: kernel entry and first data in LDS
        unsigned long long* r = trace + ((size_t)blockIdx.x * kChainTraceTiles + kChainTraceTiles - 1) * 4;
        r[0] = 0xffffffffull;
        r[1] = t_entry;
        r[2] = t_start;
        r[3] = 0;
      }
    }
    read(fr[0], 0, 0);
    read(fr[1], 0, 1);
    int stage = 0;
    for (;;) {
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
      const int rel_at = kc > STAGES + 1 ? 1 : 0;
      if (pending && ckt == rel_at) {
        release(pend_tile);
        pending = false;
      }
      if (wave == 0) {
        if (ckt == rel_at) next_raw = grab();
        if (ckt == max(0, kc - STAGES - 1)) {
          next_id = id_of(next_raw);
          next_tile = next_id >= 0 ? q.decode(next_id) : ChainTile{0, 0, 0};
          if (next_tile.p > 0 && lane == 0)
            poll_raw = atomic_load_agent(deps + (next_tile.p - 1) * a->row_panels + next_tile.rp);
        }
        if (ckt == kc - STAGES) {
          int ready = 1;
          if (next_id >= 0 && next_tile.p > 0) {
            const unsigned need = (unsigned)(CHAIN_FIELD(a, next_tile.p - 1, tiles_n) * kWaves + a->dep_extra);
            ready = __builtin_amdgcn_readfirstlane(poll_raw) >= need ? 1 : 0;
          }
          publish(n + 1, next_id, ready);
        }
      }
      __syncthreads();  // barrier(s)
      stage = stage + 1 == STAGES ? 0 : stage + 1;
      // The next k-tile's first fragments (unless the tile ends without its
      // successor streamed in), then this k-tile's last MFMAs.
      const bool last = ckt + 1 == kc;
      const int nid = last ? __builtin_amdgcn_readfirstlane(slot_id[(n + 1) & 3]) : 0;
      const bool streamed = !last || (nid >= 0 && __builtin_amdgcn_readfirstlane(slot_ready[(n + 1) & 3]));
      if (streamed) {
        read(fr[0], stage, 0);
        read(fr[1], stage, 1);
      }
      __builtin_amdgcn_sched_barrier(0);
      mma(fr[2]);
      __builtin_amdgcn_sched_barrier(0);
      mma(fr[3]);
      __builtin_amdgcn_sched_barrier(0);
      if (!last) {
        ++ckt;
        continue;
      }
      if (trace) t_epi = wall_clock64();
      epilogue(ct);
      zero_acc();
      if (streamed) {
        pending = true;
        pend_tile = ct;
      } else {
        release(ct);
      }
      if (trace) record();
      if (nid < 0) break;
      if (!streamed) {
        __syncthreads();  // barrier(D): the producers have the next tile's first k-tiles in
        read(fr[0], stage, 0);
        read(fr[1], stage, 1);
      }
      if (trace) {
        t_start = wall_clock64();
        drained = !streamed;
        cur_id = nid;
      }
      ++n;
      ct = q.decode(nid);
      kc = CHAIN_FIELD(a, ct.p, kt_count);
      ckt = 0;
    }
  }

  // ------------------------------------------------------------------ the end
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();  // B_final
  if (!active && tid == 0)
    __hip_atomic_fetch_or(a->err, kChainErrXcc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (wave == 0) {
    if (chain_exit_last(a->bank, lane)) {
      // The last workgroup: every queue must have been drained (an XCD
      // without workgroups would leave its tiles undone), then the bank is
      // cleared for the next launch.
      if (lane < a->nxcd) {
        const XcdQueue ql(lane, a->nxcd, a->row_panels, a->nproj, tiles_n);
        if ((int)atomic_load_agent(heads + lane) < ql.total)
          __hip_atomic_fetch_or(a->err, kChainErrUndrained, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      const int words = kChainHeader + a->nproj * a->row_panels;
      for (int i = lane; i < words; i += 64)
        __hip_atomic_store(a->bank + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---------------------------------------------------------------------------
// The same chain for a few dozen tokens: a weight stream.  Up to 64 token rows
// (one 64-row tile), every projection is a stream of its weight, and a
// projection's rows depend on all of the previous projection's output
// columns.  Work items are 32-column blocks of a projection over the whole K
// (the skinny kernels' tile: K split over the NW waves of a workgroup, f32
// partials summed in LDS in wave order), taken from one queue in
// projection-major order by every CU.  A workgroup issues the loads of its
// item's weight share first -- they depend on nothing -- and only then waits
// until the previous projection's items are all done, so the weight of the
// next projection streams in while the current one finishes.  Outputs and
// activations cross XCDs here (below: how they stay coherent); the
// dependency counters are agent-scope atomics.
constexpr int kPolicySc1 = 16;
#ifndef SYS1_STREAM_FENCES
#define SYS1_STREAM_FENCES 0
#endif
// Coherence across XCDs.  Default (0): every output store writes through
// and every activation / residual load bypasses the L2 (sc1), as the
// stream-K partials do.  1: ordinary cached accesses, with an agent-scope
// release fence before each counter add (the XCD's L2 written back) and an
// acquire fence after each wait (the L2 invalidated), so an activation is
// read once per XCD rather than once per workgroup.  2: write-through stores
// and the acquire fence only.  Measured (ModernBERT-large chain, M = 1 and
// 64): 0 fastest, 2 +5-8%, 1 +15-30% -- the L2 write-back and invalidation
// on every item cost more than the re-reads they save.
constexpr int kStreamPolicy = SYS1_STREAM_FENCES ? 0 : kPolicySc1;
constexpr int kStreamStorePolicy = SYS1_STREAM_FENCES == 1 ? 0 : kPolicySc1;

template <int FM, int FN, int NW, int SMAX, int G>
__global__ __launch_bounds__(NW * 64) void stream_chain_kernel(ChainArgs) {
  const KArgs a = (KArgs)__builtin_amdgcn_kernarg_segment_ptr();
  constexpr int BM = FM * 16, BN = FN * 16;
  constexpr int kRowF32 = BN + 4;
  static_assert(NW * BM * kRowF32 * 4 <= 160 * 1024, "LDS budget");
  static_assert(FN % 2 == 0, "whole 32-row gate/up groups per item");
  static_assert(BM * BN / 8 <= NW * 64, "one epilogue vector per thread");
  __shared__ __attribute__((aligned(16))) float red[NW * BM * kRowF32];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, q = lane >> 4;
  unsigned* const aborted = a->bank + kChainXcdMax + 1;
  // Items finished, per projection, counted on kStreamSlots counters (item
  // cb on counter cb % kStreamSlots, one 128-byte line each): same-address
  // atomics serialise, and one counter for the 164 items of a GeGLU
  // projection cost microseconds.
  unsigned* const deps = a->bank + kChainHeader;
  auto dep_word = [&](int p, int s) { return deps + (p * kStreamSlots + s) * kStreamSlotStride; };
  int total = 0;
#pragma unroll
  for (int p = 0; p < kChainMax; ++p) total += p < a->nproj ? a->proj[p].tiles_n : 0;
  auto decode = [&](int i, int& p, int& cb) {
    p = 0;
    int base = 0;
#pragma unroll
    for (int pp = 0; pp + 1 < kChainMax; ++pp) {
      const int c = a->proj[pp].tiles_n;
      if (p == pp && pp + 1 < a->nproj && i >= base + c) {
        base += c;
        p = pp + 1;
      }
    }
    cb = i - base;
  };
  // Whether every item of projection p is done: lane s reads counter s.
  auto items_done = [&](int p) -> bool {
    unsigned need = 0, have = 0;
    if (lane < kStreamSlots) {
      const int tn = a->proj[p].tiles_n;
      need = (unsigned)(max(0, (tn - lane + kStreamSlots - 1) / kStreamSlots) + a->dep_extra);
      have = atomic_load_agent(dep_word(p, lane));
    }
    return __ballot(have < need) == 0;
  };
  // Bounded wait (wave 0) for all items of projection p: as the tile chain's.
  auto wait_items = [&](int p) {
    if (items_done(p) || atomic_load_agent(aborted)) return;
    const uint64_t t0 = wall_clock64();
    const uint64_t budget = (uint64_t)a->wait_us * 100;
    for (int n = 1; !items_done(p); ++n) {
      if (wall_clock64() - t0 > budget || ((n & 15) == 0 && atomic_load_agent(aborted))) {
        if (lane == 0) {
          __hip_atomic_store(aborted, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_fetch_or(a->err, kChainErrTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
      }
      __builtin_amdgcn_s_sleep(4);
    }
  };

  // Optional timeline (a->trace): per item, {id | p << 32, start, end of
  // the dependency wait, end}, wall-clock ticks of 10 ns.
  unsigned long long* const trace = a->trace;
  uint64_t t_item = 0, t_dep = 0;
  // A static schedule: workgroup b takes items b, b + grid, b + 2 grid, ...
  // (every workgroup's items in increasing order, so the lowest unfinished
  // item is always some workgroup's current one, and its dependencies --
  // items of lower index -- are done: no deadlock).  With one resident
  // workgroup per CU and ModernBERT-large's 324 items, the second round is
  // the last projection's, taken by the workgroups of the first two.
  for (int n = 0;; ++n) {
    const int64_t id64 = (int64_t)blockIdx.x + (int64_t)n * gridDim.x;
    if (id64 >= total) break;
    const int id = (int)id64;
    if (trace) t_item = wall_clock64();
    int p, cb;
    decode(id, p, cb);
    const ChainProj P = proj_at(a, p);
    const int n0 = cb * BN;

    // ---- this wave's share of K: k-steps [s0, s1) of 32
    const int ksteps = (P.K + 31) / 32;
    const int s0 = wave * ksteps / NW, s1 = (wave + 1) * ksteps / NW;
    const rsrc_t wr = make_rsrc_uniform(P.w, 0x7ffffff0);
    const rsrc_t xr = make_rsrc_uniform(P.x, 0x7ffffff0);
    unsigned wo[FN], xo[FM];
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      const int nr = min(n0 + i * 16 + r16, P.N - 1);
      wo[i] = P.w_kt ? (unsigned)((nr / kBlkRows) * P.w_kt * kBlkBytes + (nr % kBlkRows) * (kBlkK * 2) + q * 16)
                     : (unsigned)((int64_t)nr * P.ldw * 2 + q * 16);
    }
#pragma unroll
    for (int j = 0; j < FM; ++j) xo[j] = (unsigned)((int64_t)min(j * 16 + r16, a->M - 1) * P.ldx * 2 + q * 16);
    auto wstep = [&](int st) { return P.w_kt ? (st >> 1) * kBlkBytes + (st & 1) * 64 : st * 64; };
    // The weight share first: it depends on nothing.  (A wave without
    // k-steps -- K below 32 NW -- issues out-of-range loads at offset 0,
    // never a negative one.)
    i32x4 wreg[SMAX][FN];
#pragma unroll
    for (int u = 0; u < SMAX; ++u) {
      const int st = s0 + u;
      const bool ok = st < s1 && st * 32 + q * 8 < P.K;
      const int sw = __builtin_amdgcn_readfirstlane(wstep(max(0, min(st, s1 - 1))));
#pragma unroll
      for (int i = 0; i < FN; ++i)
        wreg[u][i] = __builtin_amdgcn_raw_buffer_load_b128(wr, ok ? (int)wo[i] : (int)kOutOfRange, sw, 0);
    }
    // Then the dependency: every item of the previous projection.
    if (p > 0 && wave == 0) {
      wait_items(p - 1);
      if (SYS1_STREAM_FENCES) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    if (trace) t_dep = wall_clock64();
    // This thread's epilogue vector (8 output columns of one row), and its
    // residual, loaded now beside the activations rather than after the
    // reduction (after the wait, so a residual written by the previous
    // projection is complete).
    const bool gated = P.epi == kEpiGeglu || P.epi == kEpiSwiglu;
    const int kVecs = gated ? BN / 16 : BN / 8;
    const int out_n0 = gated ? n0 / 2 : n0;
    const int er = tid / kVecs, ec0 = (tid % kVecs) * 8, enn = out_n0 + ec0;
    const bool ep_ok = tid < BM * kVecs && er < a->M && enn < P.Nout;  // (Nout % 8 == 0: whole vectors)
    i32x4 rv_raw = i32x4{0, 0, 0, 0};
    if (P.epi == kEpiResidual && ep_ok) {
      const rsrc_t rr = make_rsrc_uniform(P.resid, 0x7ffffff0);
      rv_raw = __builtin_amdgcn_raw_buffer_load_b128(rr, (int)(((int64_t)er * P.ldr + enn) * 2), 0, kStreamPolicy);
    }
    f32x4 acc[FN][FM];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int g = 0; g < SMAX; g += G) {
      if (s0 + g < s1) {
        i32x4 xreg[G][FM];
#pragma unroll
        for (int u = 0; u < G; ++u) {
          const int st = s0 + g + u;
          const bool ok = g + u < SMAX && st < s1 && st * 32 + q * 8 < P.K;
          const int so = __builtin_amdgcn_readfirstlane(max(0, min(st, s1 - 1)) * 64);
#pragma unroll
          for (int j = 0; j < FM; ++j)
            xreg[u][j] = __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? (int)xo[j] : (int)kOutOfRange, so, kStreamPolicy);
        }
#pragma unroll
        for (int u = 0; u < G; ++u)
          if (g + u < SMAX)
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
              for (int j = 0; j < FM; ++j) acc[i][j] = mfma16(wreg[g + u][i], xreg[u][j], acc[i][j]);
      }
    }
    // Partials to LDS (wave w's block (i, j): rows 16 j + l % 16, columns
    // 16 i + 4 (l / 16) .. + 3), summed below in wave order.
    float* mine = red + wave * BM * kRowF32;
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j)
        *reinterpret_cast<f32x4*>(mine + (j * 16 + r16) * kRowF32 + i * 16 + 4 * q) = acc[i][j];
    __syncthreads();
    // Epilogue: one thread per 8 output columns of a row.
    const rsrc_t yr = make_rsrc_uniform(P.y, 0x7ffffff0);
    if (ep_ok) {
      const int r = er, c0 = ec0, nn = enn;
      const int pc = gated ? (c0 / 16) * 32 + c0 % 16 : c0;
      float v[8], gu[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = gu[e] = 0.0f;
      for (int ww = 0; ww < NW; ++ww) {
        const float* row = red + (ww * BM + r) * kRowF32;
        const f32x4 p0 = *reinterpret_cast<const f32x4*>(row + pc);
        const f32x4 p1 = *reinterpret_cast<const f32x4*>(row + pc + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] += p0[e];
          v[4 + e] += p1[e];
        }
        if (gated) {
          const f32x4 u0 = *reinterpret_cast<const f32x4*>(row + pc + 16);
          const f32x4 u1 = *reinterpret_cast<const f32x4*>(row + pc + 20);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            gu[e] += u0[e];
            gu[4 + e] += u1[e];
          }
        }
      }
      bf16x8 o;
      const unsigned yoff = (unsigned)(((int64_t)r * P.ldy + nn) * 2);
      if (P.epi == kEpiGeglu) {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = to_bf16(epi_gate<kEpiGeglu>(v[e], gu[e]));
      } else if (P.epi == kEpiSwiglu) {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = to_bf16(epi_gate<kEpiSwiglu>(v[e], gu[e]));
      } else if (P.epi == kEpiResidual) {
        const bf16x8 rv = __builtin_bit_cast(bf16x8, rv_raw);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = to_bf16(epi_apply<kEpiResidual>(v[e], 0.0f, to_f32(rv[e])));
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = to_bf16(epi_apply<kEpiNone>(v[e], 0.0f, 0.0f));
      }
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, o), yr, (int)yoff, 0, kStreamStorePolicy);
    }
    // The item is done once every thread's stores are: count it.
    vm_wait<0>();
    __syncthreads();
    if (wave == 0) {
      if (SYS1_STREAM_FENCES == 1) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      if (lane == 0) {
        __hip_atomic_fetch_add(dep_word(p, cb % kStreamSlots), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (trace && n < kChainTraceTiles) {
          unsigned long long* r = trace + ((size_t)blockIdx.x * kChainTraceTiles + n) * 4;
          r[0] = (unsigned long long)id | ((unsigned long long)p << 32);
          r[1] = t_item;
          r[2] = t_dep;
          r[3] = wall_clock64();
        }
      }
    }
    __syncthreads();
  }

  // ---- the end: the last workgroup clears the bank
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (wave == 0 && chain_exit_last(a->bank, lane)) {
    for (int i = lane; i < kChainHeader; i += 64)
      __hip_atomic_store(a->bank + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int i = lane; i < a->nproj * kStreamSlots; i += 64)
      __hip_atomic_store(dep_word(i / kStreamSlots, i % kStreamSlots), 0u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The weight-streaming chain's shape: 64 token rows x 32 columns per item,
// K over 12 waves (three per SIMD, 170 registers each), at most 7 k-steps of
// 32 per wave (K <= 2688), activations loaded 4 k-steps at a time.
const ChainKernel kStreamChainKernel = {
    reinterpret_cast<const void*>(&stream_chain_kernel<4, 2, 12, 7, 4>), 64, 32, 7 * 32 * 12, 12 * 64};

// The chain's tile shape: ModernBERT-base's output projections' shape
// (N = 768 -> four 192-wide tiles), eight 32 x 96 compute waves and four
// producer waves, three stages (120 KB of LDS), one workgroup per CU.
#define SYS1_CHAIN_SHAPE 128, 192, 4, 2, 3, 4
const ChainKernel kChainKernel = {
    reinterpret_cast<const void*>(&chain_kernel<SYS1_CHAIN_SHAPE>), 128, 192, 3, (4 * 2 + 4) * 64};

}  // namespace sys1
