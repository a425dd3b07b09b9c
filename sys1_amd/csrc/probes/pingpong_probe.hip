// Measurement probe, not part of libsys1hip: a rotating-group ("ping-pong")
// bf16 GEMM y[M,N] = x[M,K] . w[N,K]^T for gfx950, with switches that take
// parts of its k-loop away, so that each part's cost can be read off.
//
// Build and run (one MI355X):
//   hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature \
//         -Xclang -packed-fp32-ops sys1_amd/csrc/probes/pingpong_probe.hip -o /tmp/pingpong_probe
//   /tmp/pingpong_probe [modes|epilogue|rotation|square]   (no argument: all)
//   (run each GPU step under `timeout -k 10 120`)
//
// Kernel.  A workgroup computes a BM x BN output tile (BM tokens, BN output
// features) with 4 NG waves in NG groups of four (group = wave / 4; waves are
// placed round-robin on the four SIMDs, so each SIMD holds one wave of every
// group).  Each wave owns a (BM / WM) x (BN / WN) sub-tile of 16 x 16 blocks
// on v_mfma_f32_16x16x32_bf16.  K runs in units of 32; S LDS stages of
// (BM + BN) rows x 64 B are filled by direct-to-LDS buffer loads (1 KB per
// instruction: 16 rows x 64 B) that every wave issues its share of.  The
// groups rotate through barrier intervals: in each interval exactly one group
// runs its MFMAs on fragments it read earlier while the others read their
// next fragments from LDS and issue refills.  The first group starts computing
// one interval after the initial barrier, the next one interval later, and so
// on.
//   LDS layout: a 64-byte row holds 4 chunks of 8 k values; chunk c of row r
//   sits at position c ^ ((r >> 1) & 3).  With 16 x 16 x 32 operand reads
//   (lane l: row l % 16, chunk l / 16) that arrangement measured free of LDS
//   bank conflicts on gfx950 (SQ_LDS_BANK_CONFLICT = 0); (r ^ (r >> 2)) & 3
//   measured 4 conflict cycles per read.
//
// MODE (what the k-loop keeps):
//   0  everything (the GEMM);
//   1  no refills after the prologue (LDS reads and MFMAs on stale stages);
//   2  no LDS reads and no refills (MFMAs and barriers only, on constant
//      fragments: a data-dependent shader clock is not separated from it);
//   3  refills as in 0 but no LDS reads (MFMAs on constant fragments);
//   4  LDS reads and refills as in 0, the refills from a 64-row window of
//      x and of w (L2-resident after the first touch).
// The shader clock printed with each timeline separates clock effects.
// EPI_LDS: the epilogue stages the bf16 tile in LDS (two halves of BM / 2
//   rows) and stores it with 16-byte row-contiguous lane accesses; otherwise
//   each lane stores its 4 features of a block (8 bytes).
// ROT: 1 starts each tile's k-loop at unit (3 tn + 7 tm) mod (K / 32), so
//   workgroups that share an x or w panel read different k-slices at a time.
//
// Timeline: each workgroup records s_memrealtime (100 MHz) at entry, after
// the prologue's loads, after the k-loop and after the epilogue, and
// s_memtime (shader clock) at entry and exit; the host prints their spread,
// their averages and the mean shader clock for one launch.
//
// Output is checked against a plain f32 GPU reference on the shapes marked so
// (relative Frobenius error; bf16 rounding of the output gives ~1.7e-3).
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <vector>

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;
typedef __attribute__((address_space(3))) void lds_void;
typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Raw buffer descriptor from a wave-uniform base.  Both halves of the address
// are kept as unsigned 32-bit values: widening a signed low half would
// sign-extend into the high half and corrupt every address whose bit 31 is
// set.
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, int bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0,
                                           __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}
__device__ __forceinline__ f32x4 mfma16(const i32x4& a, const i32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}
template <int N>
__device__ __forceinline__ void vm_wait() {  // s_waitcnt vmcnt(N)
  __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15) | ((N >> 4) << 14));
}
__device__ __forceinline__ void lgkm_wait0() { __builtin_amdgcn_s_waitcnt(0xc07f); }
// A workgroup barrier that neither the compiler's scheduler nor its memory
// model moves anything across (and that adds no waits of its own).
__device__ __forceinline__ void bar() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}
__device__ __forceinline__ int swz4(int r) { return (r >> 1) & 3; }

template <int BM, int BN, int WM, int WN, int MODE, int S, bool EPI_LDS, int ROT>
__global__ __launch_bounds__(WM * WN * 64) __attribute__((amdgpu_waves_per_eu(WM * WN / 4))) void pp_kernel(
    const __bf16* __restrict__ x, const __bf16* __restrict__ w, __bf16* __restrict__ y, int M, int N, int K,
    uint64_t* tl) {
  uint64_t t_entry = __builtin_amdgcn_s_memrealtime(), t_loaded = 0, t_looped = 0;
  const uint64_t c_entry = __builtin_amdgcn_s_memtime();
  constexpr int NW = WM * WN, NG = NW / 4;
  static_assert(NW % 4 == 0, "whole groups of four waves");
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 16, FN = TN / 16;
  static_assert(TM % 16 == 0 && TN % 16 == 0, "whole 16 x 16 blocks");
  constexpr int kXBytes = BM * 64, kStage = (BM + BN) * 64;
  constexpr int DT = (BM + BN) / 16;  // 1 KB refill instructions per unit
  constexpr int XT = BM / 16;         // of which x
  constexpr int kDmaMax = (DT + NW - 1) / NW;
  static_assert(2 * kDmaMax < 64, "vmcnt field");
  __shared__ __attribute__((aligned(1024))) char lds[S * kStage];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2;
  const int wm = wave % WM, wn = wave / WM;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int tiles = tiles_m * tiles_n;
  const int U = K / 32;  // (K % 32 == 0: checked on the host)
  // Descriptor ranges end at the tensors: a read past them returns zeros.
  const rsrc_t xr = make_rsrc(x, M * K * 2), wr = make_rsrc(w, N * K * 2);
  // Refill instruction i * NW + wave of a unit is this wave's; the last
  // round of instructions may not reach every wave.
  const bool full = wave + (kDmaMax - 1) * NW < DT;

  const int lrow = lane >> 2, lpos = lane & 3;  // refill: 16 rows x 4 chunks
  const int r16 = lane & 15, q = lane >> 4;     // fragment: row, k chunk
  int xaddr[FM], waddr[FN];
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int r = wm * TM + j * 16 + r16;
    xaddr[j] = r * 64 + ((q ^ swz4(r)) << 4);
  }
#pragma unroll
  for (int i = 0; i < FN; ++i) {
    const int r = wn * TN + i * 16 + r16;
    waddr[i] = kXBytes + r * 64 + ((q ^ swz4(r)) << 4);
  }

  // Persistent walk: XCD x (= blockIdx % 8) takes the contiguous id range
  // [x T / 8, (x + 1) T / 8) of a raster that runs down 4 tile rows, then
  // across.
  constexpr int G = 4;
  const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8, slots = gridDim.x / 8;
  const int lo = (int)((int64_t)xcd * tiles / 8), hi = (int)((int64_t)(xcd + 1) * tiles / 8);
  for (int id = lo + slot; id < hi; id += slots) {
    const int group = id / (G * tiles_n);
    const int fm = group * G;
    const int gm = min(G, tiles_m - fm);
    const int in = id - group * G * tiles_n;
    const int tm = fm + in % gm, tn = in / gm;
    const int m0 = tm * BM, n0 = tn * BN;

    unsigned src[kDmaMax];
#pragma unroll
    for (int i = 0; i < kDmaMax; ++i) {
      const int u = i * NW + wave;  // rows 16 u .. 16 u + 15 of [x rows; w rows]
      const int r = u * 16 + lrow;
      if (u < XT) {
        const int row = MODE == 4 ? (r & 63) : m0 + r;
        src[i] = (unsigned)(min(row, M - 1) * K * 2 + ((lpos ^ swz4(r)) << 4));
      } else {
        const int rw = r - BM;
        const int row = MODE == 4 ? (rw & 63) : n0 + rw;
        src[i] = (unsigned)(min(row, N - 1) * K * 2 + ((lpos ^ swz4(rw)) << 4));
      }
    }
    const int rot = ROT == 1 ? (3 * tn + 7 * tm) % U : 0;
    auto issue = [&](int unit) {  // refill of unit `unit` into stage unit % S
      char* base = lds + (unit % S) * kStage;
      int ku = unit + rot;
      if (ku >= U) ku -= U;
#pragma unroll
      for (int i = 0; i < kDmaMax; ++i) {
        const int u = i * NW + wave;
        if (i < kDmaMax - 1 || full)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(u < XT ? xr : wr, (lds_void*)(base + u * 1024), 16, (int)src[i],
                                                   ku * 64, 0, 0);
      }
    };
    // Wait until at most `units` of this wave's refills are outstanding.
    auto wait_units = [&](int units) {
      if (full) {
        if (units >= 2) vm_wait<2 * kDmaMax>();
        else if (units == 1) vm_wait<kDmaMax>();
        else vm_wait<0>();
      } else {
        if (units >= 2) vm_wait<2 * (kDmaMax - 1)>();
        else if (units == 1) vm_wait<kDmaMax - 1>();
        else vm_wait<0>();
      }
    };
    static_assert(S <= 4, "wait_units covers at most two units in flight");
    f32x4 acc[FN][FM];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j) acc[i][j] = f32x4{0, 0, 0, 0};
    i32x4 fx[FM], fw[FN];
#pragma unroll
    for (int j = 0; j < FM; ++j) fx[j] = i32x4{lane, 1, 2, 3};
#pragma unroll
    for (int i = 0; i < FN; ++i) fw[i] = i32x4{lane, 3, 2, 1};

    for (int t = 0; t < S - 1; ++t)
      if (t < U) issue(t);
    wait_units(min(S - 2, U - 1));
    __syncthreads();
    if (!t_loaded) t_loaded = __builtin_amdgcn_s_memrealtime();
    for (int g = 0; g < grp; ++g) bar();  // group g starts g intervals late
    for (int u = 0; u < U; ++u) {
      // Memory interval: fragments of unit u, the refill of unit u + S - 1
      // (its stage was last read before this group's previous compute
      // interval ended), then wait for this wave's share of unit u + 1.
      const char* sb = lds + (u % S) * kStage;
      constexpr bool kReads = MODE != 2 && MODE != 3;
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        if (kReads) fx[j] = *reinterpret_cast<const i32x4*>(sb + xaddr[j]);
        else asm volatile("" : "+v"(fx[j]));
      }
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        if (kReads) fw[i] = *reinterpret_cast<const i32x4*>(sb + waddr[i]);
        else asm volatile("" : "+v"(fw[i]));
      }
      if (MODE != 1 && MODE != 2) {
        if (u + S - 1 < U) issue(u + S - 1);
        wait_units(min(S - 2, U - 2 - u));
      }
      lgkm_wait0();
      bar();
      for (int g = 2; g < NG; ++g) bar();  // the further memory intervals of a rotation
      // Compute interval.
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = mfma16(fw[i], fx[j], acc[i][j]);
      bar();
    }
    t_looped = __builtin_amdgcn_s_memrealtime();
    // Lane l of block (i, j) holds features 4 (l / 16) + e of token l % 16.
    if constexpr (EPI_LDS) {
      for (int g = grp; g < NG - 1; ++g) bar();  // every group leaves the rotation together
      constexpr int LR = BN * 2 + 16;            // padded LDS row bytes
      constexpr int HR = BM / 2;
      static_assert(HR * LR <= S * kStage, "half a tile fits the stages");
      static_assert(WM % 2 == 0, "halves of whole wave rows");
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        __syncthreads();
        if ((wm >= WM / 2) == (h == 1)) {
#pragma unroll
          for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int j = 0; j < FM; ++j) {
              const int r = wm * TM + j * 16 + r16 - h * HR;
              const int c = wn * TN + i * 16 + 4 * q;
              bf16x4 o;
#pragma unroll
              for (int e = 0; e < 4; ++e) o[e] = (__bf16)acc[i][j][e];
              *reinterpret_cast<bf16x4*>(lds + r * LR + c * 2) = o;
            }
        }
        __syncthreads();
        constexpr int CPR = BN / 8;  // 16-byte chunks per row
        for (int idx = threadIdx.x; idx < HR * CPR; idx += NW * 64) {
          const int r = idx / CPR, c = (idx % CPR) * 8;
          const int m = m0 + h * HR + r, n = n0 + c;
          if (m < M && n + 8 <= N)
            *reinterpret_cast<bf16x8*>(y + (int64_t)m * N + n) = *reinterpret_cast<const bf16x8*>(lds + r * LR + c * 2);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) {
          const int m = m0 + wm * TM + j * 16 + r16;
          const int n = n0 + wn * TN + i * 16 + 4 * q;
          if (m < M && n + 4 <= N) {
            bf16x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = (__bf16)acc[i][j][e];
            *reinterpret_cast<bf16x4*>(y + (int64_t)m * N + n) = o;
          }
        }
      for (int g = grp; g < NG - 1; ++g) bar();
    }
    __syncthreads();
  }
  __builtin_amdgcn_s_waitcnt(0);
  const uint64_t t_done = __builtin_amdgcn_s_memrealtime();
  const uint64_t c_done = __builtin_amdgcn_s_memtime();
  if (tl && threadIdx.x == 0) {
    tl[blockIdx.x * 5] = t_entry;
    tl[blockIdx.x * 5 + 1] = t_loaded;
    tl[blockIdx.x * 5 + 2] = t_looped;
    tl[blockIdx.x * 5 + 3] = t_done;
    tl[blockIdx.x * 5 + 4] = c_done - c_entry;
  }
}

__global__ void ref_kernel(const __bf16* x, const __bf16* w, float* y, int M, int N, int K) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x, m = blockIdx.y;
  if (n >= N) return;
  float s = 0;
  for (int k = 0; k < K; ++k) s += (float)x[(int64_t)m * K + k] * (float)w[(int64_t)n * K + k];
  y[(int64_t)m * N + n] = s;
}

#define CK(x)                                                                   \
  do {                                                                          \
    hipError_t e_ = (x);                                                        \
    if (e_ != hipSuccess) {                                                     \
      printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      exit(1);                                                                  \
    }                                                                           \
  } while (0)

template <int BM, int BN, int WM, int WN, int MODE, int S, bool EPI_LDS, int ROT>
void run(int M, int N, int K, bool check) {
  if (K % 32 != 0 || N % 8 != 0 || (int64_t)M * K * 2 >= 0x7ffffff0ll || (int64_t)N * K * 2 >= 0x7ffffff0ll) {
    printf("unsupported shape\n");
    exit(1);
  }
  const size_t nx = (size_t)M * K, nw = (size_t)N * K, ny = (size_t)M * N;
  std::vector<__bf16> hx(nx), hw(nw);
  uint32_t s = 12345;
  auto rnd = [&]() {
    s = s * 1664525u + 1013904223u;
    return ((s >> 8) & 0xffff) / 65536.0f - 0.5f;
  };
  for (auto& v : hx) v = (__bf16)rnd();
  for (auto& v : hw) v = (__bf16)(rnd() * 0.1f);
  __bf16 *dx, *dw, *dy;
  float* dr;
  CK(hipMalloc(&dx, nx * 2));
  CK(hipMalloc(&dw, nw * 2));
  CK(hipMalloc(&dy, ny * 2));
  CK(hipMalloc(&dr, ny * 4));
  CK(hipMemcpy(dx, hx.data(), nx * 2, hipMemcpyHostToDevice));
  CK(hipMemcpy(dw, hw.data(), nw * 2, hipMemcpyHostToDevice));
  const int grid = 256;  // one workgroup per CU, eight XCDs of 32
  auto launch = [&](uint64_t* tl) {
    pp_kernel<BM, BN, WM, WN, MODE, S, EPI_LDS, ROT><<<grid, WM * WN * 64>>>(dx, dw, dy, M, N, K, tl);
  };
  launch(nullptr);
  CK(hipDeviceSynchronize());
  printf("BM %d BN %d waves %dx%d S %d mode %d epi %s rot %d, M %d N %d K %d:", BM, BN, WM, WN, S, MODE,
         EPI_LDS ? "lds" : "direct", ROT, M, N, K);
  if (check) {
    ref_kernel<<<dim3((N + 255) / 256, M), 256>>>(dx, dw, dr, M, N, K);
    CK(hipDeviceSynchronize());
    std::vector<__bf16> hy(ny);
    std::vector<float> hr(ny);
    CK(hipMemcpy(hy.data(), dy, ny * 2, hipMemcpyDeviceToHost));
    CK(hipMemcpy(hr.data(), dr, ny * 4, hipMemcpyDeviceToHost));
    double num = 0, den = 0;
    for (size_t i = 0; i < ny; ++i) {
      const double d = (double)(float)hy[i] - hr[i];
      num += d * d;
      den += (double)hr[i] * hr[i];
    }
    printf(" rel_fro %.2e,", sqrt(num / den));
  }
  hipEvent_t a, b;
  CK(hipEventCreate(&a));
  CK(hipEventCreate(&b));
  for (int i = 0; i < 20; ++i) launch(nullptr);
  const int iters = 100;
  CK(hipEventRecord(a));
  for (int i = 0; i < iters; ++i) launch(nullptr);
  CK(hipEventRecord(b));
  CK(hipEventSynchronize(b));
  float ms;
  CK(hipEventElapsedTime(&ms, a, b));
  const double us = ms * 1000.0 / iters;
  printf(" %.2f us/launch, %.1f TFLOP/s\n", us, 2.0 * M * N * K / us / 1e6);

  uint64_t* tl;
  CK(hipMalloc(&tl, grid * 40));
  std::vector<uint64_t> h(grid * 5);
  launch(tl);
  CK(hipDeviceSynchronize());
  CK(hipMemcpy(h.data(), tl, grid * 40, hipMemcpyDeviceToHost));
  uint64_t first = ~0ull, last_start = 0, last_end = 0;
  double s1 = 0, s2 = 0, s3 = 0, cyc = 0, real = 0;
  for (int g = 0; g < grid; ++g) {
    const uint64_t* t = &h[5 * g];
    first = std::min(first, t[0]);
    last_start = std::max(last_start, t[0]);
    last_end = std::max(last_end, t[3]);
    s1 += (t[1] - t[0]) * 0.01;
    s2 += (t[2] - t[1]) * 0.01;
    s3 += (t[3] - t[2]) * 0.01;
    cyc += (double)t[4];
    real += (t[3] - t[0]) * 0.01;
  }
  printf("    timeline (us): start spread %.2f, prologue %.2f, k-loop %.2f, epilogue %.2f, first start to last end %.2f;"
         " shader clock %.2f GHz\n",
         (last_start - first) * 0.01, s1 / grid, s2 / grid, s3 / grid, (last_end - first) * 0.01, cyc / real / 1e3);
  CK(hipFree(tl));
  CK(hipFree(dx));
  CK(hipFree(dw));
  CK(hipFree(dy));
  CK(hipFree(dr));
}

int main(int argc, char** argv) {
  const char* which = argc > 1 ? argv[1] : "all";
  auto want = [&](const char* s) { return !strcmp(which, "all") || !strcmp(which, s); };
  // ModernBERT-base Wqkv shape (M = 8192 tokens, 768 -> 2304), one round of
  // 256 x 288 tiles on twelve waves (three groups of 64 x 96 wave tiles).
  if (want("modes")) {
    run<256, 288, 4, 3, 0, 4, true, 0>(8192, 2304, 768, true);
    run<256, 288, 4, 3, 1, 4, true, 0>(8192, 2304, 768, false);
    run<256, 288, 4, 3, 2, 4, true, 0>(8192, 2304, 768, false);
    run<256, 288, 4, 3, 3, 4, true, 0>(8192, 2304, 768, false);
    run<256, 288, 4, 3, 4, 4, true, 0>(8192, 2304, 768, false);
  }
  if (want("epilogue")) {
    run<256, 288, 4, 3, 0, 4, false, 0>(8192, 2304, 768, true);
    run<256, 288, 4, 3, 2, 4, false, 0>(8192, 2304, 768, false);
    run<256, 288, 4, 3, 2, 4, true, 0>(8192, 2304, 768, false);
  }
  if (want("rotation")) run<256, 288, 4, 3, 0, 4, true, 1>(8192, 2304, 768, true);
  // 8192^3 on 256 x 256 tiles, eight waves (two groups of 64 x 128 wave tiles).
  if (want("square")) {
    run<256, 256, 4, 2, 0, 4, true, 0>(1024, 1024, 1024, true);
    run<256, 256, 4, 2, 0, 4, true, 0>(8192, 8192, 8192, false);
    run<256, 256, 4, 2, 1, 4, true, 0>(8192, 8192, 8192, false);
    run<256, 256, 4, 2, 2, 4, true, 0>(8192, 8192, 8192, false);
    run<256, 256, 4, 2, 3, 4, true, 0>(8192, 8192, 8192, false);
    run<256, 256, 4, 2, 4, 4, true, 0>(8192, 8192, 8192, false);
  }
  return 0;
}
