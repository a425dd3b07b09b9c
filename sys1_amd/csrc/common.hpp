// Shared device helpers for the gfx950 projection kernels: vector types,
// bf16 conversion, MFMA wrappers and the fused epilogue arithmetic.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sys1hip.h"  // include/ is on the include path

namespace sys1 {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;
typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;

// Epilogue ids used as template arguments (a subset of flag combinations that
// the dispatcher accepts; see epi_id_from_flags in the ABI source).
enum Epi : int {
  kEpiNone = 0,
  kEpiBias = 1,
  kEpiGeglu = 2,
  kEpiSwiglu = 3,
  kEpiResidual = 4,
  kEpiBiasGelu = 5,
  kEpiBiasResidual = 6,
  kEpiRopeQkv = 7,   // Wqkv: RoPE on q and k, q/k/v written as three planes
  // Pre-norm projections (the norm's weight folded into w; per-row mean and
  // reciprocal deviation in `stats`, per-row sums of the folded w in
  // `colsum`): y = epi(r_m (acc - mu_m c_n)) for LayerNorm, epi(r_m acc) for
  // RMSNorm, with epi the base epilogue named.
  kEpiNormLn = 8,
  kEpiNormLnGeglu = 9,
  kEpiNormRms = 10,
  kEpiNormRmsSwiglu = 11,
  // Qwen3.5 DeltaNet in_proj: causal conv (4 taps) + SiLU over the first
  // conv_ch columns, the rest plain; optionally after an RMSNorm.
  kEpiConvSilu = 12,
  kEpiNormRmsConvSilu = 13,
  // Bias, then the tanh-approximate GELU (the Qwen3.5 vision tower's fc1:
  // src/archs/qwen35_vision.rs:166-169, candle's `gelu`).
  kEpiBiasGeluTanh = 14,
  kEpiCount = 15,
};

constexpr int kConvTaps = 4;  // DeltaNet conv kernel size (linear_conv_kernel_dim)
constexpr int kConvHalo = kConvTaps - 1;

enum NormKind : int { kNormNone = 0, kNormLayer = 1, kNormRms = 2 };

__host__ __device__ constexpr int epi_norm(int e) {
  return e == kEpiNormLn || e == kEpiNormLnGeglu                              ? kNormLayer
         : e == kEpiNormRms || e == kEpiNormRmsSwiglu || e == kEpiNormRmsConvSilu ? kNormRms
                                                                                   : kNormNone;
}
// The epilogue applied after the normalisation.
__host__ __device__ constexpr int epi_base(int e) {
  return e == kEpiNormLn || e == kEpiNormRms ? kEpiNone
         : e == kEpiNormLnGeglu              ? kEpiGeglu
         : e == kEpiNormRmsSwiglu            ? kEpiSwiglu
         : e == kEpiNormRmsConvSilu          ? kEpiConvSilu
                                             : e;
}
__host__ __device__ constexpr bool epi_gated(int e) {
  return epi_base(e) == kEpiGeglu || epi_base(e) == kEpiSwiglu;
}

// f32 -> bf16 with round-to-nearest-even (clang lowers this to the gfx950
// hardware conversion), and back.
__device__ __forceinline__ __bf16 to_bf16(float v) { return static_cast<__bf16>(v); }
__device__ __forceinline__ float to_f32(__bf16 v) { return static_cast<float>(v); }
__device__ __forceinline__ float round_bf16(float v) { return to_f32(to_bf16(v)); }

// erfc(x) for x >= 0 with fractional error below 1.2e-7: the Chebyshev fit
// "erfcc" of W. H. Press et al., Numerical Recipes in C, 2nd ed., section
// 6.2: erfc(x) = t exp(-x^2 + P(t)), t = 1 / (1 + x / 2), P of degree 9.
// Branch-free; the reciprocal and exponential are the hardware ones.
__device__ __forceinline__ float erfc_nr(float x) {
  const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, x, 1.0f));
  float p = 0.17087277f;
  p = fmaf(p, t, -0.82215223f);
  p = fmaf(p, t, 1.48851587f);
  p = fmaf(p, t, -1.13520398f);
  p = fmaf(p, t, 0.27886807f);
  p = fmaf(p, t, -0.18628806f);
  p = fmaf(p, t, 0.09678418f);
  p = fmaf(p, t, 0.37409196f);
  p = fmaf(p, t, 1.00002368f);
  return t * __expf(fmaf(p, t, -1.26551223f) - x * x);
}

// Exact (erf) GELU: 0.5 v (1 + erf(v / sqrt 2)), the activation of the
// reference's GeGLU (src/kernels/modernbert.cu:9-14 writes it as v * Phi(v))
// and of candle's gelu_erf, in the reference's f32 sequence: erf is formed
// as 1 - erfc or erfc - 1, then 1 + erf is rounded as the reference rounds
// it.  Over every finite bf16 input this gives the bf16 result of the same
// sequence with a correctly rounded f32 erf.
__device__ __forceinline__ float gelu_erf(float v) {
  const float e = erfc_nr(fabsf(v) * 0.70710678118654752f);
  // erf(v / sqrt 2): 1 - e for v >= 0, e - 1 = -(1 - e) (exactly) below.
  const float erf = __builtin_copysignf(1.0f - e, v);
  return 0.5f * v * (1.0f + erf);
}

// Tanh-approximate GELU: 0.5 v (1 + tanh(y)), y = sqrt(2/pi) (v + 0.044715 v^3),
// written as v / (1 + e^-2y) (the same function; this form keeps full
// relative precision where 1 + tanh(y) is small), with the hardware
// exponential and reciprocal.
__device__ __forceinline__ float gelu_tanh(float v) {
  const float y = 0.7978845608028654f * fmaf(0.044715f * v, v * v, v);
  return v * __builtin_amdgcn_rcpf(1.0f + __expf(-2.0f * y));
}

// SiLU: v / (1 + e^-v) (src/archs/qwen35_text.rs:239), with the hardware
// exponential and reciprocal (the IEEE division costs ~6% of a gated
// projection); its bf16 results match the correctly rounded f32 sequence on
// all but a few of the bf16 inputs, by one ulp.
__device__ __forceinline__ float silu(float v) { return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }

// One output element of the non-gated epilogues from the f32 accumulator.
// Rounding mirrors the unfused reference: projection -> bf16, then each op
// in f32 -> bf16.
template <int EPI>
__device__ __forceinline__ float epi_apply(float acc, float bias, float resid) {
  float v = round_bf16(acc);
  if constexpr (EPI == kEpiBias || EPI == kEpiBiasGelu || EPI == kEpiBiasResidual || EPI == kEpiBiasGeluTanh)
    v = round_bf16(v + bias);
  if constexpr (EPI == kEpiBiasGelu) v = round_bf16(gelu_erf(v));
  if constexpr (EPI == kEpiBiasGeluTanh) v = round_bf16(gelu_tanh(v));
  if constexpr (EPI == kEpiResidual || EPI == kEpiBiasResidual) v = round_bf16(v + resid);
  return v;
}

// The register-side part of the non-gated epilogues (everything before the
// residual add): projection -> bf16, + bias -> bf16, gelu -> bf16.  The
// residual add then runs on the bf16 value: bf16(v + r).
template <int EPI>
__device__ __forceinline__ float epi_pre(float acc, float bias) {
  float v = round_bf16(acc);
  if constexpr (EPI == kEpiBias || EPI == kEpiBiasGelu || EPI == kEpiBiasResidual || EPI == kEpiBiasGeluTanh)
    v = round_bf16(v + bias);
  if constexpr (EPI == kEpiBiasGelu) v = round_bf16(gelu_erf(v));
  if constexpr (EPI == kEpiBiasGeluTanh) v = round_bf16(gelu_tanh(v));
  return v;
}

// One output element of the gated epilogues: gate and up accumulators of the
// same output column.  GeGLU follows src/kernels/modernbert.cu:9-14 (the
// activated gate is rounded to the storage type before the multiply);
// SwiGLU follows candle's silu(gate) * up on bf16 tensors.
template <int EPI>
__device__ __forceinline__ float epi_gate(float g_acc, float u_acc) {
  // both rounded to bf16 by one packed conversion
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t gu = __builtin_convertvector((f32x2_t){g_acc, u_acc}, bf16x2_t);
  const float g = to_f32(gu[0]);
  const float u = to_f32(gu[1]);
  float a;
  if constexpr (EPI == kEpiGeglu)
    a = round_bf16(gelu_erf(g));
  else
    a = round_bf16(silu(g));
  return round_bf16(a * u);
}

template <int EPI>
__host__ __device__ constexpr bool epi_has_bias() {
  return EPI == kEpiBias || EPI == kEpiBiasGelu || EPI == kEpiBiasResidual || EPI == kEpiBiasGeluTanh;
}
template <int EPI>
__host__ __device__ constexpr bool epi_has_resid() {
  return EPI == kEpiResidual || EPI == kEpiBiasResidual;
}

// ---- buffer and LDS-DMA helpers shared by the GEMM kernels.

typedef __attribute__((address_space(3))) void lds_void;

// Raw buffer descriptor over [base, base + 2 GiB): offsets at or past
// kOutOfRange fall outside it and read as zeros.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr unsigned kOutOfRange = 0x80000000u;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, int bytes = 0x7ffffff0) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}
// The same from values the caller knows to be wave-uniform, moved to SGPRs
// explicitly: a descriptor the compiler cannot prove uniform is otherwise
// consumed through a readfirstlane loop around every load.
__device__ __forceinline__ rsrc_t make_rsrc_uniform(const void* base, int bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  return make_rsrc(reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo),
                   __builtin_amdgcn_readfirstlane(bytes));
}

// Asynchronous 16-byte-per-lane copy global -> LDS: lane i's 16 bytes (from
// byte offset `off` of the buffer) land at lds_base + 16 * i; lds_base is
// wave-uniform.
__device__ __forceinline__ void dma16(rsrc_t r, unsigned off, lds_void* lds_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds_base, 16, (int)off, 0, 0, 0);
}
// Cache-policy bits of a gfx950 buffer access: nt (non-temporal: streamed
// through the caches rather than kept).
constexpr int kCachePolicyNt = 2;
template <int POL>
__device__ __forceinline__ void dma16_pol(rsrc_t r, unsigned off, lds_void* lds_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds_base, 16, (int)off, 0, 0, POL);
}

// s_waitcnt vmcnt(N) with the LDS and export counters left unconstrained.
template <int N>
__device__ __forceinline__ void vm_wait() {
  __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15) | ((N >> 4) << 14));
}

// Arguments shared by every GEMM kernel.
struct GemmArgs {
  const __bf16* x;      // [M, K], ld ldx
  const __bf16* w;      // [N, K], ld ldw (packed gate/up layout when gated)
  const __bf16* bias;   // [Nout] or null
  const __bf16* resid;  // [M, Nout] ld ldr or null
  __bf16* y;            // [M, Nout] ld ldy
  float* ws;            // stream-K partials (head/tail slot per workgroup)
  unsigned* counters;   // stream-K arrival counter per (split tile, wave) (zero between calls)
  int64_t ldx, ldw, ldr, ldy;
  int M, N, K, Nout;
  int dp_tiles;         // stream-K kernels: tiles run whole before the stream phase
  int group_m;          // tile rows per raster group of the persistent schedule
  // kEpiRopeQkv: y holds planes q, k, v of [M, H] (H = Nout / 3, ld ldy),
  // `plane` elements apart; head_dim 64; cos/sin [positions, 32] f32;
  // pos[m] is token m's rotary position.
  const float* rope_cos;
  const float* rope_sin;
  const int* pos;
  int rope_rows;        // table rows: positions are clamped into [0, rope_rows)
  int64_t plane;
  // Pre-norm epilogues: stats[2m] = mean (0 for RMSNorm), stats[2m+1] =
  // 1/sqrt(var + eps) of input row m; colsum[n] = sum_k w[n, k] (LayerNorm).
  const float* stats;
  const float* colsum;
  // Conv epilogues: conv_w bf16 [conv_ch, 4] (taps oldest first), pos[m] =
  // token m's position in its sequence.
  const __bf16* conv_w;
  int conv_ch;
  // Weight layout.  0: row-major [N, ldw].  > 0: the blocked layout of
  // sys1hip_pack_blocked_weight with this many 64-wide k-tiles per row
  // block: 32-row x 64-k blocks of 4 KB, row-major inside, ordered
  // [N / 32][w_kt] (rows and K zero-padded), so one k-tile of a 32-row block
  // is 4 KB of contiguous memory.
  int w_kt;
};

constexpr int kBlkRows = 32;                  // rows of a weight block
constexpr int kBlkK = 64;                     // k values of a weight block
constexpr int kBlkBytes = kBlkRows * kBlkK * 2;  // 4 KB

// Map the hardware workgroup id to a logical tile id so that each XCD gets a
// contiguous range of logical tiles.  Workgroups are dispatched round-robin
// over the 8 XCDs (id % 8); the mapping is a bijection for any count.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  constexpr int kXcds = 8;
  const int per = nblocks / kXcds;
  const int rem = nblocks % kXcds;
  const int xcd = bid % kXcds;
  const int idx = bid / kXcds;
  return xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
}

// Store 4 consecutive bf16 of one row: one 8-byte store when all 4 are in
// range and the address is 8-byte aligned, else element by element (odd
// output widths and leading dimensions).
__device__ __forceinline__ bool aligned8(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 7) == 0;
}

__device__ __forceinline__ void store4(__bf16* p, const float v[4], int valid) {
  if (valid >= 4 && aligned8(p)) {
    bf16x4 o;
    o[0] = to_bf16(v[0]);
    o[1] = to_bf16(v[1]);
    o[2] = to_bf16(v[2]);
    o[3] = to_bf16(v[3]);
    *reinterpret_cast<bf16x4*>(p) = o;
  } else {
    for (int j = 0; j < valid && j < 4; ++j) p[j] = to_bf16(v[j]);
  }
}

__device__ __forceinline__ void load4(const __bf16* p, float v[4], int valid) {
  if (valid >= 4 && aligned8(p)) {
    const bf16x4 i = *reinterpret_cast<const bf16x4*>(p);
    v[0] = to_f32(i[0]);
    v[1] = to_f32(i[1]);
    v[2] = to_f32(i[2]);
    v[3] = to_f32(i[3]);
  } else {
    for (int j = 0; j < 4; ++j) v[j] = j < valid ? to_f32(p[j]) : 0.0f;
  }
}

__device__ __forceinline__ bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

// 8 consecutive bf16 of one row: one 16-byte access when all 8 are in range
// and the address is 16-byte aligned, else element by element.
__device__ __forceinline__ void store8(__bf16* p, bf16x8 v, int valid) {
  if (valid >= 8 && aligned16(p)) {
    *reinterpret_cast<bf16x8*>(p) = v;
  } else {
    for (int j = 0; j < valid && j < 8; ++j) p[j] = v[j];
  }
}

__device__ __forceinline__ void load8(const __bf16* p, float v[8], int valid) {
  if (valid >= 8 && aligned16(p)) {
    const bf16x8 i = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = to_f32(i[j]);
  } else {
    for (int j = 0; j < 8; ++j) v[j] = j < valid ? to_f32(p[j]) : 0.0f;
  }
}

// The same 8 values as bf16 (zeros past `valid`).
__device__ __forceinline__ bf16x8 load8_bf16(const __bf16* p, int valid) {
  if (valid >= 8 && aligned16(p)) return *reinterpret_cast<const bf16x8*>(p);
  bf16x8 v;
  for (int j = 0; j < 8; ++j) v[j] = j < valid ? p[j] : __bf16(0.0f);
  return v;
}

}  // namespace sys1
