/*
 * CPU oracle for the projection hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C, the arithmetic that sys1's projection call
 * sites perform on the CPU backend.  It is the checker for the HIP kernels and
 * the CPU baseline timed by bench.py; nothing in the shipped library links it.
 *
 * The reference itself keeps the GEMM in third-party crates that are not under
 * the reference tree (candle-nn 0.11.0 `Linear::forward`, candle-core 0.11.0,
 * `gemm` 0.19.0; Cargo.lock:419-421,488-490,1474-1476).  What is restated is
 * their published contract: weight [out,in] row-major, y = x.W^T (+ b), f32
 * arithmetic on the CPU path.  Call sites that fix this contract:
 *   src/archs/modernbert.rs:1036-1046  (linear_no_bias_dtype, weight [out,in])
 *   src/archs/qwen35_text.rs:174-176   (linear, no bias)
 *   src/models/laya.rs:620-630         (linear_dtype, with bias)
 *
 * Every function below carries the reference lines it follows.  Pinning of each
 * function (which test checks it against what) is listed in tests/test_oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

#define ORC_EXPORT __attribute__((visibility("default")))

ORC_EXPORT float orc_round_bf16(float v);

/* ---------------------------------------------------------------- GEMM ---- */

/* y[M,N] = x[M,K] . w[N,K]^T (+ bias[N]), f32 accumulation.
 * Restates candle_nn::Linear::forward (a9); call sites
 * src/archs/modernbert.rs:184-187,191,522,525 and src/archs/qwen35_text.rs:232-240.
 * Blocked over (rows, output features, k) with a 4x4 register block and
 * parallel over output tiles with OpenMP, so that it also serves as the timed
 * CPU baseline.  Summation order within one output: k in blocks of KB, inside
 * a block 8 interleaved partial sums combined pairwise, blocks added in order. */
#define MB 64
#define NB 64
#define KB 256
typedef float f8 __attribute__((vector_size(32)));

static inline float hsum8(f8 v) {
    return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
}

ORC_EXPORT void orc_linear_f32(const float* x, int64_t ldx, const float* w, int64_t ldw,
                               const float* bias, float* y, int64_t ldy,
                               int64_t M, int64_t N, int64_t K) {
    const int64_t mt = (M + MB - 1) / MB, nt = (N + NB - 1) / NB;
    #pragma omp parallel for schedule(dynamic, 1)
    for (int64_t t = 0; t < mt * nt; ++t) {
        const int64_t m0 = (t / nt) * MB, n0 = (t % nt) * NB;
        const int64_t m1 = m0 + MB < M ? m0 + MB : M;
        const int64_t n1 = n0 + NB < N ? n0 + NB : N;
        float acc[MB][NB];
        memset(acc, 0, sizeof(acc));
        for (int64_t k0 = 0; k0 < K; k0 += KB) {
            const int64_t k1 = k0 + KB < K ? k0 + KB : K;
            const int64_t kv = k0 + ((k1 - k0) / 8) * 8;
            /* 4x4 register block of 8-wide partial sums over k. */
            for (int64_t m = m0; m < m1; m += 4) {
                for (int64_t n = n0; n < n1; n += 4) {
                    const float* xr[4];
                    const float* wr[4];
                    for (int i = 0; i < 4; ++i) xr[i] = x + (m + i < m1 ? m + i : m) * ldx;
                    for (int j = 0; j < 4; ++j) wr[j] = w + (n + j < n1 ? n + j : n) * ldw;
                    f8 s[4][4];
                    memset(s, 0, sizeof(s));
                    for (int64_t k = k0; k < kv; k += 8) {
                        f8 a[4], b[4];
                        for (int i = 0; i < 4; ++i) memcpy(&a[i], xr[i] + k, 32);
                        for (int j = 0; j < 4; ++j) memcpy(&b[j], wr[j] + k, 32);
                        for (int i = 0; i < 4; ++i)
                            for (int j = 0; j < 4; ++j) s[i][j] += a[i] * b[j];
                    }
                    for (int i = 0; i < 4 && m + i < m1; ++i)
                        for (int j = 0; j < 4 && n + j < n1; ++j) {
                            float r = hsum8(s[i][j]);
                            for (int64_t k = kv; k < k1; ++k) r += xr[i][k] * wr[j][k];
                            acc[m + i - m0][n + j - n0] += r;
                        }
                }
            }
        }
        for (int64_t m = m0; m < m1; ++m)
            for (int64_t n = n0; n < n1; ++n)
                y[m * ldy + n] = acc[m - m0][n - n0] + (bias ? bias[n] : 0.0f);
    }
}

/* Same contract, accumulated in double and returned in double: the
 * high-precision reference the f32 path and the GPU path are both measured
 * against in the golden checks. */
ORC_EXPORT void orc_linear_f64(const float* x, int64_t ldx, const float* w, int64_t ldw,
                               const float* bias, double* y, int64_t ldy,
                               int64_t M, int64_t N, int64_t K) {
    #pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t n = 0; n < N; ++n) {
            double s = 0.0;
            for (int64_t k = 0; k < K; ++k) s += (double)x[m * ldx + k] * (double)w[n * ldw + k];
            y[m * ldy + n] = s + (bias ? (double)bias[n] : 0.0);
        }
    }
}

/* ------------------------------------------------------- activations ---- */

/* gelu_erf(v) = 0.5 v (1 + erf(v / sqrt 2)), the exact (erf) GELU that candle's
 * `gelu_erf` computes and that the CUDA GeGLU kernel expresses as v * Phi(v)
 * (src/kernels/modernbert.cu:9-14).  Evaluated in double, returned as f32. */
ORC_EXPORT float orc_gelu_erf(float v) {
    const double d = (double)v;
    return (float)(0.5 * d * (1.0 + erf(d * 0.70710678118654752440)));
}

/* gelu_tanh(v) = 0.5 v (1 + tanh(y)), y = sqrt(2/pi) (v + 0.044715 v^3), the
 * tanh-approximate GELU that candle's `gelu` computes (the Qwen3.5 vision
 * tower's mlp: src/archs/qwen35_vision.rs:166-169).  Evaluated in double as
 * v / (1 + e^-2y), the same function without the cancellation of 1 + tanh(y)
 * far left (at v = -7, 1 + tanh(y) ~ 1e-14 keeps only two digits in double),
 * returned as f32. */
ORC_EXPORT float orc_gelu_tanh(float v) {
    const double d = (double)v;
    const double y = 0.79788456080286535588 * (d + 0.044715 * d * d * d);
    return (float)(d / (1.0 + exp(-2.0 * y)));
}

/* silu(v) = v / (1 + exp(-v)) (candle `silu`, used at src/archs/qwen35_text.rs:239). */
ORC_EXPORT float orc_silu(float v) {
    const double d = (double)v;
    return (float)(d / (1.0 + exp(-d)));
}

/* GeGLU split of the Wi output: in[M, 2I] -> out[M, I],
 * out = gelu_erf(in[:, :I]) * in[:, I:]   (src/archs/modernbert.rs:531-532;
 * first chunk is the gate, second the linear half). */
ORC_EXPORT void orc_geglu(const float* in, int64_t ldin, float* out, int64_t ldout,
                          int64_t M, int64_t I) {
    #pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m)
        for (int64_t j = 0; j < I; ++j)
            out[m * ldout + j] = orc_gelu_erf(in[m * ldin + j]) * in[m * ldin + I + j];
}

/* SwiGLU: out = silu(gate) * up  (src/archs/qwen35_text.rs:232-240). */
ORC_EXPORT void orc_swiglu(const float* gate, int64_t ldg, const float* up, int64_t ldu,
                           float* out, int64_t ldout, int64_t M, int64_t I) {
    #pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m)
        for (int64_t j = 0; j < I; ++j)
            out[m * ldout + j] = orc_silu(gate[m * ldg + j]) * up[m * ldu + j];
}

/* LayerNorm with weight and bias over the last dim, eps given
 * (candle_nn::layer_norm; Laya scorer norm, src/models/laya.rs:258).
 * Mean and variance accumulated in double. */
ORC_EXPORT void orc_layer_norm(const float* x, int64_t ldx, const float* g, const float* b,
                               float eps, float* y, int64_t ldy, int64_t M, int64_t H) {
    for (int64_t m = 0; m < M; ++m) {
        double mean = 0.0, var = 0.0;
        for (int64_t h = 0; h < H; ++h) mean += x[m * ldx + h];
        mean /= (double)H;
        for (int64_t h = 0; h < H; ++h) {
            const double d = x[m * ldx + h] - mean;
            var += d * d;
        }
        var /= (double)H;
        const double inv = 1.0 / sqrt(var + (double)eps);
        for (int64_t h = 0; h < H; ++h)
            y[m * ldy + h] = (float)((x[m * ldx + h] - mean) * inv) * g[h] + (b ? b[h] : 0.0f);
    }
}

/* RMSNorm with alpha = 1 + w (src/archs/qwen35_text.rs:178-203): in f32,
 * variance = mean(x^2), scale = 1 / sqrt(variance + eps), y = x * scale *
 * alpha.  Mean of squares accumulated in double. */
ORC_EXPORT void orc_rms_norm(const float* x, int64_t ldx, const float* w, float eps, float* y,
                             int64_t ldy, int64_t M, int64_t H) {
    for (int64_t m = 0; m < M; ++m) {
        double ss = 0.0;
        for (int64_t h = 0; h < H; ++h) ss += (double)x[m * ldx + h] * x[m * ldx + h];
        const float var = (float)(ss / (double)H);
        const float scale = 1.0f / sqrtf(var + eps);
        for (int64_t h = 0; h < H; ++h) y[m * ldy + h] = x[m * ldx + h] * scale * (1.0f + w[h]);
    }
}

/* Qwen3.5 DeltaNet causal depthwise conv + SiLU over packed ragged rows
 * (src/archs/qwen35_text.rs:632-650 causal_conv_silu; the CUDA kernel
 * src/kernels/qwen35.cu:3-29 computes the same): for token m at position
 * pos[m] of its sequence and channel c,
 *   v = sum over tap = 0..kernel-1 of p[m + tap - kernel + 1, c] * w[c, tap],
 * taps before the sequence start (pos[m] + tap - kernel + 1 < 0) reading the
 * zero padding; out = v / (1 + e^-v).  bf16 != 0 applies the reference's bf16
 * arithmetic: every product and every partial sum rounded to bf16, the
 * result rounded once more after the SiLU. */
ORC_EXPORT void orc_conv_silu(const float* p, int64_t ldp, const float* w, const int32_t* pos,
                              int64_t M, int64_t C, int64_t kernel, int bf16, float* out,
                              int64_t ldo) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t c = 0; c < C; ++c) {
            float v = 0.0f;
            for (int64_t tap = 0; tap < kernel; ++tap) {
                const int64_t back = kernel - 1 - tap;
                if (pos[m] < back) continue;
                float prod = p[(m - back) * ldp + c] * w[c * kernel + tap];
                if (bf16) prod = orc_round_bf16(prod);
                v = v + prod;
                if (bf16) v = orc_round_bf16(v);
            }
            float y = v / (1.0f + expf(-v));
            out[m * ldo + c] = bf16 ? orc_round_bf16(y) : y;
        }
}

/* Argmax with ties broken towards the lowest index (src/models/laya.rs:909-916:
 * max_by with total_cmp, then reversed index order). */
ORC_EXPORT int64_t orc_argmax(const float* v, int64_t n) {
    if (n <= 0) return 0;
    int64_t best = 0;
    for (int64_t i = 1; i < n; ++i)
        if (v[i] > v[best]) best = i;
    return best;
}

/* ----------------------------------------------------- bf16 rounding ---- */

/* Round-to-nearest-even f32 -> bf16 -> f32 (what `to_dtype(BF16)` does to a
 * finite value).  NaN stays NaN. */
ORC_EXPORT float orc_round_bf16(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return v;
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    float r;
    memcpy(&r, &u, 4);
    return r;
}

ORC_EXPORT void orc_round_bf16_array(float* v, int64_t n) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) v[i] = orc_round_bf16(v[i]);
}

/* ---------------------------------------------------- seeded inputs ---- */

/* SplitMix64 (Steele, Lea & Flood 2014): state += golden gamma, then the
 * variant-13 finaliser.  Element i of a stream depends only on (seed, i), so a
 * stream can be generated in parallel and reproduced anywhere. */
static inline uint64_t splitmix64_at(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Uniform in (0, 1]: top 53 bits, offset by one ulp so log() is finite. */
static inline double u01(uint64_t r) { return ((double)(r >> 11) + 1.0) * (1.0 / 9007199254740992.0); }

/* out[i] ~ N(0, std^2) by Box-Muller on the pair (2*(i/2), 2*(i/2)+1) of the
 * SplitMix64 stream: even i takes the cosine branch, odd i the sine branch. */
ORC_EXPORT void orc_fill_normal(float* out, int64_t n, uint64_t seed, float stddev) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const uint64_t p = (uint64_t)(i / 2) * 2;
        const double u1 = u01(splitmix64_at(seed, p));
        const double u2 = u01(splitmix64_at(seed, p + 1));
        const double r = sqrt(-2.0 * log(u1));
        const double t = 6.283185307179586476925 * u2;
        out[i] = (float)((double)stddev * r * ((i & 1) ? sin(t) : cos(t)));
    }
}

/* Ragged packing of sequence lengths: draw L ~ U[lo, hi] (integers, inclusive)
 * from the SplitMix64 stream until the next length would exceed `budget`
 * tokens.  With `exact` set, the last sequence is truncated so the total is
 * exactly `budget` (the prefill configs).  Returns the number of sequences and
 * writes them to `lengths` (at most `cap`). */
ORC_EXPORT int64_t orc_pack_ragged(uint64_t seed, int64_t lo, int64_t hi, int64_t budget,
                                   int exact, int64_t* lengths, int64_t cap) {
    int64_t total = 0, count = 0;
    const uint64_t span = (uint64_t)(hi - lo + 1);
    for (uint64_t i = 0; count < cap; ++i) {
        const int64_t len = lo + (int64_t)(splitmix64_at(seed, i) % span);
        if (total + len > budget) {
            if (exact && total < budget) lengths[count++] = budget - total, total = budget;
            break;
        }
        lengths[count++] = len;
        total += len;
        if (total == budget) break;
    }
    return count;
}

/* Elementwise array forms of the two activations, for the checks. */
ORC_EXPORT void orc_gelu_erf_array(const float* in, float* out, int64_t n) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = orc_gelu_erf(in[i]);
}

ORC_EXPORT void orc_gelu_tanh_array(const float* in, float* out, int64_t n) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = orc_gelu_tanh(in[i]);
}

ORC_EXPORT void orc_silu_array(const float* in, float* out, int64_t n) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = orc_silu(in[i]);
}

/* ---------------------------------------------------------------- RoPE ---- */

/* Rotary tables of ModernBERT's RotaryEmbedding::new
 * (src/archs/modernbert.rs:67-83): dim = hidden / heads, inv_freq[i] =
 * 1 / theta^(2i / dim) for i < dim/2 (the f64 power rounded to f32),
 * frequencies = positions (f32) x inv_freq (an f32 outer product),
 * cos/sin [positions, dim/2] in f32. */
ORC_EXPORT void orc_rope_tables(double theta, int64_t dim, int64_t positions, float* cos_out,
                                float* sin_out) {
  const int64_t half = dim / 2;
  for (int64_t p = 0; p < positions; ++p)
    for (int64_t i = 0; i < half; ++i) {
      const float inv = 1.0f / (float)pow(theta, (double)(2 * i) / (double)dim);
      const float f = (float)p * inv;
      cos_out[p * half + i] = cosf(f);
      sin_out[p * half + i] = sinf(f);
    }
}

/* Fused RoPE + q/k/v split of src/kernels/modernbert.cu:31-74 (rope_qkv),
 * as the Wqkv epilogue sees it on packed tokens.  qkv [M, 3*heads*dim]
 * holds q | k | v blocks; for token m (rotary position pos[m]), head h and
 * column c < dim/2, with x0 = q[c], x1 = q[c + dim/2]:
 *   out_q[c]          = x0 * cos - x1 * sin
 *   out_q[c + dim/2]  = x0 * sin + x1 * cos
 * the same for k, and v copied.  Output planes out[3][M][heads*dim].  The
 * reference indexes positions as token % length on its padded rectangle;
 * packed tokens carry their position within their sequence instead. */
ORC_EXPORT void orc_rope_qkv(const float* qkv, int64_t ldqkv, const float* cos_t,
                             const float* sin_t, const int32_t* pos, int64_t M, int64_t heads,
                             int64_t dim, float* out) {
  const int64_t half = dim / 2, H = heads * dim;
  for (int64_t m = 0; m < M; ++m) {
    const float* row = qkv + m * ldqkv;
    const float* c = cos_t + (int64_t)pos[m] * half;
    const float* s = sin_t + (int64_t)pos[m] * half;
    for (int64_t h = 0; h < heads; ++h)
      for (int64_t j = 0; j < half; ++j) {
        for (int plane = 0; plane < 2; ++plane) {
          const float x0 = row[plane * H + h * dim + j], x1 = row[plane * H + h * dim + j + half];
          float* o = out + plane * M * H + m * H + h * dim;
          o[j] = x0 * c[j] - x1 * s[j];
          o[j + half] = x0 * s[j] + x1 * c[j];
        }
        float* ov = out + 2 * M * H + m * H + h * dim;
        ov[j] = row[2 * H + h * dim + j];
        ov[j + half] = row[2 * H + h * dim + j + half];
      }
  }
}
