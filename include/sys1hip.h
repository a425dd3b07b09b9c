/*
 * sys1hip -- C ABI of the MI355X (gfx950) projection-GEMM path.
 *
 * Drop-in for the dense projections that sys1's model code runs through
 * `candle_nn::Linear` (weight [out,in] row-major, y = x.W^T (+ b)):
 *   src/archs/modernbert.rs:1036-1046  linear_no_bias_dtype -> Linear::new(w, None)
 *   src/archs/qwen35_text.rs:174-176   linear -> Linear::new(w, None)
 *   src/models/laya.rs:620-630         linear_dtype -> Linear::new(w, Some(b))
 * and, as fused epilogues, for the elementwise ops that follow them:
 *   src/archs/modernbert.rs:521-533 + src/kernels/modernbert.cu:4-29  (GeGLU)
 *   src/archs/qwen35_text.rs:232-240                                 (SwiGLU)
 *   src/archs/modernbert.rs:883,886; src/archs/qwen35_text.rs:938-939 (residual)
 *   src/models/laya.rs:510-520                                        (bias + gelu_erf)
 *   src/archs/qwen35_vision.rs:163-171                                (bias + tanh GELU)
 *
 * Conventions
 *   - All tensors are device pointers (hipMalloc'd or torch-owned) in bf16,
 *     row-major, leading dimensions in elements.  x is [M,K], w is [N,K],
 *     y is [M,Nout] with Nout = N, or N/2 for the gated epilogues.
 *   - K, ldx and ldw must be multiples of 8 elements and x, w 16-byte
 *     aligned (128-bit loads).  y, residual and bias have no alignment rule
 *     beyond bf16's 2 bytes (aligned runs use 64-bit stores).  M may be 0.
 *   - The call allocates no device memory and does not synchronise: work is
 *     enqueued on the context's stream (default: the context's own stream, or
 *     the one set by sys1hip_set_stream).  The first call of a shape adds
 *     its chosen kernel plan to the context's host-side plan cache (a small
 *     heap allocation; calls of a known shape allocate nothing).
 *   - One context per stream.  Calls on one context must not overlap: the
 *     stream-K workspace and tile counters held by the context are shared
 *     by its calls.
 *   - Return value 0 on success, a negative SYS1HIP_E* code otherwise; the
 *     message is available from sys1hip_last_error (per calling thread).
 *     This mirrors the reference's native-op error path, which bails with a
 *     message on bad layout, dtype or launch size
 *     (src/archs/modernbert.rs:553-572,610).
 */
#ifndef SYS1HIP_H
#define SYS1HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SYS1HIP_API __attribute__((visibility("default")))

#define SYS1HIP_OK 0
#define SYS1HIP_EINVAL (-22)   /* bad shape, null pointer, unsupported epilogue   */
#define SYS1HIP_EALIGN (-14)   /* pointer or leading dimension not 16-byte aligned */
#define SYS1HIP_EDEVICE (-19)  /* no HIP device / HIP runtime error                */
#define SYS1HIP_ERANGE (-34)   /* a size overflows what the kernels index          */

/* Epilogue flags for sys1hip_linear_bf16 (bitwise OR).  Rounding follows the
 * reference's unfused bf16 sequence: the projection is rounded to bf16 first,
 * then each following op computes in f32 and rounds to bf16. */
#define SYS1HIP_EPI_NONE 0
#define SYS1HIP_EPI_BIAS 1     /* y = bf16(bf16(xW^T) + b)            candle Linear bias add */
#define SYS1HIP_EPI_GEGLU 2    /* y = bf16(bf16(gelu_erf(g)) * u)     modernbert.cu:9-14     */
#define SYS1HIP_EPI_SWIGLU 4   /* y = bf16(bf16(silu(g)) * u)         qwen35_text.rs:239     */
#define SYS1HIP_EPI_RESIDUAL 8 /* y = bf16(bf16(...) + r)             modernbert.rs:883,886  */
#define SYS1HIP_EPI_GELU 16    /* y = bf16(gelu_erf(bf16(... + b)))   laya.rs:513-515        */
#define SYS1HIP_EPI_GELU_TANH 64 /* y = bf16(gelu_tanh(bf16(... + b))) qwen35_vision.rs:166-169 */
/* Not an epilogue: the weight argument is in the blocked layout of
 * sys1hip_pack_blocked_weight (ldw is then unused).  Accepted by
 * sys1hip_linear_bf16, sys1hip_linear_bf16_noalloc and
 * sys1hip_norm_linear_bf16. */
#define SYS1HIP_EPI_BLOCKED_W 32

/* Packing granularity of gated weights: rows are interleaved in groups of
 * this many gate rows followed by as many up rows. */
#define SYS1HIP_GATE_GROUP 16

/* Library version (major*10000 + minor*100 + patch). */
SYS1HIP_API int sys1hip_version(void);

/* Create a context on HIP device `device`: selects the device, creates a
 * stream and the stream-K workspace.  Counterpart of src/device.rs:43-65
 * (`device::load()` -> Device::new_cuda(0)). */
SYS1HIP_API int sys1hip_init(int device, void** ctx);

/* Destroy a context (synchronises its stream first). */
SYS1HIP_API int sys1hip_destroy(void* ctx);

/* Enqueue subsequent work on `stream` (a hipStream_t; NULL is HIP's null
 * stream).  Lets a caller share the stream of the framework that owns the
 * buffers (e.g. torch's current stream).  When the stream changes, the new
 * stream is made to wait for the work already enqueued on the old one (an
 * event recorded there), so calls before and after the switch never overlap
 * on the context's shared workspace.  While either stream is being captured
 * into a HIP graph no wait is inserted: ordering a captured graph's replays
 * against eager work on another stream is then the caller's. */
SYS1HIP_API int sys1hip_set_stream(void* ctx, void* stream);

/* Block until the context's stream is idle. */
SYS1HIP_API int sys1hip_sync(void* ctx);

/* Message of the last failing call on this thread ("" if none). */
SYS1HIP_API const char* sys1hip_last_error(void* ctx);

/* The projection: y[M,Nout] = epilogue(x[M,K] . w[N,K]^T).
 * Replaces `Tensor::apply(&Linear)` / `Linear::forward` (candle-nn 0.11.0) at
 * the call sites listed above.
 *   bias      [N] (or [N/2] gated), required iff SYS1HIP_EPI_BIAS
 *   residual  [M,Nout] with leading dim ldr, required iff SYS1HIP_EPI_RESIDUAL
 *   GEGLU / SWIGLU require w in the packed gate/up layout written by
 *   sys1hip_pack_gated_weight, N even and N/2 a multiple of 16. */
SYS1HIP_API int sys1hip_linear_bf16(void* ctx,
                        const uint16_t* x, int64_t ldx,
                        const uint16_t* w, int64_t ldw,
                        const uint16_t* bias,
                        const uint16_t* residual, int64_t ldr,
                        uint16_t* y, int64_t ldy,
                        int64_t M, int64_t N, int64_t K,
                        int32_t epilogue);

/* One projection of a chain (sys1hip_linear_chain_bf16): the arguments of
 * sys1hip_linear_bf16 for it, without bias. */
typedef struct sys1hip_chain_proj {
  const uint16_t* x; int64_t ldx;          /* [M,K] bf16 */
  const uint16_t* w; int64_t ldw;          /* [N,K] bf16, or blocked (SYS1HIP_EPI_BLOCKED_W) */
  const uint16_t* residual; int64_t ldr;   /* [M,Nout], required iff SYS1HIP_EPI_RESIDUAL */
  uint16_t* y; int64_t ldy;                /* [M,Nout] */
  int64_t N, K;
  int32_t epilogue;                        /* NONE, RESIDUAL, GEGLU or SWIGLU (| BLOCKED_W) */
} sys1hip_chain_proj;

/* `count` (1..4) consecutive projections of one layer in one launch: the
 * row-local run of a layer between two attention calls, e.g. ModernBERT's
 * attn.Wo(+residual) -> Wi(+GeGLU) -> mlp.Wo(+residual) -> next layer's Wqkv
 * (src/archs/modernbert.rs:857-887: the `.apply(&linear)` calls at :191,
 * :522, :525-532 and the next layer's :184-187), or Qwen3.5's out_proj ->
 * gate_up(+SwiGLU) -> down(+residual) -> next in_proj
 * (src/archs/qwen35_text.rs:932-940).  Same results, bit for bit, as the
 * same projections issued one sys1hip_linear_bf16 call each.
 * Contract: projection p may read (as x or residual) rows that projections
 * before it wrote, at the same rows only -- a token row of p depends on
 * nothing but that row of earlier projections (attention, which mixes rows,
 * must not sit inside a chain).  Projection p's rows are computed after
 * projection p-1 has finished those rows.
 * K must be a multiple of 64 and at least 192; gated epilogues need N % 32 ==
 * 0; a residual needs Nout and ldr multiples of 8.  M <= 131072.
 * One persistent launch on the context's stream; a dependency wait that
 * does not resolve within the context's limit (sys1hip_set_chain_wait) is
 * abandoned and flagged instead of hanging: check sys1hip_chain_status. */
SYS1HIP_API int sys1hip_linear_chain_bf16(void* ctx, const sys1hip_chain_proj* proj, int32_t count, int64_t M);

/* The chain kernel's tile queue of XCD `xcc` (no device needed; for
 * host-side tests of the schedule, no counterpart in the reference): for
 * `count` projections of N[p] output rows over M tokens, writes (projection,
 * row panel, column tile) of each queue entry, in queue order, into
 * tiles[3 i .. 3 i + 2] (up to `cap` ints) and returns the queue length. */
SYS1HIP_API int sys1hip_chain_queue(int32_t xcc, int64_t M, int32_t count, const int64_t* N, int32_t* tiles,
                        int64_t cap);

/* Synchronise the context's stream and return (in *flags) the error bits
 * that chain launches since the last call set, then clear them: 1 = a
 * dependency wait expired (the results of that launch are not valid),
 * 2 = a row panel's queue was not drained, 4 = a workgroup ran on an
 * unexpected XCD id.  0 means every chain launch completed normally. */
SYS1HIP_API int sys1hip_chain_status(void* ctx, int32_t* flags);

/* Test and tuning knob, no counterpart in the reference: the real time (in
 * microseconds, 1..10^6, default 20000) a chain dependency wait may take
 * before it gives up, and an amount added to every dependency target (> 0
 * makes every wait expire: the error path, exercised without a hang).  Once
 * one wait of a launch has expired, its other waits give up at once. */
SYS1HIP_API int sys1hip_set_chain_wait(void* ctx, int32_t wait_us, int32_t extra);

/* Measurement knob, no counterpart in the reference: a device buffer that
 * later chain launches fill with their timeline (null: off), 64 records of
 * 4 x u64 per workgroup -- {queue index | XCD << 32 | drained << 40, start,
 * stores done, projection}, on the 100 MHz constant clock; it must hold
 * workgroups x 64 x 32 bytes (CUs workgroups), else nothing is recorded. */
SYS1HIP_API int sys1hip_set_chain_trace(void* ctx, void* buffer, int64_t bytes);

/* Re-order a gated weight [2I, K] = [gate rows; up rows] (the reference's
 * chunk(2) split, src/archs/modernbert.rs:531-532, or gate_proj/up_proj
 * stacked, src/archs/qwen35_text.rs:205-231) into groups of 16 gate rows
 * followed by the matching 16 up rows, so that one output tile holds both
 * halves.  Load-time only (counterpart of the weight cast in
 * linear_no_bias_dtype, src/archs/modernbert.rs:1043).  `packed` must not
 * alias `w`.  N = 2I, I a multiple of 16. */
SYS1HIP_API int sys1hip_pack_gated_weight(void* ctx, const uint16_t* w, uint16_t* packed,
                              int64_t N, int64_t K);

/* Kernel choice for a shape (for profiling and reports): returns the kernel
 * id sys1hip_linear_bf16 would launch for these epilogue flags, and writes
 * its name into `name` (up to `cap` bytes including the terminator).  It
 * covers sys1hip_linear_bf16 only: the RoPE, pre-norm and conv entry points
 * restrict or extend the choice (head-aligned tiles, norm epilogues), so
 * their kernel can differ. */
SYS1HIP_API int sys1hip_query_kernel(void* ctx, int64_t M, int64_t N, int64_t K, int32_t epilogue,
                         char* name, int64_t cap);

/* The same choice without a device or context, for planning and host-side
 * tests (no counterpart in the reference): the plan sys1hip_linear_bf16
 * would make on a GPU with `cus` compute units, priced with the shapes'
 * fitted occupancies (a device context uses the runtime's, which agree
 * unless an epilogue variant spills).  Returns the kernel id, writes the
 * workgroup count to *grid (nullable) and the plan's name as
 * sys1hip_query_kernel does. */
SYS1HIP_API int sys1hip_plan_kernel(int32_t cus, int64_t M, int64_t N, int64_t K, int32_t epilogue,
                        int64_t* grid, char* name, int64_t cap);

/* The same with the call's leading dimensions (elements; ldw is ignored for
 * a blocked weight): operands whose rows span 2 GiB or more from their base
 * rule out the skinny kernels, whose buffer offsets are 32-bit.
 * sys1hip_plan_kernel is this with ldx = ldw = K. */
SYS1HIP_API int sys1hip_plan_kernel_strided(int32_t cus, int64_t M, int64_t N, int64_t K, int64_t ldx,
                        int64_t ldw, int32_t epilogue, int64_t* grid, char* name, int64_t cap);

/* Force a kernel id for subsequent calls on this context (-1 = automatic
 * choice).  Used by the tile sweep and by tests that cover every kernel. */
SYS1HIP_API int sys1hip_set_kernel(void* ctx, int32_t kernel_id);

/* Force the persistent grid size (workgroups) for subsequent calls on this
 * context (0 = automatic).  Tile shapes launch min(tiles, this); stream-K
 * shapes divide their (tile, k-tile) iteration space into this many equal
 * ranges, clamped to the iteration count and to what the workspace holds. */
SYS1HIP_API int sys1hip_set_grid(void* ctx, int32_t workgroups);

/* Wqkv with the rotary embedding fused into the epilogue: replaces the
 * projection at src/archs/modernbert.rs:184-187 followed by the fused
 * RoPE + q/k/v split of src/archs/modernbert.rs:112-120 /
 * src/kernels/modernbert.cu:31-74 (rope_qkv).
 *   x [M, K] (packed tokens), w [3H, K] with q | k | v row blocks,
 *   H = heads * head_dim, head_dim = 64 (ModernBERT base and large);
 *   rope_cos, rope_sin: f32 [rope_rows, head_dim/2] device tables
 *   (RotaryEmbedding::new, src/archs/modernbert.rs:67-83), 16-byte aligned;
 *   positions: int32 [M], token m's rotary position within its sequence
 *   (the reference's padded rectangle uses token % length), each in
 *   [0, rope_rows); the kernel clamps values outside that range into it, so
 *   a bad position never reads outside the tables;
 *   qkv: bf16 [3][M][H] output planes q, k, v, each [M, heads, head_dim] --
 *   the packed (varlen) attention layout.
 * Per element: the projection is rounded to bf16, rotated in f32
 * (x0 cos - x1 sin, x0 sin + x1 cos over columns c, c + 32 of a head) and
 * rounded once; v is the rounded projection. */
SYS1HIP_API int sys1hip_linear_rope_qkv_bf16(void* ctx, const uint16_t* x, int64_t ldx,
                                             const uint16_t* w, int64_t ldw, const float* rope_cos,
                                             const float* rope_sin, int64_t rope_rows,
                                             const int32_t* positions, uint16_t* qkv, int64_t M,
                                             int64_t heads, int64_t head_dim, int64_t K);

/* Pre-norm projections: the norm that precedes a projection in the
 * reference's layers, fused into it.
 *   SYS1HIP_NORM_LAYER  bias-free LayerNorm, ModernBERT attn_norm / mlp_norm
 *                       (src/archs/modernbert.rs:1005-1034, used at :865-868,884)
 *   SYS1HIP_NORM_RMS    RMSNorm with alpha = 1 + weight, Qwen3.5
 *                       input_layernorm / post_attention_layernorm
 *                       (src/archs/qwen35_text.rs:178-203, used at :933,939)
 * Replaces `x.apply(&norm)?.apply(&linear)` at those sites: the norm weight
 * is folded into the projection weight once at load (fold_norm_weight), the
 * call computes per-row statistics of x and then the projection of the raw
 * x with the normalisation applied to the accumulators. */
#define SYS1HIP_NORM_LAYER 1
#define SYS1HIP_NORM_RMS 2

/* Load time: w_folded[n,k] = bf16(w[n,k] * a_k), a = gamma (LayerNorm) or
 * 1 + gamma (RMSNorm), gamma f32 [K]; for LayerNorm also colsum[n] = sum_k
 * w_folded[n,k] (f32 [N], 16-byte aligned; may be null for RMSNorm).  For a
 * gated projection pass the packed weight (sys1hip_pack_gated_weight first):
 * the fold is per row, so colsum then follows the packed row order.
 * w_folded may alias w. */
SYS1HIP_API int sys1hip_fold_norm_weight(void* ctx, const uint16_t* w, const float* gamma,
                                         int32_t norm, uint16_t* w_folded, float* colsum,
                                         int64_t N, int64_t K);

/* y[M,Nout] = epilogue(norm(x) . W^T) with W given folded:
 *   LayerNorm: y = epi(r_m (x_m . w_folded_n - mu_m colsum_n)),
 *   RMSNorm:   y = epi(r_m (x_m . w_folded_n)),
 * mu_m, r_m = mean and 1/sqrt(var + eps) of row m of x (f32; RMSNorm:
 * var = mean of squares), computed by the call.  epilogue: SYS1HIP_EPI_NONE,
 * or SYS1HIP_EPI_GEGLU with LayerNorm (ModernBERT Wi), SYS1HIP_EPI_SWIGLU with
 * RMSNorm (Qwen gate/up).  M up to 2^20 rows per call. */
SYS1HIP_API int sys1hip_norm_linear_bf16(void* ctx, const uint16_t* x, int64_t ldx,
                                         const uint16_t* w_folded, int64_t ldw, const float* colsum,
                                         int32_t norm, float eps, uint16_t* y, int64_t ldy,
                                         int64_t M, int64_t N, int64_t K, int32_t epilogue);

/* Qwen3.5 DeltaNet in_proj with its causal conv + SiLU fused: replaces
 * `x.apply(&self.qkv)` followed by causal_conv_silu / cuda_conv_silu
 * (src/archs/qwen35_text.rs:515-526,632-650; CUDA src/kernels/qwen35.cu:3-29),
 * and with norm = SYS1HIP_NORM_RMS also the input RMSNorm before it (:933).
 *   w [N, K]: the in_proj rows, qkv first (conv_ch rows), then z, b, a (or
 *   just the qkv rows, N = conv_ch); folded by sys1hip_fold_norm_weight when
 *   norm is set;
 *   conv_w bf16 [conv_ch, 4]: the conv1d weight [conv_ch, 1, 4], taps
 *   oldest first; conv_ch a multiple of 8; y 16-byte aligned, ldy a
 *   multiple of 8;
 *   positions int32 [M]: token m's position within its sequence (packed
 *   ragged rows; taps before a sequence's first token read zeros, as the
 *   reference's left zero padding does).
 * y[:, :conv_ch] = bf16(silu(c)), c the 4-tap sum over the bf16-rounded
 * projection accumulated in f32 (the reference rounds each product and
 * partial sum to bf16; the two agree to the projection tolerance), and
 * y[:, conv_ch:N] is the rounded projection.  M up to 2^20 rows. */
SYS1HIP_API int sys1hip_linear_conv_silu_bf16(void* ctx, const uint16_t* x, int64_t ldx,
                                              const uint16_t* w, int64_t ldw, int32_t norm, float eps,
                                              const uint16_t* conv_w, int64_t conv_ch,
                                              const int32_t* positions, uint16_t* y, int64_t ldy,
                                              int64_t M, int64_t N, int64_t K);

/* Tuning and test knob, no counterpart in the reference: force how many
 * tiles a stream-K kernel runs whole before its stream phase, for every
 * later call on this context (-1 = automatic; clamped to the tile count).
 * 0 is pure stream-K; the tile count is the plain tile schedule. */
SYS1HIP_API int sys1hip_set_dp_tiles(void* ctx, int32_t tiles);

/* sys1hip_linear_bf16 without a context, allocating nothing.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, checks, arithmetic and
 * kernel choice as sys1hip_linear_bf16, on the current HIP device, enqueued
 * on `stream` (a hipStream_t, NULL = the null stream).  Its stream-K
 * workspace is a static device array of 64 MB of partials plus 65536
 * arrival counters (64.25 MB in all), one per GPU.  Being a file-scope
 * __device__ array, it is allocated when the library's code object loads
 * on a device and held until the process ends, for every user of the
 * library on that device, whether or not it ever calls this entry point:
 * count these 64.25 MB per GPU in the memory budget.  The kernel plan is
 * limited to that workspace, and a call that would need more split tiles
 * than there are counters is refused (SYS1HIP_ERANGE).  The first call on
 * a device looks up the array's address and the kernels' occupancy (and
 * clears the counters when not under capture); it allocates nothing
 * either.  A set-up that fails returns the error and is tried again by the
 * next call.  Every call
 * on one GPU shares that GPU's array: calls that overlap on one GPU (on
 * different streams, or from several threads) race on it and must not.
 * Errors: as sys1hip_linear_bf16, message from sys1hip_last_error(NULL). */
SYS1HIP_API int sys1hip_linear_bf16_noalloc(void* stream,
                        const uint16_t* x, int64_t ldx,
                        const uint16_t* w, int64_t ldw,
                        const uint16_t* bias,
                        const uint16_t* residual, int64_t ldr,
                        uint16_t* y, int64_t ldy,
                        int64_t M, int64_t N, int64_t K,
                        int32_t epilogue);

/* The blocked weight layout, a load-time repacking with no counterpart in
 * the reference (whose weights stay [out,in] row-major): [N, K] bf16 as
 * 32-row x 64-column blocks of 4 KB, row-major inside a block, blocks
 * ordered by row block then k block, rows and K zero-padded.  One k-step of
 * 32 weight rows is then 4 KB of contiguous memory instead of 32 pieces of
 * 128 bytes, which is what the weight-streaming (small-M) kernels read.
 * Packs w [N, ldw] (row-major; a gated weight after
 * sys1hip_pack_gated_weight) into `packed`, which holds
 * sys1hip_blocked_weight_bytes(N, K) bytes.  Returns that size, or -1 for a
 * bad shape. */
SYS1HIP_API int64_t sys1hip_blocked_weight_bytes(int64_t N, int64_t K);
SYS1HIP_API int sys1hip_pack_blocked_weight(void* ctx, const uint16_t* w, int64_t ldw, uint16_t* packed,
                                            int64_t N, int64_t K);

/* Number of kernel ids and the name of one id (for sweeps). */
SYS1HIP_API int sys1hip_kernel_count(void);
SYS1HIP_API const char* sys1hip_kernel_name(int32_t kernel_id);

#ifdef __cplusplus
}
#endif

#endif /* SYS1HIP_H */
