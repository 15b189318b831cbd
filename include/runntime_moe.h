/* runntime_moe.h — C ABI of the MI355X int8 mixture-of-experts layer.
 *
 * The drop-in boundary for ruNNtime's `runntime/core` MoE ops. Every entry
 * point replaces one reference interface (paths relative to
 * packages/runntime/ in software-mansion/runntime):
 *
 *   moe_topk         topk(x, k)                    src/core/graph/ops/reduce.ts:93-100,
 *                                                  kernel src/core/kernels/reduce/topkSelect.ts:21-92
 *   moe_router_topk  topk(gate.forward(xn), k)     src/zoo/privacy-filter/moeMlp.ts:83 (router
 *                                                  Linear, src/core/nn/layers.ts:252-263, fused with topk)
 *   moe_up           moeUp(x, route, glu, lin, {bits, groupSize})
 *                                                  src/core/graph/ops/matmul.ts:220-244,
 *                                                  kernel src/core/kernels/matmul/moeQuantW.ts:122-175
 *   moe_down         moeDown(act, route, out, residual, {bits, groupSize})
 *                                                  src/core/graph/ops/matmul.ts:246-272,
 *                                                  kernel src/core/kernels/matmul/moeQuantW.ts:188-237
 *   moe_layer        the quantized branch of EagerMoeMlp.forward after rmsNorm:
 *                    topk(router) → moeUp → moeDown  src/zoo/privacy-filter/moeMlp.ts:82-121
 *   moe_rmsnorm      rmsNorm(x, weight, eps, {group, residual, scale})
 *                                                  src/core/graph/ops/reduce.ts:61-92,
 *                                                  kernel src/core/kernels/reduce/rmsNorm.ts
 *   moe_block        the quantized EagerMoeMlp.forward whole: rmsNorm(x) →
 *                    topk(router) → moeUp → moeDown(+x)  src/zoo/privacy-filter/moeMlp.ts:79-121
 *   moe_matmul_gather matmulGather(a, w, expertIdx, {bias})
 *                                                  src/core/graph/ops/matmul.ts:180-210,
 *                                                  kernel src/core/kernels/matmul/matmulGather.ts
 *   moe_block_float  EagerMoeMlp.forward, float weights  src/zoo/privacy-filter/moeMlp.ts:79-100
 *   moe_viterbi_decode  ViterbiDecoder.decode (host code, no GPU)
 *                                                  src/zoo/privacy-filter/viterbi.ts:85-148
 *   moe_linear       Linear.forward(x, {addend}) with a float (or load-time dequantized)
 *                    weight [in, out]             src/core/nn/layers.ts:166-263,
 *                                                  src/core/graph/compose.ts:45-53
 *   moe_attention    the privacy filter's attention core, rope(q), rope(k), sdpa over one
 *                    qkv tensor (src/zoo/privacy-filter/attnBlock.ts:39-55); no single
 *                    reference op: the three calls fused into one kernel
 *   moe_rope         rope(x, cos, sin, {headDim, srcStart, width})
 *                                                  src/core/graph/ops/attention.ts:220-262,
 *                                                  kernel src/core/kernels/attention/rope.ts
 *   moe_sdpa         sdpa(q, k, v, {qHeads, kvHeads, headDim, windowLeft, windowRight,
 *                    qPosOffset, sinks, segments, keyBias}) and sdpaPacked (row strides)
 *                                                  src/core/graph/ops/attention.ts:28-214,
 *                                                  kernels src/core/kernels/attention/attn*.ts
 *   moe_weights_upload / _view / _dispose / _release
 *                    a QuantExpertWeight's buffers uploaded and owned by the
 *                    library (Parameter, src/core/nn/module.ts:20-65)
 *   moe_ctx_* / moe_sync / moe_last_error
 *                    the executor contract the ops run under: one queue per
 *                    context, errors as codes (src/core/graph/evalCore.ts:14-31,
 *                    src/core/error.ts:3-50)
 *
 * Conventions
 *   - All tensor pointers are DEVICE pointers (HBM), plain and unowned. The
 *     caller keeps them alive until the work is done (moe_sync, or an event
 *     on the stream given to moe_ctx_create).
 *   - Layouts are the reference's (src/core/graph/ops/matmul.ts:212-218):
 *       route    f32 [T, 2k]: k expert ids stored as exact floats, then k
 *                gate weights (topkSelect.ts:13-18, :148-156)
 *       w        quantW u32 words of the logical [E·K, N] int8/int4 weight:
 *                16-value tiles per (expert, 4-column unit, 4-row chunk),
 *                column-major in the tile (src/core/kernels/quantCommon.ts:8-15)
 *       scales   f32 [E·K/groupSize, N]
 *       bias     f32 [E, N] (may be NULL: zero)
 *       act      f32 [T·k, N], row t·k + s
 *   - The reference compiles in k = 4 (moeQuantW.ts:28); here k is a
 *     parameter, 1 ≤ k ≤ 16, and k = 4 is the reference's case.
 *   - Every call is asynchronous on the context's stream. Return value: 0 on
 *     success, else an moe_status code with a message in moe_last_error().
 */
#ifndef RUNNTIME_MOE_H
#define RUNNTIME_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef MOE_API
#define MOE_API __attribute__((visibility("default")))
#endif

/* The reference's RunntimeError codes that this layer can raise
 * (src/core/error.ts:3-21). */
typedef enum moe_status {
  MOE_OK = 0,
  MOE_INVALID_ARGUMENT = 1, /* 'INVALID_ARGUMENT' */
  MOE_EXECUTION_FAILED = 2, /* 'EXECUTION_FAILED' */
  MOE_NOT_INITIALIZED = 3,  /* 'NOT_INITIALIZED'  */
  MOE_RESOURCE_DISPOSED = 4 /* 'RESOURCE_DISPOSED' */
} moe_status;

/* Element type of a float input (the reference's 'f32' | 'f16' dtypes,
 * src/core/graph/value.ts). */
typedef enum moe_dtype { MOE_F32 = 0, MOE_F16 = 1 } moe_dtype;

typedef struct moe_ctx moe_ctx;

/* One routed layer's weights for all E experts — the reference's
 * `interface QuantExpertWeight { w; scales; bias }`
 * (src/core/graph/ops/matmul.ts:212-218). */
typedef struct moe_expert_weight {
  const uint32_t *w;    /* quantW words, E·K·N·bits/32 of them */
  const float *scales;  /* [E·K/groupSize, N] */
  const float *bias;    /* [E, N] or NULL */
} moe_expert_weight;

/* Library version, for the binding to check it loaded what it expects. */
MOE_API int moe_version(void);

/* Message of the last failed call on this thread ("" if none). */
MOE_API const char *moe_last_error(void);

/* The device's null (legacy default) stream, as a `stream` argument: the
 * stream a caller with no stream of its own enqueues on (HIP's stream 0,
 * torch's default stream). Work on it is ordered with the caller's; NULL
 * instead selects the context's own non-blocking stream, which is not. */
#define MOE_NULL_STREAM ((void *)1)
/* A context owns one HIP stream (or borrows `stream`, a hipStream_t, when it
 * is not NULL; MOE_NULL_STREAM for the null stream) and the device workspace
 * the layer needs between kernels.
 * Replaces initRunntime(root)/gpuExecutor(root) (src/core/gpu/eval.ts:80-100). */
MOE_API int moe_ctx_create(int device, void *stream, moe_ctx **out);
/* Switch the stream later calls enqueue on (NULL: the context's own;
 * MOE_NULL_STREAM: the null stream). */
MOE_API int moe_ctx_set_stream(moe_ctx *ctx, void *stream);
/* Grow the workspace now for layers up to these sizes, so later calls with
 * no larger shapes allocate nothing. */
MOE_API int moe_ctx_reserve(moe_ctx *ctx, int T, int d, int I, int E, int k);
/* As moe_ctx_reserve, for moe_layer_batched with up to `calls` calls. */
MOE_API int moe_ctx_reserve_batched(moe_ctx *ctx, int calls, int T, int d, int I, int E, int k);
/* Pin (pin = 1) or unpin (pin = 0) the context's workspace: while pinned at
 * least once, a call that needs a larger workspace fails with
 * EXECUTION_FAILED instead of reallocating it, so graphs captured over the
 * workspace keep a valid address. Pins nest; unpinning an unpinned context is
 * INVALID_ARGUMENT. A call made while its stream is capturing never grows
 * the workspace either (reserve before capture). No reference counterpart:
 * the reference's BufferPool (src/core/gpu/bufferPool.ts:1-25) hands out
 * buffers per dispatch and has no captured graphs. */
MOE_API int moe_ctx_pin_workspace(moe_ctx *ctx, int pin);
MOE_API int moe_ctx_destroy(moe_ctx *ctx);
/* Wait for the context's stream; reports a device fault as EXECUTION_FAILED. */
MOE_API int moe_sync(moe_ctx *ctx);

/* topk(x, k): x [T, E] logits (f32 or f16) → route f32 [T, 2k]. Descending,
 * lowest id on ties, softmax over the k picked logits; the reference's
 * −3.4e38 start value is kept (a logit at or below it never enters). */
MOE_API int moe_topk(moe_ctx *ctx, const void *logits, moe_dtype dtype, int T, int E, int k,
             float *route);

/* Router + topk fused: logits = x·W + b with W f32 [d, E] (the reference's
 * Linear weight after its load-time transpose), summed in this library's
 * canonical f32 order (64-wide fma chunks folded left to right, then + b),
 * then topk as moe_topk. x is f32 or f16 [T, d]; b may be NULL. */
MOE_API int moe_router_topk(moe_ctx *ctx, const void *x, moe_dtype x_dtype, const float *w_router,
                    const float *b_router, int T, int d, int E, int k, float *route);

/* moeUp: act[t·k + s] = clampedSwiglu(x[t]·glu[e] + glu.bias[e],
 * x[t]·lin[e] + lin.bias[e]), e = route[t, s]. x [T, K] (f32, or f16 as an
 * extension), act f32 [T·k, N]. The two biases are passed apart (the
 * reference concatenates them per forward, ops/matmul.ts:240). */
MOE_API int moe_up(moe_ctx *ctx, const void *x, moe_dtype x_dtype, const float *route,
           const moe_expert_weight *glu, const moe_expert_weight *lin, int T, int K, int N,
           int E, int k, int bits, int group_size, float *act);

/* moeDown: out[t] = residual[t] + Σ_s gate_s·(act[t·k + s]·w[e_s] + bias[e_s]).
 * act f32 [T·k, K], residual f32 [T, N] or NULL, out f32 [T, N]. */
MOE_API int moe_down(moe_ctx *ctx, const float *act, const float *route, const moe_expert_weight *down,
             const float *residual, int T, int K, int N, int E, int k, int bits,
             int group_size, float *out);

/* The whole routed layer in one call: router+topk → dispatch → grouped
 * gate/up+SwiGLU → grouped down → weighted combine + residual.
 * x [T, d] f32/f16; router W f32 [d, E], b [E] or NULL; glu/lin K = d,
 * N = I; down K = I, N = d; residual f32 [T, d] or NULL; route_out f32
 * [T, 2k] or NULL; out f32 [T, d]. group_size_up divides d, group_size_down
 * divides I (d and I themselves for one scale per output channel). */
MOE_API int moe_layer(moe_ctx *ctx, const void *x, moe_dtype x_dtype, const float *w_router,
              const float *b_router, const moe_expert_weight *glu, const moe_expert_weight *lin,
              const moe_expert_weight *down, const float *residual, int T, int d, int I, int E,
              int k, int bits, int group_size_up, int group_size_down, float *route_out,
              float *out);

/* moe_layer with no allocation: the same computation (bit for bit) on the
 * same arguments, for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, hosts that forbid hipMalloc). No
 * reference counterpart. The workspace is a static device array of
 * MOE_NOALLOC_SCRATCH_BYTES per GPU, owned by the library until the process
 * ends, instead of the context's growable one; the call allocates nothing
 * and creates no timing events. A shape whose workspace exceeds it is
 * INVALID_ARGUMENT with the size it needs (decode-sized calls fit: T·k of a
 * few hundred rows). Every call on a GPU shares that GPU's array. The
 * library records which context and stream used it last: a call from
 * another context or stream while that stream still has work queued is
 * INVALID_ARGUMENT (synchronise the other stream first). What the record
 * cannot see still races: work captured into a graph on another stream and
 * replayed later, and calls from two host threads at once. */
#define MOE_NOALLOC_SCRATCH_BYTES (16u << 20)
MOE_API int moe_layer_noalloc(moe_ctx *ctx, const void *x, moe_dtype x_dtype,
                              const float *w_router, const float *b_router,
                              const moe_expert_weight *glu, const moe_expert_weight *lin,
                              const moe_expert_weight *down, const float *residual, int T, int d,
                              int I, int E, int k, int bits, int group_size_up,
                              int group_size_down, float *route_out, float *out);

/* EagerMoeMlp.forward for the quantized formats
 * (src/zoo/privacy-filter/moeMlp.ts:79-121): xn = rmsNorm(x, norm_w, eps),
 * route = topk(xn·W + b, k), out = x + moeDown(moeUp(xn, route, glu, lin),
 * route, down). The residual is x itself, in its own dtype. x and norm_w
 * share x_dtype (f32 or f16); norm_w is [d]; the privacy filter's eps is
 * 1e-5 (moeMlp.ts:23). The norm's sum of squares follows this library's
 * canonical order (see moe_rmsnorm), so the expert ids are reproducible. */
MOE_API int moe_block(moe_ctx *ctx, const void *x, moe_dtype x_dtype, const void *norm_w,
                      float eps, const float *w_router, const float *b_router,
                      const moe_expert_weight *glu, const moe_expert_weight *lin,
                      const moe_expert_weight *down, int T, int d, int I, int E, int k, int bits,
                      int group_size_up, int group_size_down, float *route_out, float *out);
/* rmsNorm(x, weight, eps, {group, residual, scale})
 * (src/core/graph/ops/reduce.ts:61-92): over each run of `group` columns of
 * a [rows, cols] row, out = (residual + x · 1/sqrt(mean(x²) + eps) · w) · scale.
 * x, weight, residual (NULL: none) and out share `dtype`; weight_len is
 * `group` (one weight shared by every run) or `cols` (a slice per run).
 * Sums in f32 in a canonical order: lane l of a 64-wide wavefront adds the
 * squares of the quads q ≡ l (mod 64) in ascending order, the 64 lane sums
 * meet in an xor butterfly (strides 32..1), then 1/sqrt(sum/group + eps),
 * each operation correctly rounded. */
MOE_API int moe_rmsnorm(moe_ctx *ctx, const void *x, moe_dtype dtype, int rows, int cols,
                        const void *weight, int weight_len, float eps, int group,
                        const void *residual, float scale, void *out);
/* matmulGather(a, w, expertIdx, {bias}) (src/core/graph/ops/matmul.ts:180-210):
 * out[i] = a[i]·W[e_i] + bias[e_i], W = rows [e·K, (e+1)·K) of the float
 * weight w [E·K, N] (row-major), e_i = expert_idx[i] (f32 [M], exact
 * integers). a [M, K], w, bias [E, N] (or NULL) and out [M, N] share dtype.
 * N must be divisible by 4. A row whose index is not an expert is zero. */
MOE_API int moe_matmul_gather(moe_ctx *ctx, const void *a, moe_dtype dtype, const void *w,
                              const void *bias, const float *expert_idx, int M, int K, int N,
                              int E, void *out);
/* EagerMoeMlp.forward for float weights (src/zoo/privacy-filter/moeMlp.ts
 * :79-100): xn = rmsNorm(x), route = topk(xn·W + b, k), and per slot
 * swiglu(gather(xn, glu) , gather(xn, lin)) → gather(·, out), weighted by the
 * gates and summed over the slots, + x. x, norm_w and the expert weights
 * and biases share dtype (f32 or f16): glu_w, lin_w [E·d, I], out_w [E·I, d]
 * row-major, biases [E, I] / [E, d] (or NULL); router W f32 [d, E], b [E] or
 * NULL. Intermediates are f32; out f32 [T, d]. */
MOE_API int moe_block_float(moe_ctx *ctx, const void *x, moe_dtype dtype, const void *norm_w,
                            float eps, const float *w_router, const float *b_router,
                            const void *glu_w, const void *glu_b, const void *lin_w,
                            const void *lin_b, const void *out_w, const void *out_b, int T, int d,
                            int I, int E, int k, float *route_out, float *out);
/* The privacy filter's constrained Viterbi decode (src/zoo/privacy-filter/
 * viterbi.ts:85-148), host memory, no GPU: path [T] = the best label path
 * under start [n], end [n] and trans [n·n] (prev-major) f64 scores and
 * log_probs [T, n] f32; ties keep the lower previous / last label; when no
 * score stays finite, the per-token argmax. */
MOE_API int moe_viterbi_decode(const double *start, const double *end, const double *trans,
                               const float *log_probs, int T, int n, int32_t *path);
/* Linear (src/core/nn/layers.ts:166-263): out [T, N] = x [T, K] · w [K, N]
 * + bias [N] (or NULL) + addend [T, N] (or NULL), all f32, w row-major
 * [in, out] (a quantized checkpoint weight dequantized once at load). Uses
 * the context workspace for K-slice partial products. */
MOE_API int moe_linear(moe_ctx *ctx, const float *x, const float *w, const float *bias,
                       const float *addend, int T, int K, int N, float *out);
/* The attention core of the privacy filter's block (src/zoo/privacy-filter/
 * attnBlock.ts:39-55): over one qkv tensor [T, (q_heads + 2·kv_heads)·
 * head_dim] read in place, q and k are roped with cos/sin (f32 [T,
 * head_dim], pair-duplicated, scale folded in) as they are staged, then the
 * banded sdpa of moe_sdpa (q_pos_offset 0, no segments or key bias) writes
 * out [T, q_heads·head_dim]. It equals moe_rope on the q and k column
 * blocks followed by moe_sdpa, in one kernel; it has no single counterpart
 * in the reference. */
MOE_API int moe_attention(moe_ctx *ctx, const void *qkv, moe_dtype dtype, int T, int q_heads,
                          int kv_heads, int head_dim, int64_t window_left, int64_t window_right,
                          const float *sinks, const float *cos_t, const float *sin_t, void *out);
/* rope (src/core/graph/ops/attention.ts:220-262): out [rows, width] =
 * the interleaved pairs of x's columns [src_start, src_start + width)
 * rotated by cos/sin (f32 [rows, head_dim], pair-duplicated, any scale
 * folded in): out[2p] = x0·c − x1·s, out[2p+1] = x1·c + x0·s. x is
 * [rows, cols] of dtype; out has x's dtype. */
MOE_API int moe_rope(moe_ctx *ctx, const void *x, moe_dtype dtype, int rows, int cols,
                     int head_dim, int src_start, int width, const float *cos_t,
                     const float *sin_t, void *out);
/* sdpa (src/core/graph/ops/attention.ts:28-145) and sdpaPacked (:146-214,
 * pass the qkv tensor's q, k and v column blocks with its row stride):
 * out [q_len, q_heads·head_dim] (dtype) = softmax(q·kᵀ + key bias)·v per
 * query row i and head h over the keys j with qPos − window_left ≤ j ≤
 * qPos + window_right (qPos = q_pos_offset + i; a negative window is
 * unbounded) inside the row's segment [segments[2i], segments[2i+1]) if
 * given; query head h reads kv head h / (q_heads / kv_heads). q and k
 * arrive pre-scaled. sinks (f32 [q_heads] or NULL) add exp(sink · ln 2) to
 * the denominator alone. key_bias adds key_bias_value to the scores of keys
 * [key_bias_start, key_bias_end). A row that sees no key is 0. Strides are
 * in elements; head_dim ≤ 128. */
MOE_API int moe_sdpa(moe_ctx *ctx, moe_dtype dtype, const void *q, int64_t q_stride,
                     const void *k, int64_t k_stride, const void *v, int64_t v_stride,
                     int q_len, int kv_len, int q_heads, int kv_heads, int head_dim,
                     int64_t window_left, int64_t window_right, int q_pos_offset,
                     const float *sinks, const float *segments, int key_bias,
                     int key_bias_start, int key_bias_end, float key_bias_value, void *out);
/* Strides between the calls of moe_layer_batched, in elements of each
 * tensor (u32 words for quantW weights). 0 shares a tensor between calls. */
typedef struct moe_call_strides {
  int64_t x, router_w, router_b;
  int64_t glu_w, glu_scales, glu_bias;
  int64_t lin_w, lin_scales, lin_bias;
  int64_t down_w, down_scales, down_bias;
  int64_t residual, route, out;
} moe_call_strides;

/* `calls` independent moe_layer calls of identical shape, enqueued as one
 * set of kernels: call c reads and writes every tensor at
 * base + c·stride (strides NULL: all 0, valid for calls == 1). Each call is
 * routed, dispatched and computed on its own, exactly as moe_layer would;
 * the calls only share the launches. x, out and route_out need non-zero
 * strides when calls > 1. No reference counterpart: it lets single-token
 * decode calls of separate layer instances (e.g. independent requests on
 * separate weight sets) fill the GPU instead of running one launch-bound
 * call at a time. */
MOE_API int moe_layer_batched(moe_ctx *ctx, int calls, const moe_call_strides *strides,
                              const void *x, moe_dtype x_dtype, const float *w_router,
                              const float *b_router, const moe_expert_weight *glu,
                              const moe_expert_weight *lin, const moe_expert_weight *down,
                              const float *residual, int T, int d, int I, int E, int k, int bits,
                              int group_size_up, int group_size_down, float *route_out,
                              float *out);

/* Per-kernel-group timing on the context's stream — the reference's
 * GpuPerfSink with perOp (src/core/gpu/perf.ts:1-23, timing.ts:62-111).
 * While enabled, every launch group is bracketed by a HIP event pair.
 * moe_prof_read waits for the stream and returns, per group (index: 0 topk,
 * 1 router, 2 dispatch, 3 up, 4 down, 5 combine, 6 norm; 8 slots), the summed
 * milliseconds and the number of timed groups; reset != 0 clears them. */
MOE_API int moe_prof_enable(moe_ctx *ctx, int on);
MOE_API int moe_prof_read(moe_ctx *ctx, int reset, double *ms_out, int64_t *count_out);

/* Test and diagnostic hook: the dispatch permutation of a route, as the
 * layer builds it. perm [T·k] (sorted position → assignment t·k + s, −1
 * past the valid ones), offsets [E + 1]. No reference counterpart: the
 * reference has no permutation (moeQuantW.ts:131-134); exposed so its
 * bit-exactness can be checked. */
MOE_API int moe_dispatch(moe_ctx *ctx, const float *route, int T, int E, int k, int32_t *perm,
                 int32_t *offsets);

/* Packs E experts' signed int weights into quantW words on the device:
 * replaces packQuantW (src/core/weights/quantPack.ts:12-28) applied per
 * expert with the words concatenated expert-major (the upload step of the
 * weights). ints: device int8 [E][n][k] (each expert output-first, torch's
 * Linear layout; int4 values in [-8, 7] one per byte). words: device
 * uint32 [E·k·n·bits/32], the logical [E·k, n] quantW weight. k and n must
 * be multiples of 4; bits 8 or 4. */
MOE_API int moe_pack_quantw(moe_ctx *ctx, const int8_t *ints, int E, int k, int n, int bits,
                            uint32_t *words);

/* An expert weight owned by the library: device copies of one
 * QuantExpertWeight's w, scales and bias — the weight-load step the
 * reference does through a Parameter, which owns its GPU buffer
 * (src/core/nn/module.ts:20-65; weights uploaded with upload(),
 * test/gpu.ts:73-83, packed by packQuantW, src/core/weights/quantPack.ts).
 * host: quantW words (E·K·N·bits/32 u32) when raw_int8 is 0, else int8
 * [E][N][K] (each expert output-first, one value per byte) packed on the
 * device; scales f32 [E·K/groupSize, N]; bias f32 [E, N] or NULL. All host
 * pointers; the call returns once they may be freed. An empty shape is
 * INVALID_ARGUMENT, as the reference's upload of an empty tensor
 * (test/core/kernels/matmul/moeQuantW.gpu.test.ts:167-171). */
typedef struct moe_weights moe_weights;
MOE_API int moe_weights_upload(moe_ctx *ctx, const void *host, int raw_int8, const float *scales,
                               const float *bias, int E, int K, int N, int bits, int group_size,
                               moe_weights **out);
/* The device pointers of an uploaded weight, for moe_up / moe_down /
 * moe_layer. RESOURCE_DISPOSED after moe_weights_dispose (the reference's
 * use of a disposed Value). */
MOE_API int moe_weights_view(const moe_weights *h, moe_expert_weight *view);
/* Frees the device buffers (Parameter.dispose()); the handle stays valid
 * and reports RESOURCE_DISPOSED. Waits for work already enqueued. */
MOE_API int moe_weights_dispose(moe_weights *h);
/* Disposes if needed and frees the handle itself. */
MOE_API int moe_weights_release(moe_weights *h);

/* ------------------------------------------------ executor plumbing (host)
 *
 * What a ruNNtime Executor backed by this library needs besides the ops
 * (src/core/graph/evalCore.ts:14-43): the shape checks its op builders run,
 * and device buffers to hand out, fill and read back. */

/* A Value's metadata, as ValueMeta (src/core/graph/value.ts:17-24): the
 * element count in units of dtype (u32 words for quantW) and the dims when
 * the value has a logical shape (rank 0: none). */
typedef enum moe_value_dtype {
  MOE_VALUE_F32 = 0, MOE_VALUE_F16 = 1, MOE_VALUE_QUANTW = 2
} moe_value_dtype;
typedef struct moe_value_desc {
  int dtype;       /* moe_value_dtype */
  int rank;        /* number of dims, 0..4 */
  int64_t dims[4];
  int64_t elems;
} moe_value_desc;

/* checkExpertWeight (src/core/graph/ops/matmul.ts:274-315), host only, no
 * context: the checks moeUp / moeDown run on one routed layer's weight
 * {w, scales, bias} against its input's K (k_in) and the route of t tokens
 * with `slots` ids per token (the reference's 4). INVALID_ARGUMENT with the
 * reference's message on the first failed check; else n_out and
 * experts_out (may be NULL) receive N and the expert count. */
MOE_API int moe_check_expert_weight(const char *op, const moe_value_desc *w,
                                    const moe_value_desc *scales, const moe_value_desc *bias,
                                    const moe_value_desc *route, int64_t k_in, int64_t t,
                                    int slots, int bits, int group_size, int64_t *n_out,
                                    int64_t *experts_out);

/* Device buffers on the context's device: the Executor's acquireOutput /
 * releaseOutput (evalCore.ts:14-17), an upload (the reference's
 * upload(), test/gpu.ts:73-83) and a Readback (evalCore.ts:38-43).
 * Write and read are synchronous with the context's stream (they wait for
 * the work queued before them). A zero-byte buffer is INVALID_ARGUMENT, as
 * the reference's empty upload. */
MOE_API int moe_buffer_alloc(moe_ctx *ctx, size_t bytes, void **out);
MOE_API int moe_buffer_free(moe_ctx *ctx, void *ptr);
MOE_API int moe_buffer_write(moe_ctx *ctx, void *dst, const void *host, size_t bytes);
MOE_API int moe_buffer_read(moe_ctx *ctx, void *host, const void *src, size_t bytes);

#ifdef __cplusplus
}
#endif
#endif /* RUNNTIME_MOE_H */
