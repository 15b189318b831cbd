// Internal declarations shared by the HIP translation units of libmoe.so.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/runntime_moe.h"

#define MOE_VERSION 1

// ------------------------------------------------------------------ errors

void moe_set_error(const std::string &msg);
int moe_fail(int code, const std::string &msg);

#define MOE_HIP_CHECK(expr)                                                               \
  do {                                                                                    \
    hipError_t _e = (expr);                                                               \
    if (_e != hipSuccess)                                                                 \
      return moe_fail(MOE_EXECUTION_FAILED,                                               \
                      std::string(#expr) + ": " + hipGetErrorString(_e));                 \
  } while (0)

// ----------------------------------------------------------------- context

// Per-kernel-group timing (the reference's GpuPerfSink, src/core/gpu/perf.ts):
// an event pair around every launch group while enabled, resolved on read.
constexpr int PROF_GROUPS = 8;
struct ProfRecord {
  int group;
  hipEvent_t begin, end;
};

struct moe_ctx {
  int device = 0;
  hipStream_t stream = nullptr;      // stream the calls enqueue on
  hipStream_t own_stream = nullptr;  // created by the context
  char *ws = nullptr;                // device workspace
  size_t ws_size = 0;
  int ws_pins = 0;                   // > 0: the workspace must not move
  bool disposed = false;
  bool prof_on = false;
  std::vector<ProfRecord> prof_pending;  // recorded, not yet resolved
  std::vector<hipEvent_t> prof_free;     // reusable events
  double prof_ms[PROF_GROUPS] = {};
  int64_t prof_count[PROF_GROUPS] = {};
};

// Kernel groups the timing sink reports.
enum ProfGroup {
  PG_TOPK = 0, PG_ROUTER = 1, PG_DISPATCH = 2, PG_UP = 3, PG_DOWN = 4, PG_COMBINE = 5, PG_NORM = 6
};
extern const char *const PROF_NAMES[PROF_GROUPS];

// Brackets the launches of one group with events when timing is on.
struct ProfScope {
  moe_ctx *ctx;
  int group;
  bool on;
  hipEvent_t b = nullptr;
  // enable false: no timing (the allocation-free entry point creates no events)
  ProfScope(moe_ctx *c, int g, bool enable = true);
  ~ProfScope();
};

// Bump allocator over the context workspace. Sizes are rounded to 256 B.
struct WsPlan {
  size_t off = 0;
  size_t take(size_t bytes) {
    size_t at = off;
    off += (bytes + 255) & ~size_t(255);
    return at;
  }
};

int moe_ws_ensure(moe_ctx *ctx, size_t bytes);

// ------------------------------------------------------------ constants

// Assignments per dispatch block (counting-sort tile).
constexpr int DISPATCH_TILE = 1024;
// Width of one canonical router chunk (the fma chain length).
constexpr int ROUTER_CHUNK = 64;
// Largest expert count the fused router keeps in registers.
constexpr int ROUTER_MAX_E = 512;
// Largest expert count the standalone topk handles.
constexpr int TOPK_MAX_E = 4096;
constexpr int MAX_K = 16;
// Largest expert count of the dispatch and expert kernels (LDS arrays).
constexpr int DISPATCH_MAX_E = 1024;

// Device-side bookkeeping written by the dispatch scan (int32 each).
enum MetaSlot { META_VALID = 0, META_ACTIVE = 1, META_MAXCNT = 2, META_TILES = 3, META_N = 8 };

// Largest token count whose routing and dispatch one block does (fused).
constexpr int SMALL_T = 16;
// Calls up to FUSED_T tokens (T·k ≤ FUSED_T·MAX_K) run the router's fold,
// top-k and dispatch in one block per call.
constexpr int FUSED_T = 64;
// Rows per M-tile of the grouped GEMM; the dispatch counts M-tiles with it.
constexpr int GEMM_TILE_M = 128;

// Dispatch workspace of a batch of calls. Each call owns a slice: the
// per-call sizes below are the strides between them.
struct DispatchBufs {
  int32_t *blk_counts;  // [nblk, E] per call
  int32_t *blk_base;    // [nblk, E] per call
  int32_t *offsets;     // [E + 1] per call
  int32_t *tile_off;    // [E + 1] per call: cumulative M-tiles per expert
  int32_t *active;      // [E][4] per call: {expert, first row, rows, first M-tile} of the
                        // experts with rows, ascending; then {-1, 0, 0, 0}
  int32_t *meta;        // [META_N] per call
  int32_t *perm;        // [A] per call: sorted position → assignment
  int E, A, nblk;       // sizes that give the per-call strides
  __host__ __device__ int64_t cnt_cs() const { return (int64_t)nblk * E; }
  __host__ __device__ int64_t off_cs() const { return (int64_t)E + 1; }
  __host__ __device__ int64_t act_cs() const { return 4 * (int64_t)E; }
  __host__ __device__ int64_t meta_cs() const { return META_N; }
  __host__ __device__ int64_t perm_cs() const { return A; }
};

// ---------------------------------------------------------- launchers

// Launchers refuse NULL device pointers: a kernel must never be handed one.
#define MOE_NONNULL(ptr)                                                                  \
  do {                                                                                    \
    if (!(ptr)) return moe_fail(MOE_EXECUTION_FAILED, std::string(__func__) + ": " #ptr " is NULL"); \
  } while (0)

// Every launcher takes `calls` independent calls of identical shape; call c
// reads and writes each tensor at base + c·stride (elements; words for
// quantW). A stride of 0 shares the tensor between calls.

int launch_topk(const void *logits, moe_dtype dt, int T, int E, int k, float *route,
                hipStream_t s);

struct RouterArgs {
  const void *x;
  moe_dtype x_dtype;
  int64_t x_cs;
  const float *w;
  int64_t w_cs;
  const float *b;  // may be NULL
  int64_t b_cs;
  float *route;
  int64_t route_cs;
  float *partial;  // workspace, T·J·E floats per call
  int T, d, E, k, calls;
  // moe_block's pre-norm, applied while staging x (one call): weight [d] of
  // x's dtype, or NULL; the chunk kernels also write each token's inverse
  // RMS to inv [T].
  const void *norm_w;
  float norm_eps;
  float *inv;
  // Only the chunk sums (partial): the fold, top-k and dispatch run in the
  // up product's prologue (ExpertArgs::fr_partial).
  int chunks_only;
};
// Router + top-k. With T <= FUSED_T and `db` given, the dispatch of each call
// is built in the same kernel and `dispatched` is set.
int launch_router_topk(const RouterArgs &ra, const DispatchBufs *db, int tile_m, bool *dispatched,
                       hipStream_t s);
int launch_dispatch(const float *route, int64_t route_cs, int T, int E, int k, int calls,
                    int tile_m, const DispatchBufs &db, hipStream_t s);

enum ExpertMode { MODE_UP = 0, MODE_DOWN = 1 };

struct ExpertArgs {
  int mode;                 // ExpertMode
  const void *a;            // x [T, K] (up) or act [T·k, K] (down)
  moe_dtype a_dtype;
  int64_t a_cs;
  int a_row_div;            // source row = assignment / a_row_div (k for up, 1 for down)
  const float *route;       // [T, 2k]
  int64_t route_cs;
  int k;
  moe_expert_weight w0;     // glu (up) or down
  moe_expert_weight w1;     // lin (up); unused for down
  int64_t w0_cs, s0_cs, b0_cs, w1_cs, s1_cs, b1_cs;
  int K, N, E, bits, g;
  float *out;               // act [T·k, N] (up) or y [T·k, N] (down), row = assignment
  int64_t out_cs;
  int A;                    // T·k
  int calls;
  // Intermediate rows in dispatch (sorted) order instead of assignment
  // order: up writes act row p for sorted position p, down reads it there.
  // The fused layer sets it for both products when both run on the grouped
  // GEMM or both on the decode kernels. Such act is private to the two
  // products: on the grouped GEMM each f32 value is stored as its f16 hi +
  // lo split (the operands down's MFMAs take), hi(n), hi(n + 1), lo(n),
  // lo(n + 1) per column pair; on the decode kernels it stays f32.
  int dispatch_order;
  // Down on the grouped GEMM: K split into `parts` halves whose partial
  // products go to out + part·A·N (the combine adds them). 0 or 1 = whole K.
  int parts;
  // Both products of the fused layer on the int8-limb act form: up (the
  // f16-x grouped GEMM) writes act as int8 limbs over padded rows, down runs
  // on the int8 matrix cores (gemm_i8.hip). Implies dispatch_order.
  int act_i8;
  // Up of moe_block on the skinny kernel: x is normalised while staging,
  // row t scaled by a_inv[t] (written by the router) and the weight
  // a_normw [K] of x's dtype; NULL for plain x.
  const float *a_inv;
  const void *a_normw;
  // Up of single-token calls on the skinny kernel (fr_partial non-NULL):
  // the router's fold and top-k and the call's dispatch run in the kernel's
  // prologue from the chunk sums fr_partial [J·E] per call (fr_J chunks) and
  // the router bias fr_b (may be NULL; fr_b_cs per call); block (0, 0) of
  // each call writes the route row (route) and the dispatch buffers that
  // down and the combine read.
  const float *fr_partial;
  const float *fr_b;
  int64_t fr_b_cs;
  int fr_J;
  int fr_tile_m;
};

int launch_expert(const ExpertArgs &ea, const DispatchBufs &db, hipStream_t s);
// Whether the up product of these arguments can take the router's fold,
// top-k and dispatch into its prologue (single-token calls on the skinny
// kernel, E ≤ 256, J ≤ 16 chunks).
bool expert_fuses_route(const ExpertArgs &up, int J);
// The grouped GEMM (gemm.hip) for many rows per expert.
bool gemm_eligible(const ExpertArgs &ea);
// Whether launch_expert runs these arguments on the grouped GEMM.
bool expert_uses_gemm(const ExpertArgs &ea);
// Whether the gate/up product can normalise x while staging it (a_inv,
// a_normw): the skinny MFMA kernel.
bool expert_stages_norm(const ExpertArgs &ea);
// K parts the grouped GEMM uses for this down product (1 or 2): 2 when the
// split evens out the last round of tiles over the CUs.
int gemm_down_parts(const ExpertArgs &ea);
// The int8-limb act form of the fused layer (gemm_i8.hip): whether down can
// take it, and the bytes of act in that form.
bool gemm_i8_down_eligible(const ExpertArgs &dn);
// The direct-weight up GEMM (gemm_wide.hip) takes these arguments.
bool gemm_wide_eligible(const ExpertArgs &ea);
int64_t gemm_i8_act_bytes(int A, int E, int K);
int launch_expert_gemm(const ExpertArgs &ea, const DispatchBufs &db, hipStream_t s);
// Fills n floats with 0 (a kernel, not hipMemsetAsync, so a captured graph
// replays it correctly).
int launch_zero(float *p, size_t n, hipStream_t s);
// out[t] = residual[t] + Σ_s gate_s · y[t·k + s] per call.
int launch_pack_quantw(const int8_t *ints, int E, int k, int n, int bits, uint32_t *words,
                       hipStream_t s);
// y holds `parts` partial products, part_cs floats apart (per call). The
// residual is f32 or f16 (res_dtype), or NULL.
int launch_combine(const float *y, int64_t y_cs, int parts, int64_t part_cs, const float *route,
                   int64_t route_cs, const void *residual, moe_dtype res_dtype, int64_t res_cs,
                   int T, int N, int E, int k, float *out, int64_t out_cs, int calls,
                   hipStream_t s);

// RMSNorm over runs of `group` columns (norm.hip). x, weight, residual and
// out share `dtype`; weight is `group` long (shared by every run) or `cols`
// long (a slice per run); residual may be NULL.
struct NormArgs {
  const void *x;
  const void *weight;
  const void *residual;
  void *out;
  moe_dtype dtype;
  int rows, cols, group, weight_len;
  float eps, scale;
};
int launch_rmsnorm(const NormArgs &a, hipStream_t s);

// Attention ops (attn.hip). Row strides are in elements; windows < 0 are
// unbounded; segs f32 [q_len, 2] (first key, end key) or NULL.
struct AttnArgs {
  const void *q, *k, *v;
  int64_t q_rs, k_rs, v_rs;
  void *out;
  int64_t o_rs;
  moe_dtype dtype;
  int q_len, kv_len, q_heads, kv_heads, head_dim;
  long long window_left, window_right;
  int q_pos_offset;
  const float *sinks;
  const float *segs;
  int has_kb, kb_start, kb_end;
  float kb_value;
  // Optional rope of q and k while staging (f32 [rows, head_dim] tables,
  // pair-duplicated, indexed by the q / k row), or NULL.
  const float *rope_cos, *rope_sin;
  int rows_per_block;  // set by the launcher
};
int launch_rope(const void *x, moe_dtype dt, int rows, int cols, int hd, int src_start, int width,
                const float *cs, const float *sn, void *out, hipStream_t s);
int launch_sdpa(AttnArgs a, hipStream_t s);
// Dense f32 Linear (linear.hip): y = x·W + bias + addend; `part` holds
// linear_ws_bytes(T, K, N) of K-slice partial products.
size_t linear_ws_bytes(int T, int K, int N);
int launch_linear(const float *x, const float *w, const float *bias, const float *addend, float *y,
                  float *part, int T, int K, int N, hipStream_t s);
int moe_ws_ensure(moe_ctx *ctx, size_t bytes);

// Float-weight expert products (float.hip): rows grouped by the dispatch,
// weights row-major [E·K, N] of f32 or f16, biases [E, N] of the same type
// (may be NULL). MODE_UP: act = swiglu(a·w0 + b0, a·w1 + b1), f32 out;
// MODE_DOWN: out = a·w0 + b0. Row r of a is perm / a_row_div; out row is the
// assignment.
struct FloatArgs {
  const void *a;
  int64_t a_cs;
  int a_row_div;
  const void *w0, *b0, *w1, *b1;
  int64_t w0_cs, b0_cs, w1_cs, b1_cs;
  int K, N;
  void *out;
  int64_t out_cs;
  DispatchBufs db;
};
int launch_float_expert(const FloatArgs &p, int mode, moe_dtype a_dt, moe_dtype w_dt,
                        moe_dtype o_dt, int max_active, int calls, hipStream_t s);
// route [M, 2] = {idx[i], 1} for a one-slot gather.
int launch_idx_route(const float *idx, int M, float *route, hipStream_t s);
