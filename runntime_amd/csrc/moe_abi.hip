// C ABI of libmoe.so: argument checks, the context and its workspace, and the
// order of kernel launches for each op. Declarations and the reference
// interface each entry replaces are in include/runntime_moe.h.
#include <stdio.h>

#include <string>

#include "moe_internal.h"

#include <mutex>

// ------------------------------------------------------------------ errors

static thread_local std::string g_last_error;

void moe_set_error(const std::string &msg) { g_last_error = msg; }

int moe_fail(int code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

extern "C" const char *moe_last_error(void) { return g_last_error.c_str(); }
extern "C" int moe_version(void) { return MOE_VERSION; }

// ------------------------------------------------------------------ timing

const char *const PROF_NAMES[PROF_GROUPS] = {"topk", "router", "dispatch", "up",
                                             "down", "combine", "norm", ""};

static hipEvent_t prof_event(moe_ctx *c) {
  if (!c->prof_free.empty()) {
    hipEvent_t e = c->prof_free.back();
    c->prof_free.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

ProfScope::ProfScope(moe_ctx *c, int g, bool enable) : ctx(c), group(g), on(enable && c->prof_on) {
  if (!on) return;
  b = prof_event(ctx);
  if (b) (void)hipEventRecord(b, ctx->stream);
}

ProfScope::~ProfScope() {
  if (!on || !b) return;
  hipEvent_t e = prof_event(ctx);
  if (!e) return;
  (void)hipEventRecord(e, ctx->stream);
  ctx->prof_pending.push_back({group, b, e});
}

extern "C" int moe_prof_enable(moe_ctx *ctx, int on) {
  if (!ctx) return moe_fail(MOE_NOT_INITIALIZED, "moe_prof_enable: context is NULL");
  ctx->prof_on = on != 0;
  return MOE_OK;
}

extern "C" int moe_prof_read(moe_ctx *ctx, int reset, double *ms_out, int64_t *count_out) {
  if (!ctx) return moe_fail(MOE_NOT_INITIALIZED, "moe_prof_read: context is NULL");
  MOE_HIP_CHECK(hipSetDevice(ctx->device));
  MOE_HIP_CHECK(hipStreamSynchronize(ctx->stream));
  for (auto &r : ctx->prof_pending) {
    float ms = 0.f;
    MOE_HIP_CHECK(hipEventElapsedTime(&ms, r.begin, r.end));
    ctx->prof_ms[r.group] += ms;
    ctx->prof_count[r.group] += 1;
    ctx->prof_free.push_back(r.begin);
    ctx->prof_free.push_back(r.end);
  }
  ctx->prof_pending.clear();
  for (int g = 0; g < PROF_GROUPS; g++) {
    if (ms_out) ms_out[g] = ctx->prof_ms[g];
    if (count_out) count_out[g] = ctx->prof_count[g];
    if (reset) {
      ctx->prof_ms[g] = 0;
      ctx->prof_count[g] = 0;
    }
  }
  return MOE_OK;
}

// ------------------------------------------------------------------ context

// ------------------------------------------------ allocation-free scratch
//
// moe_layer_noalloc's workspace: a file-scope device array, one per GPU the
// library runs on, held until the process ends. Host code never uses the
// array's name as an address (on the host it is a stand-in, not device
// memory): its address on each device comes from hipGetSymbolAddress, taken
// once per device with that device current (at moe_ctx_create), and only
// that pointer goes to kernels.
static __device__ __align__(256) char scratch[MOE_NOALLOC_SCRATCH_BYTES];
constexpr int SCRATCH_MAX_DEVICES = 64;
static char *g_scratch_ptr[SCRATCH_MAX_DEVICES];
// The last (context, stream) that used a device's scratch. A call from
// another context or stream while that stream still has work queued would
// race on the scratch; moe_layer_noalloc refuses it.
struct ScratchOwner {
  const moe_ctx *ctx;
  hipStream_t stream;
};
static ScratchOwner g_scratch_owner[SCRATCH_MAX_DEVICES];
static std::mutex g_scratch_mu;

// The scratch address on `device` (current); NULL and an error if unknown.
// A failed lookup is not remembered: the next call tries again.
static char *scratch_on(int device, hipError_t *err) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (device < 0 || device >= SCRATCH_MAX_DEVICES) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  *err = hipSuccess;
  if (!g_scratch_ptr[device]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      (void)hipGetLastError();
      *err = e != hipSuccess ? e : hipErrorInvalidSymbol;
      return nullptr;
    }
    g_scratch_ptr[device] = (char *)p;
  }
  return g_scratch_ptr[device];
}

// Claims `device`'s scratch for (ctx, ctx->stream): refused (false, with the
// reason in *why) while another context or stream that used it last still
// has work queued. Calls on one stream are ordered by the stream itself.
static bool scratch_claim(const moe_ctx *ctx, std::string *why) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchOwner &o = g_scratch_owner[ctx->device];
  // Under a stream capture nothing runs now (and querying other streams is
  // not allowed while capturing): the record only moves to the capturing
  // stream.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(ctx->stream, &cap) != hipSuccess) {
    (void)hipGetLastError();
    cap = hipStreamCaptureStatusNone;
  }
  if (cap == hipStreamCaptureStatusNone && o.ctx && (o.ctx != ctx || o.stream != ctx->stream)) {
    const hipError_t q = hipStreamQuery(o.stream);
    (void)hipGetLastError();  // a not-ready query must not reach the next error check
    if (q == hipErrorNotReady || q == hipErrorStreamCaptureUnsupported ||
        q == hipErrorStreamCaptureInvalidated) {
      *why = std::string(o.ctx != ctx ? "another context" : "another stream of this context") +
             " used the static scratch of device " + std::to_string(ctx->device) +
             " last and its stream has not finished: synchronise it first (calls that overlap "
             "on one GPU would share the scratch)";
      return false;
    }
  }
  o.ctx = ctx;
  o.stream = ctx->stream;
  return true;
}

// A destroyed context no longer owns any scratch.
static void scratch_release(const moe_ctx *ctx) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  for (auto &o : g_scratch_owner)
    if (o.ctx == ctx) o = ScratchOwner{};
}

extern "C" int moe_ctx_create(int device, void *stream, moe_ctx **out) {
  if (!out) return moe_fail(MOE_INVALID_ARGUMENT, "moe_ctx_create: out is NULL");
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
    return moe_fail(MOE_NOT_INITIALIZED, "moe_ctx_create: no HIP device is visible");
  if (device < 0 || device >= n)
    return moe_fail(MOE_INVALID_ARGUMENT, "moe_ctx_create: device " + std::to_string(device) +
                                              " out of range (" + std::to_string(n) + " visible)");
  MOE_HIP_CHECK(hipSetDevice(device));
  // The allocation-free entry point's scratch on this device (once per
  // device; its failure surfaces only in moe_layer_noalloc).
  hipError_t scratch_err = hipSuccess;
  (void)scratch_on(device, &scratch_err);
  moe_ctx *c = new moe_ctx();
  c->device = device;
  if (stream == MOE_NULL_STREAM) {
    c->stream = nullptr;  // HIP's null stream
  } else if (stream) {
    c->stream = (hipStream_t)stream;
  } else {
    hipError_t e = hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
      delete c;
      return moe_fail(MOE_EXECUTION_FAILED,
                      std::string("hipStreamCreate: ") + hipGetErrorString(e));
    }
    c->stream = c->own_stream;
  }
  *out = c;
  return MOE_OK;
}

static int check_ctx(moe_ctx *ctx, const char *op) {
  if (!ctx) return moe_fail(MOE_NOT_INITIALIZED, std::string(op) + ": context is NULL");
  if (ctx->disposed) return moe_fail(MOE_RESOURCE_DISPOSED, std::string(op) + ": context disposed");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess)
    return moe_fail(MOE_EXECUTION_FAILED, std::string("hipSetDevice: ") + hipGetErrorString(e));
  return MOE_OK;
}

extern "C" int moe_ctx_set_stream(moe_ctx *ctx, void *stream) {
  int rc = check_ctx(ctx, "moe_ctx_set_stream");
  if (rc) return rc;
  if (stream == MOE_NULL_STREAM) {
    ctx->stream = nullptr;  // HIP's null stream
    return MOE_OK;
  }
  if (stream) {
    ctx->stream = (hipStream_t)stream;
    return MOE_OK;
  }
  if (!ctx->own_stream)
    MOE_HIP_CHECK(hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking));
  ctx->stream = ctx->own_stream;
  return MOE_OK;
}

int moe_ws_ensure(moe_ctx *ctx, size_t bytes) {
  if (bytes <= ctx->ws_size) return MOE_OK;
  // A graph captured over the workspace holds its address: never move it
  // while pinned, nor inside a capture (the synchronize and the allocation
  // below are not capturable).
  if (ctx->ws_pins > 0)
    return moe_fail(MOE_EXECUTION_FAILED,
                    "workspace is pinned (captured graphs use it) and holds " +
                        std::to_string(ctx->ws_size) + " bytes; this call needs " +
                        std::to_string(bytes) + ": reserve before pinning");
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  MOE_HIP_CHECK(hipStreamIsCapturing(ctx->stream, &cap));
  if (cap != hipStreamCaptureStatusNone)
    return moe_fail(MOE_EXECUTION_FAILED,
                    "workspace of " + std::to_string(ctx->ws_size) + " bytes is too small for a "
                    "call inside a stream capture (needs " + std::to_string(bytes) +
                    "): reserve before capturing");
  // Work already queued may still read the old workspace.
  MOE_HIP_CHECK(hipStreamSynchronize(ctx->stream));
  if (ctx->ws) MOE_HIP_CHECK(hipFree(ctx->ws));
  ctx->ws = nullptr;
  ctx->ws_size = 0;
  size_t want = bytes + bytes / 4;
  MOE_HIP_CHECK(hipMalloc((void **)&ctx->ws, want));
  ctx->ws_size = want;
  return MOE_OK;
}

extern "C" int moe_ctx_pin_workspace(moe_ctx *ctx, int pin) {
  int rc = check_ctx(ctx, "moe_ctx_pin_workspace");
  if (rc) return rc;
  if (pin) {
    ctx->ws_pins++;
  } else {
    if (ctx->ws_pins == 0)
      return moe_fail(MOE_INVALID_ARGUMENT, "moe_ctx_pin_workspace: workspace is not pinned");
    ctx->ws_pins--;
  }
  return MOE_OK;
}

extern "C" int moe_ctx_destroy(moe_ctx *ctx) {
  if (!ctx) return MOE_OK;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  if (ctx->ws) (void)hipFree(ctx->ws);
  for (auto &r : ctx->prof_pending) {
    (void)hipEventDestroy(r.begin);
    (void)hipEventDestroy(r.end);
  }
  for (auto e : ctx->prof_free) (void)hipEventDestroy(e);
  if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
  scratch_release(ctx);
  ctx->disposed = true;
  delete ctx;
  return MOE_OK;
}

extern "C" int moe_sync(moe_ctx *ctx) {
  int rc = check_ctx(ctx, "moe_sync");
  if (rc) return rc;
  MOE_HIP_CHECK(hipStreamSynchronize(ctx->stream));
  MOE_HIP_CHECK(hipGetLastError());
  return MOE_OK;
}

// ---------------------------------------------------------------- checks

#define REQUIRE(cond, msg)                                   \
  do {                                                       \
    if (!(cond)) return moe_fail(MOE_INVALID_ARGUMENT, msg); \
  } while (0)

static std::string S(long v) { return std::to_string(v); }

// topk needs at least k columns; the expert ops take any route, including
// one that names an expert twice (fewer experts than slots).
static int check_k(const char *op, int k, int E, bool need_k_columns) {
  REQUIRE(k >= 1 && k <= MAX_K, std::string(op) + ": k must be in 1.." + S(MAX_K) + ", got " + S(k));
  if (need_k_columns)
    REQUIRE(E >= k, std::string(op) + ": need at least " + S(k) + " columns, got " + S(E));
  REQUIRE(E >= 1, std::string(op) + ": need at least one expert");
  return MOE_OK;
}

// checkExpertWeight (src/core/graph/ops/matmul.ts:274-315).
static int check_weight(const char *op, const moe_expert_weight *w, int K, int N, int E, int bits,
                        int g) {
  std::string o(op);
  REQUIRE(bits == 8 || bits == 4, o + ": bits must be 8 or 4, got " + S(bits));
  REQUIRE(w && w->w, o + ": w must be a quantW [E·" + S(K) + ", N] weight");
  REQUIRE(K % 4 == 0 && N % 4 == 0,
          o + ": K " + S(K) + " and N " + S(N) + " must be multiples of 4");
  REQUIRE(g > 0 && g % 4 == 0 && K % g == 0,
          o + ": groupSize " + S(g) + " must be a multiple of 4 that divides K " + S(K));
  REQUIRE(w->scales, o + ": scales must be f32 [" + S((long)E * K / g) + ", " + S(N) + "]");
  REQUIRE(E >= 1 && E <= 1024, o + ": expert count must be in 1..1024, got " + S(E));
  return MOE_OK;
}

// ------------------------------------------------------------- workspace

struct LayerWs {
  DispatchBufs db;
  float *route = nullptr;
  float *partial = nullptr;
  float *act = nullptr;
  float *y = nullptr;
  void *xn = nullptr;  // normalised input of moe_block
};

// Workspace for `calls` calls over T tokens each (A = T·k assignments per
// call). Sections that a call does not need have size 0.
// A workspace given instead of the context's (the allocation-free entry
// point): base and size; base NULL means the context workspace.
struct FixedWs {
  char *base = nullptr;
  size_t size = 0;
  const char *op = "";
};

static int plan_ws(moe_ctx *ctx, int calls, int T, int k, int E, size_t route_floats,
                   size_t partial_floats, size_t act_floats, size_t y_floats, LayerWs &L,
                   size_t xn_bytes = 0, const FixedWs *fixed = nullptr) {
  const int A = T * k;
  const int nblk = (A + DISPATCH_TILE - 1) / DISPATCH_TILE;
  const size_t C = (size_t)calls;
  WsPlan p;
  size_t o_cnt = p.take(sizeof(int32_t) * C * nblk * E);
  size_t o_base = p.take(sizeof(int32_t) * C * nblk * E);
  size_t o_off = p.take(sizeof(int32_t) * C * (E + 1));
  size_t o_toff = p.take(sizeof(int32_t) * C * (E + 1));
  size_t o_act_list = p.take(sizeof(int32_t) * C * 4 * E);
  size_t o_meta = p.take(sizeof(int32_t) * C * META_N);
  size_t o_perm = p.take(sizeof(int32_t) * C * A);
  size_t o_route = p.take(sizeof(float) * C * route_floats);
  size_t o_part = p.take(sizeof(float) * C * partial_floats);
  size_t o_actv = p.take(sizeof(float) * C * act_floats);
  size_t o_y = p.take(sizeof(float) * C * y_floats);
  size_t o_xn = p.take(C * xn_bytes);
  char *b = nullptr;
  if (fixed && fixed->base) {
    if (p.off > fixed->size)
      return moe_fail(MOE_INVALID_ARGUMENT,
                      std::string(fixed->op) + ": needs " + std::to_string(p.off) +
                          " bytes of workspace; the static scratch holds " +
                          std::to_string(fixed->size));
    b = fixed->base;
  } else {
    int rc = moe_ws_ensure(ctx, p.off);
    if (rc) return rc;
    b = ctx->ws;
  }
  L.db.blk_counts = (int32_t *)(b + o_cnt);
  L.db.blk_base = (int32_t *)(b + o_base);
  L.db.offsets = (int32_t *)(b + o_off);
  L.db.tile_off = (int32_t *)(b + o_toff);
  L.db.active = (int32_t *)(b + o_act_list);
  L.db.meta = (int32_t *)(b + o_meta);
  L.db.perm = (int32_t *)(b + o_perm);
  L.db.E = E;
  L.db.A = A;
  L.db.nblk = nblk;
  L.route = route_floats ? (float *)(b + o_route) : nullptr;
  L.partial = partial_floats ? (float *)(b + o_part) : nullptr;
  L.act = act_floats ? (float *)(b + o_actv) : nullptr;
  L.y = y_floats ? (float *)(b + o_y) : nullptr;
  L.xn = xn_bytes ? (void *)(b + o_xn) : nullptr;
  return MOE_OK;
}

static constexpr int TILE_M = GEMM_TILE_M;

static int after_launch(const char *op) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return moe_fail(MOE_EXECUTION_FAILED, std::string(op) + ": launch failed: " + hipGetErrorString(e));
  return MOE_OK;
}

static int router_partial_floats(int T, int d, int E) {
  return T * ((d + ROUTER_CHUNK - 1) / ROUTER_CHUNK) * E;
}

// ------------------------------------------------------------------- ops

extern "C" int moe_topk(moe_ctx *ctx, const void *logits, moe_dtype dtype, int T, int E, int k,
                        float *route) {
  int rc = check_ctx(ctx, "topk");
  if (rc) return rc;
  if ((rc = check_k("topk", k, E, true))) return rc;
  REQUIRE(T >= 1, "topk: T must be at least 1, got " + S(T));
  REQUIRE(E <= TOPK_MAX_E, "topk: more than " + S(TOPK_MAX_E) + " columns");
  REQUIRE(logits && route, "topk: NULL tensor");
  REQUIRE(dtype == MOE_F32 || dtype == MOE_F16, "topk: dtype must be f32 or f16");
  {
    ProfScope ps(ctx, PG_TOPK);
    if ((rc = launch_topk(logits, dtype, T, E, k, route, ctx->stream))) return rc;
  }
  return after_launch("topk");
}

extern "C" int moe_router_topk(moe_ctx *ctx, const void *x, moe_dtype x_dtype,
                               const float *w_router, const float *b_router, int T, int d, int E,
                               int k, float *route) {
  int rc = check_ctx(ctx, "router_topk");
  if (rc) return rc;
  if ((rc = check_k("router_topk", k, E, true))) return rc;
  REQUIRE(T >= 1 && d >= 1, "router_topk: T and d must be positive");
  REQUIRE(E <= ROUTER_MAX_E, "router_topk: more than " + S(ROUTER_MAX_E) + " experts");
  REQUIRE(x && w_router && route, "router_topk: NULL tensor");
  LayerWs L;
  if ((rc = plan_ws(ctx, 1, T, k, E, 0, router_partial_floats(T, d, E), 0, 0, L))) return rc;
  RouterArgs ra{x, x_dtype, 0, w_router, 0, b_router, 0, route, 0, L.partial, T, d, E, k, 1};
  {
    ProfScope ps(ctx, PG_ROUTER);
    if ((rc = launch_router_topk(ra, nullptr, TILE_M, nullptr, ctx->stream))) return rc;
  }
  return after_launch("router_topk");
}

extern "C" int moe_dispatch(moe_ctx *ctx, const float *route, int T, int E, int k, int32_t *perm,
                            int32_t *offsets) {
  int rc = check_ctx(ctx, "dispatch");
  if (rc) return rc;
  if ((rc = check_k("dispatch", k, E, false))) return rc;
  REQUIRE(T >= 1 && E <= DISPATCH_MAX_E, "dispatch: T >= 1 and E <= 1024 required");
  LayerWs L;
  if ((rc = plan_ws(ctx, 1, T, k, E, 0, 0, 0, 0, L))) return rc;
  {
    ProfScope ps(ctx, PG_DISPATCH);
    if ((rc = launch_dispatch(route, 0, T, E, k, 1, TILE_M, L.db, ctx->stream))) return rc;
  }
  if (perm)
    MOE_HIP_CHECK(hipMemcpyAsync(perm, L.db.perm, sizeof(int32_t) * (size_t)T * k,
                                 hipMemcpyDeviceToDevice, ctx->stream));
  if (offsets)
    MOE_HIP_CHECK(hipMemcpyAsync(offsets, L.db.offsets, sizeof(int32_t) * (E + 1),
                                 hipMemcpyDeviceToDevice, ctx->stream));
  return after_launch("dispatch");
}

extern "C" int moe_pack_quantw(moe_ctx *ctx, const int8_t *ints, int E, int k, int n, int bits,
                               uint32_t *words) {
  int rc = check_ctx(ctx, "packQuantW");
  if (rc) return rc;
  REQUIRE(bits == 8 || bits == 4, "packQuantW: bits must be 8 or 4");
  REQUIRE(E >= 1 && k >= 4 && n >= 4 && k % 4 == 0 && n % 4 == 0,
          "packQuantW: E >= 1 and k, n positive multiples of 4 required");
  REQUIRE(ints && words, "packQuantW: NULL tensor");
  if ((rc = launch_pack_quantw(ints, E, k, n, bits, words, ctx->stream))) return rc;
  return after_launch("packQuantW");
}

extern "C" int moe_up(moe_ctx *ctx, const void *x, moe_dtype x_dtype, const float *route,
                      const moe_expert_weight *glu, const moe_expert_weight *lin, int T, int K,
                      int N, int E, int k, int bits, int group_size, float *act) {
  int rc = check_ctx(ctx, "moeUp");
  if (rc) return rc;
  if ((rc = check_k("moeUp", k, E, false))) return rc;
  if ((rc = check_weight("moeUp", glu, K, N, E, bits, group_size))) return rc;
  if ((rc = check_weight("moeUp", lin, K, N, E, bits, group_size))) return rc;
  REQUIRE(T >= 1, "moeUp: T must be at least 1");
  REQUIRE(x && route && act, "moeUp: NULL tensor");
  LayerWs L;
  if ((rc = plan_ws(ctx, 1, T, k, E, 0, 0, 0, 0, L))) return rc;
  {
    ProfScope ps(ctx, PG_DISPATCH);
    if ((rc = launch_dispatch(route, 0, T, E, k, 1, TILE_M, L.db, ctx->stream))) return rc;
  }
  // Rows of ids that are not experts stay zero (the reference leaves them
  // undefined).
  if ((rc = launch_zero(act, (size_t)T * k * N, ctx->stream))) return rc;
  ExpertArgs ea{};
  ea.mode = MODE_UP;
  ea.a = x;
  ea.a_dtype = x_dtype;
  ea.a_row_div = k;
  ea.route = route;
  ea.k = k;
  ea.w0 = *glu;
  ea.w1 = *lin;
  ea.K = K;
  ea.N = N;
  ea.E = E;
  ea.bits = bits;
  ea.g = group_size;
  ea.out = act;
  ea.A = T * k;
  ea.calls = 1;
  {
    ProfScope ps(ctx, PG_UP);
    if ((rc = launch_expert(ea, L.db, ctx->stream))) return rc;
  }
  return after_launch("moeUp");
}

extern "C" int moe_down(moe_ctx *ctx, const float *act, const float *route,
                        const moe_expert_weight *down, const float *residual, int T, int K, int N,
                        int E, int k, int bits, int group_size, float *out) {
  int rc = check_ctx(ctx, "moeDown");
  if (rc) return rc;
  if ((rc = check_k("moeDown", k, E, false))) return rc;
  if ((rc = check_weight("moeDown", down, K, N, E, bits, group_size))) return rc;
  REQUIRE(T >= 1, "moeDown: T must be at least 1");
  REQUIRE(act && route && out, "moeDown: NULL tensor");
  ExpertArgs ea{};
  ea.mode = MODE_DOWN;
  ea.a = act;
  ea.a_dtype = MOE_F32;
  ea.a_row_div = 1;
  ea.route = route;
  ea.k = k;
  ea.w0 = *down;
  ea.K = K;
  ea.N = N;
  ea.E = E;
  ea.bits = bits;
  ea.g = group_size;
  ea.A = T * k;
  ea.calls = 1;
  ea.parts = expert_uses_gemm(ea) ? gemm_down_parts(ea) : 1;
  LayerWs L;
  if ((rc = plan_ws(ctx, 1, T, k, E, 0, 0, 0, (size_t)ea.parts * T * k * N, L))) return rc;
  ea.out = L.y;
  {
    ProfScope ps(ctx, PG_DISPATCH);
    if ((rc = launch_dispatch(route, 0, T, E, k, 1, TILE_M, L.db, ctx->stream))) return rc;
  }
  {
    ProfScope ps(ctx, PG_DOWN);
    if ((rc = launch_expert(ea, L.db, ctx->stream))) return rc;
  }
  {
    ProfScope ps(ctx, PG_COMBINE);
    if ((rc = launch_combine(L.y, 0, ea.parts, (int64_t)T * k * N, route, 0, residual, MOE_F32, 0,
                             T, N, E, k, out, 0, 1, ctx->stream)))
      return rc;
  }
  return after_launch("moeDown");
}

static const moe_call_strides kZeroStrides = {};

// The block's pre-norm: xn = rmsNorm(x, weight, eps) over whole rows.
struct PreNorm {
  const void *weight;  // [d], x's dtype
  float eps;
};

// The routed layer (moe_layer_batched), optionally behind the block's
// pre-norm (moe_block: one call). The residual is f32 or f16.
static int layer_impl(const char *op, moe_ctx *ctx, int calls, const moe_call_strides *st,
                      const void *x, moe_dtype x_dtype, const PreNorm *norm,
                      const float *w_router, const float *b_router, const moe_expert_weight *glu,
                      const moe_expert_weight *lin, const moe_expert_weight *down,
                      const void *residual, moe_dtype res_dtype, int T, int d, int I, int E,
                      int k, int bits, int group_size_up, int group_size_down, float *route_out,
                      float *out, const FixedWs *fixed = nullptr) {
  const std::string o(op);
  const bool timing = !(fixed && fixed->base);
  int rc = check_ctx(ctx, op);
  if (rc) return rc;
  if ((rc = check_k(op, k, E, true))) return rc;
  if ((rc = check_weight(op, glu, d, I, E, bits, group_size_up))) return rc;
  if ((rc = check_weight(op, lin, d, I, E, bits, group_size_up))) return rc;
  if ((rc = check_weight(op, down, I, d, E, bits, group_size_down))) return rc;
  REQUIRE(T >= 1, o + ": T must be at least 1");
  REQUIRE(calls >= 1 && calls <= 65535, o + ": calls must be in 1..65535, got " + S(calls));
  REQUIRE(E <= ROUTER_MAX_E, o + ": more than " + S(ROUTER_MAX_E) + " experts");
  REQUIRE(x && w_router && out, o + ": NULL tensor");
  REQUIRE(x_dtype == MOE_F32 || x_dtype == MOE_F16, o + ": x must be f32 or f16");
  REQUIRE(!norm || calls == 1, o + ": the pre-norm runs one call at a time");
  if (!st) st = &kZeroStrides;
  if (calls > 1)
    REQUIRE(st->x != 0 && st->out != 0 && (!route_out || st->route != 0),
            "moe_layer: calls > 1 need distinct x, out and route_out (non-zero strides)");
  const int A = T * k;
  // Expert products first (without buffers), so the workspace is sized for
  // the path they take.
  ExpertArgs up{};
  up.mode = MODE_UP;
  up.a = x;
  up.a_dtype = x_dtype;
  up.a_cs = st->x;
  up.a_row_div = k;
  up.k = k;
  up.w0 = *glu;
  up.w1 = *lin;
  up.w0_cs = st->glu_w;
  up.s0_cs = st->glu_scales;
  up.b0_cs = st->glu_bias;
  up.w1_cs = st->lin_w;
  up.s1_cs = st->lin_scales;
  up.b1_cs = st->lin_bias;
  up.K = d;
  up.N = I;
  up.E = E;
  up.bits = bits;
  up.g = group_size_up;
  up.out_cs = (int64_t)A * I;
  up.A = A;
  up.calls = calls;
  ExpertArgs dn{};
  dn.mode = MODE_DOWN;
  dn.a_dtype = MOE_F32;
  dn.a_cs = (int64_t)A * I;
  dn.a_row_div = 1;
  dn.k = k;
  dn.w0 = *down;
  dn.w0_cs = st->down_w;
  dn.s0_cs = st->down_scales;
  dn.b0_cs = st->down_bias;
  dn.K = I;
  dn.N = d;
  dn.E = E;
  dn.bits = bits;
  dn.g = group_size_down;
  dn.A = A;
  dn.calls = calls;
  // Both products on the grouped GEMM: act stays in dispatch order, so down
  // streams each tile's rows contiguously instead of gathering them; down
  // may split K in two partial products, which the combine adds.
  // With f16 x (the direct-weight up GEMM) act goes between them as int8
  // limbs and down runs on the int8 matrix cores, whole K (gemm_i8.hip).
  size_t act_floats = (size_t)A * I;
  if (expert_uses_gemm(up) && expert_uses_gemm(dn)) {
    up.dispatch_order = dn.dispatch_order = 1;
    if (gemm_wide_eligible(up) && gemm_i8_down_eligible(dn)) {
      up.act_i8 = dn.act_i8 = 1;
      dn.parts = 1;
      const size_t limb_floats = (size_t)((gemm_i8_act_bytes(A, E, I) + 3) / 4);
      if (limb_floats > act_floats) act_floats = limb_floats;
    } else {
      dn.parts = gemm_down_parts(dn);
    }
  } else {
    dn.parts = 1;
    // Both on the decode kernels: act in dispatch order too (f32), so down
    // stages its rows without waiting on the permutation.
    if (!expert_uses_gemm(up) && !expert_uses_gemm(dn)) up.dispatch_order = dn.dispatch_order = 1;
  }
  dn.out_cs = (int64_t)dn.parts * A * d;

  LayerWs L;
  const size_t esize = x_dtype == MOE_F16 ? 2 : 4;
  // The pre-norm: folded into the router's and the skinny gate/up kernel's
  // staging for calls of at most FUSED_T tokens (the router's chunk kernel
  // computes and leaves each token's inverse RMS in the xn slot); for larger
  // calls (the register-tiled router, whose many blocks per token tile would
  // each recompute it) and for the grouped GEMM (loads straight into LDS), a
  // normalised copy xn.
  const bool stage_norm = norm && T <= FUSED_T && expert_stages_norm(up);
  if ((rc = plan_ws(ctx, calls, T, k, E, route_out ? 0 : (size_t)T * 2 * k,
                    router_partial_floats(T, d, E), act_floats, (size_t)dn.parts * A * d, L,
                    norm ? (stage_norm ? (size_t)T * 4 : (size_t)T * d * esize) : 0, fixed)))
    return rc;
  hipStream_t s = ctx->stream;
  if (stage_norm) {
    up.a_inv = (const float *)L.xn;
    up.a_normw = norm->weight;
  } else if (norm) {
    // The router and the gate/up product read xn; the residual stays x.
    ProfScope ps(ctx, PG_NORM, timing);
    NormArgs na{x, norm->weight, nullptr, L.xn, x_dtype, T, d, d, d, norm->eps, 1.0f};
    if ((rc = launch_rmsnorm(na, s))) return rc;
    x = L.xn;
    up.a = L.xn;
  }
  float *route = route_out ? route_out : L.route;
  const int64_t route_cs = route_out ? st->route : (int64_t)T * 2 * k;
  up.route = dn.route = route;
  up.route_cs = dn.route_cs = route_cs;
  // A single single-token call: the router's fold, top-k and dispatch run
  // in the gate/up kernel's prologue, one launch fewer (27.0 → 26.1 µs per
  // call). Batched calls keep the separate fold: every gate/up block then
  // repeats its call's fold, which cost more than the launch it saves
  // (config 2's 1000 calls: gate/up 550 → 600 µs against router 68 → 56).
  const int Jr = (d + ROUTER_CHUNK - 1) / ROUTER_CHUNK;
  const bool fuse_route = T == 1 && calls == 1 && expert_fuses_route(up, Jr);
  if (fuse_route) {
    up.fr_partial = L.partial;
    up.fr_b = b_router;
    up.fr_b_cs = st->router_b;
    up.fr_J = Jr;
    up.fr_tile_m = TILE_M;
  }
  up.out = L.act;
  dn.a = L.act;
  dn.out = L.y;
  bool dispatched = false;
  {
    ProfScope ps(ctx, PG_ROUTER, timing);
    RouterArgs ra{x, x_dtype, st->x, w_router, st->router_w, b_router, st->router_b, route,
                  route_cs, L.partial, T, d, E, k, calls,
                  stage_norm ? norm->weight : nullptr, norm ? norm->eps : 0.f,
                  stage_norm ? (float *)L.xn : nullptr, fuse_route ? 1 : 0};
    if ((rc = launch_router_topk(ra, &L.db, TILE_M, &dispatched, s))) return rc;
  }
  if (!dispatched) {
    ProfScope ps(ctx, PG_DISPATCH, timing);
    if ((rc = launch_dispatch(route, route_cs, T, E, k, calls, TILE_M, L.db, s))) return rc;
  }
  {
    ProfScope ps(ctx, PG_UP, timing);
    if ((rc = launch_expert(up, L.db, s))) return rc;
  }
  {
    ProfScope ps(ctx, PG_DOWN, timing);
    if ((rc = launch_expert(dn, L.db, s))) return rc;
  }
  {
    ProfScope ps(ctx, PG_COMBINE, timing);
    if ((rc = launch_combine(L.y, dn.out_cs, dn.parts, (int64_t)A * d, route, route_cs, residual,
                             res_dtype, st->residual, T, d, E, k, out, st->out, calls, s)))
      return rc;
  }
  return after_launch(op);
}

extern "C" int moe_layer_batched(moe_ctx *ctx, int calls, const moe_call_strides *st,
                                 const void *x, moe_dtype x_dtype, const float *w_router,
                                 const float *b_router, const moe_expert_weight *glu,
                                 const moe_expert_weight *lin, const moe_expert_weight *down,
                                 const float *residual, int T, int d, int I, int E, int k,
                                 int bits, int group_size_up, int group_size_down,
                                 float *route_out, float *out) {
  return layer_impl("moe_layer", ctx, calls, st, x, x_dtype, nullptr, w_router, b_router, glu,
                    lin, down, residual, MOE_F32, T, d, I, E, k, bits, group_size_up,
                    group_size_down, route_out, out);
}

extern "C" int moe_layer_noalloc(moe_ctx *ctx, const void *x, moe_dtype x_dtype,
                                 const float *w_router, const float *b_router,
                                 const moe_expert_weight *glu, const moe_expert_weight *lin,
                                 const moe_expert_weight *down, const float *residual, int T,
                                 int d, int I, int E, int k, int bits, int group_size_up,
                                 int group_size_down, float *route_out, float *out) {
  int rc = check_ctx(ctx, "moe_layer_noalloc");
  if (rc) return rc;
  hipError_t e = hipSuccess;
  char *base = scratch_on(ctx->device, &e);
  if (!base)
    return moe_fail(MOE_EXECUTION_FAILED, std::string("moe_layer_noalloc: no scratch address on "
                                                      "device ") + std::to_string(ctx->device) +
                                              ": " + hipGetErrorString(e));
  std::string why;
  if (!scratch_claim(ctx, &why)) return moe_fail(MOE_INVALID_ARGUMENT, "moe_layer_noalloc: " + why);
  FixedWs fixed;
  fixed.base = base;
  fixed.size = MOE_NOALLOC_SCRATCH_BYTES;
  fixed.op = "moe_layer_noalloc";
  return layer_impl("moe_layer_noalloc", ctx, 1, nullptr, x, x_dtype, nullptr, w_router, b_router,
                    glu, lin, down, residual, MOE_F32, T, d, I, E, k, bits, group_size_up,
                    group_size_down, route_out, out, &fixed);
}

extern "C" int moe_block(moe_ctx *ctx, const void *x, moe_dtype x_dtype, const void *norm_w,
                         float eps, const float *w_router, const float *b_router,
                         const moe_expert_weight *glu, const moe_expert_weight *lin,
                         const moe_expert_weight *down, int T, int d, int I, int E, int k,
                         int bits, int group_size_up, int group_size_down, float *route_out,
                         float *out) {
  REQUIRE(norm_w, "moe_block: NULL norm weight");
  REQUIRE(eps > 0.f, "moe_block: eps must be positive, got " + std::to_string(eps));
  const PreNorm norm{norm_w, eps};
  return layer_impl("moe_block", ctx, 1, nullptr, x, x_dtype, &norm, w_router, b_router, glu,
                    lin, down, x, x_dtype, T, d, I, E, k, bits, group_size_up, group_size_down,
                    route_out, out);
}

extern "C" int moe_matmul_gather(moe_ctx *ctx, const void *a, moe_dtype dtype, const void *w,
                                 const void *bias, const float *expert_idx, int M, int K, int N,
                                 int E, void *out) {
  int rc = check_ctx(ctx, "matmulGather");
  if (rc) return rc;
  REQUIRE(dtype == MOE_F32 || dtype == MOE_F16, "matmulGather: dtype must be f32 or f16");
  REQUIRE(M >= 1 && K >= 1 && N >= 1 && E >= 1, "matmulGather: sizes must be positive");
  REQUIRE(N % 4 == 0, "matmulGather: n " + S(N) + " must be divisible by 4");
  REQUIRE(E <= DISPATCH_MAX_E, "matmulGather: more than " + S(DISPATCH_MAX_E) + " experts");
  REQUIRE(a && w && expert_idx && out, "matmulGather: NULL tensor");
  LayerWs L;
  if ((rc = plan_ws(ctx, 1, M, 1, E, (size_t)M * 2, 0, 0, 0, L))) return rc;
  hipStream_t s = ctx->stream;
  {
    ProfScope ps(ctx, PG_DISPATCH);
    if ((rc = launch_idx_route(expert_idx, M, L.route, s))) return rc;
    if ((rc = launch_dispatch(L.route, 0, M, E, 1, 1, TILE_M, L.db, s))) return rc;
  }
  {
    ProfScope ps(ctx, PG_DOWN);
    // Rows whose index is not an expert stay zero (the reference reads
    // past w for them).
    if ((rc = launch_zero((float *)out, (size_t)M * N * (dtype == MOE_F16 ? 2 : 4) / 4, s)))
      return rc;
    FloatArgs fa{};
    fa.a = a;
    fa.a_row_div = 1;
    fa.w0 = w;
    fa.b0 = bias;
    fa.K = K;
    fa.N = N;
    fa.out = out;
    fa.db = L.db;
    if ((rc = launch_float_expert(fa, MODE_DOWN, dtype, dtype, dtype, M < E ? M : E, 1, s)))
      return rc;
  }
  return after_launch("matmulGather");
}

extern "C" int moe_block_float(moe_ctx *ctx, const void *x, moe_dtype dtype, const void *norm_w,
                               float eps, const float *w_router, const float *b_router,
                               const void *glu_w, const void *glu_b, const void *lin_w,
                               const void *lin_b, const void *out_w, const void *out_b, int T,
                               int d, int I, int E, int k, float *route_out, float *out) {
  int rc = check_ctx(ctx, "moe_block_float");
  if (rc) return rc;
  if ((rc = check_k("moe_block_float", k, E, true))) return rc;
  REQUIRE(dtype == MOE_F32 || dtype == MOE_F16, "moe_block_float: dtype must be f32 or f16");
  REQUIRE(T >= 1 && d >= 1 && I >= 1, "moe_block_float: sizes must be positive");
  REQUIRE(d % 4 == 0 && I % 4 == 0,
          "moe_block_float: d " + S(d) + " and I " + S(I) + " must be multiples of 4");
  REQUIRE(E <= ROUTER_MAX_E, "moe_block_float: more than " + S(ROUTER_MAX_E) + " experts");
  REQUIRE(x && norm_w && w_router && glu_w && lin_w && out_w && out,
          "moe_block_float: NULL tensor");
  REQUIRE(eps > 0.f, "moe_block_float: eps must be positive, got " + std::to_string(eps));
  const int A = T * k;
  const size_t esize = dtype == MOE_F16 ? 2 : 4;
  LayerWs L;
  if ((rc = plan_ws(ctx, 1, T, k, E, route_out ? 0 : (size_t)T * 2 * k,
                    router_partial_floats(T, d, E), (size_t)A * I, (size_t)A * d, L,
                    (size_t)T * d * esize)))
    return rc;
  float *route = route_out ? route_out : L.route;
  hipStream_t s = ctx->stream;
  {
    ProfScope ps(ctx, PG_NORM);
    NormArgs na{x, norm_w, nullptr, L.xn, dtype, T, d, d, d, eps, 1.0f};
    if ((rc = launch_rmsnorm(na, s))) return rc;
  }
  bool dispatched = false;
  {
    ProfScope ps(ctx, PG_ROUTER);
    RouterArgs ra{L.xn, dtype, 0, w_router, 0, b_router, 0, route, 0, L.partial, T, d, E, k, 1};
    if ((rc = launch_router_topk(ra, &L.db, TILE_M, &dispatched, s))) return rc;
  }
  if (!dispatched) {
    ProfScope ps(ctx, PG_DISPATCH);
    if ((rc = launch_dispatch(route, 0, T, E, k, 1, TILE_M, L.db, s))) return rc;
  }
  const int max_active = A < E ? A : E;
  {
    ProfScope ps(ctx, PG_UP);
    FloatArgs fa{};
    fa.a = L.xn;
    fa.a_row_div = k;
    fa.w0 = glu_w;
    fa.b0 = glu_b;
    fa.w1 = lin_w;
    fa.b1 = lin_b;
    fa.K = d;
    fa.N = I;
    fa.out = L.act;
    fa.db = L.db;
    if ((rc = launch_float_expert(fa, MODE_UP, dtype, dtype, MOE_F32, max_active, 1, s))) return rc;
  }
  {
    ProfScope ps(ctx, PG_DOWN);
    FloatArgs fa{};
    fa.a = L.act;
    fa.a_row_div = 1;
    fa.w0 = out_w;
    fa.b0 = out_b;
    fa.K = I;
    fa.N = d;
    fa.out = L.y;
    fa.db = L.db;
    if ((rc = launch_float_expert(fa, MODE_DOWN, MOE_F32, dtype, MOE_F32, max_active, 1, s)))
      return rc;
  }
  {
    ProfScope ps(ctx, PG_COMBINE);
    if ((rc = launch_combine(L.y, 0, 1, (int64_t)A * d, route, 0, x, dtype, 0, T, d, E, k, out, 0,
                             1, s)))
      return rc;
  }
  return after_launch("moe_block_float");
}

extern "C" int moe_rmsnorm(moe_ctx *ctx, const void *x, moe_dtype dtype, int rows, int cols,
                           const void *weight, int weight_len, float eps, int group,
                           const void *residual, float scale, void *out) {
  int rc = check_ctx(ctx, "rmsNorm");
  if (rc) return rc;
  REQUIRE(dtype == MOE_F32 || dtype == MOE_F16, "rmsNorm: dtype must be f32 or f16");
  REQUIRE(rows >= 1 && cols >= 1, "rmsNorm: rows and cols must be positive");
  REQUIRE(group >= 1 && cols % group == 0,
          "rmsNorm: group " + S(group) + " must divide the row width " + S(cols));
  REQUIRE(weight_len == group || weight_len == cols,
          "rmsNorm: weight must be " + std::string(dtype == MOE_F16 ? "f16" : "f32") + " with " +
              (group == cols ? S(cols) : S(group) + " or " + S(cols)) + " elems, got (" +
              S(weight_len) + ")");
  REQUIRE(eps > 0.f, "rmsNorm: eps must be positive, got " + std::to_string(eps));
  REQUIRE(x && weight && out, "rmsNorm: NULL tensor");
  {
    ProfScope ps(ctx, PG_NORM);
    NormArgs na{x, weight, residual, out, dtype, rows, cols, group, weight_len, eps, scale};
    if ((rc = launch_rmsnorm(na, ctx->stream))) return rc;
  }
  return after_launch("rmsNorm");
}

extern "C" int moe_linear(moe_ctx *ctx, const float *x, const float *w, const float *bias,
                          const float *addend, int T, int K, int N, float *out) {
  int rc = check_ctx(ctx, "linear");
  if (rc) return rc;
  REQUIRE(T >= 1 && K >= 1 && N >= 1, "linear: T, K and N must be positive");
  REQUIRE(x && w && out, "linear: NULL tensor");
  if ((rc = moe_ws_ensure(ctx, linear_ws_bytes(T, K, N)))) return rc;
  if ((rc = launch_linear(x, w, bias, addend, out, (float *)ctx->ws, T, K, N, ctx->stream)))
    return rc;
  return after_launch("linear");
}

extern "C" int moe_attention(moe_ctx *ctx, const void *qkv, moe_dtype dtype, int T, int q_heads,
                             int kv_heads, int head_dim, int64_t window_left,
                             int64_t window_right, const float *sinks, const float *cos_t,
                             const float *sin_t, void *out) {
  int rc = check_ctx(ctx, "attention");
  if (rc) return rc;
  REQUIRE(dtype == MOE_F32 || dtype == MOE_F16, "attention: dtype must be f32 or f16");
  REQUIRE(T >= 1, "attention: T must be positive");
  REQUIRE(kv_heads > 0 && q_heads > 0 && q_heads % kv_heads == 0,
          "attention: qHeads " + S(q_heads) + " not divisible by kvHeads " + S(kv_heads));
  REQUIRE(head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 128,
          "attention: headDim " + S(head_dim) + " must be even and at most 128");
  REQUIRE(qkv && cos_t && sin_t && out, "attention: NULL tensor");
  const int64_t width = (int64_t)(q_heads + 2 * kv_heads) * head_dim;
  const size_t es = dtype == MOE_F16 ? 2 : 4;
  AttnArgs a{};
  a.q = qkv;
  a.k = (const char *)qkv + (size_t)q_heads * head_dim * es;
  a.v = (const char *)qkv + (size_t)(q_heads + kv_heads) * head_dim * es;
  a.q_rs = a.k_rs = a.v_rs = width;
  a.out = out;
  a.o_rs = (int64_t)q_heads * head_dim;
  a.dtype = dtype;
  a.q_len = a.kv_len = T;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.head_dim = head_dim;
  a.window_left = window_left < 0 ? -1 : window_left;
  a.window_right = window_right < 0 ? -1 : window_right;
  a.sinks = sinks;
  a.rope_cos = cos_t;
  a.rope_sin = sin_t;
  if ((rc = launch_sdpa(a, ctx->stream))) return rc;
  return after_launch("attention");
}

extern "C" int moe_rope(moe_ctx *ctx, const void *x, moe_dtype dtype, int rows, int cols,
                        int head_dim, int src_start, int width, const float *cos_t,
                        const float *sin_t, void *out) {
  int rc = check_ctx(ctx, "rope");
  if (rc) return rc;
  REQUIRE(dtype == MOE_F32 || dtype == MOE_F16, "rope: dtype must be f32 or f16");
  REQUIRE(rows >= 1 && cols >= 1, "rope: rows and cols must be positive");
  REQUIRE(head_dim > 0 && head_dim % 2 == 0,
          "rope: headDim " + S(head_dim) + " must be a positive even integer");
  REQUIRE(src_start >= 0 && src_start % 2 == 0,
          "rope: srcStart " + S(src_start) + " must be a non-negative even integer");
  REQUIRE(width > 0 && (int64_t)src_start + width <= cols,
          "rope: window [" + S(src_start) + ", " + S(src_start + width) + ") exceeds " + S(cols) +
              " input cols");
  REQUIRE(width % head_dim == 0,
          "rope: width " + S(width) + " must be a multiple of headDim " + S(head_dim));
  REQUIRE(x && cos_t && sin_t && out, "rope: NULL tensor");
  if ((rc = launch_rope(x, dtype, rows, cols, head_dim, src_start, width, cos_t, sin_t, out,
                        ctx->stream)))
    return rc;
  return after_launch("rope");
}

extern "C" int moe_sdpa(moe_ctx *ctx, moe_dtype dtype, const void *q, int64_t q_stride,
                        const void *k, int64_t k_stride, const void *v, int64_t v_stride,
                        int q_len, int kv_len, int q_heads, int kv_heads, int head_dim,
                        int64_t window_left, int64_t window_right, int q_pos_offset,
                        const float *sinks, const float *segments, int key_bias,
                        int key_bias_start, int key_bias_end, float key_bias_value, void *out) {
  int rc = check_ctx(ctx, "sdpa");
  if (rc) return rc;
  REQUIRE(dtype == MOE_F32 || dtype == MOE_F16, "sdpa: dtype must be f32 or f16");
  REQUIRE(q_len >= 1 && kv_len >= 1, "sdpa: qLen and kvLen must be positive");
  REQUIRE(kv_heads > 0 && q_heads > 0 && q_heads % kv_heads == 0,
          "sdpa: qHeads " + S(q_heads) + " not divisible by kvHeads " + S(kv_heads));
  REQUIRE(head_dim >= 1, "sdpa: headDim must be positive");
  REQUIRE(head_dim <= 128, "sdpa: headDim " + S(head_dim) + " exceeds the kernel's max (128)");
  REQUIRE(q_pos_offset >= 0,
          "sdpa: qPosOffset " + S(q_pos_offset) + " must be a non-negative integer");
  REQUIRE(window_right < 0 || (int64_t)q_pos_offset + q_len <= kv_len,
          "sdpa: qPosOffset+qLen " + S(q_pos_offset + q_len) + " exceeds key rows kvLen " +
              S(kv_len));
  REQUIRE(q_stride >= (int64_t)q_heads * head_dim && k_stride >= (int64_t)kv_heads * head_dim &&
              v_stride >= (int64_t)kv_heads * head_dim,
          "sdpa: a row stride is shorter than its heads");
  if (key_bias)
    REQUIRE(key_bias_start >= 0 && key_bias_start <= key_bias_end && key_bias_end <= kv_len,
            "sdpa: keyBias keys [" + S(key_bias_start) + ", " + S(key_bias_end) +
                ") must lie within the " + S(kv_len) + " keys");
  REQUIRE(q && k && v && out, "sdpa: NULL tensor");
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.q_rs = q_stride;
  a.k_rs = k_stride;
  a.v_rs = v_stride;
  a.out = out;
  a.o_rs = (int64_t)q_heads * head_dim;
  a.dtype = dtype;
  a.q_len = q_len;
  a.kv_len = kv_len;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.head_dim = head_dim;
  a.window_left = window_left < 0 ? -1 : window_left;
  a.window_right = window_right < 0 ? -1 : window_right;
  a.q_pos_offset = q_pos_offset;
  a.sinks = sinks;
  a.segs = segments;
  a.has_kb = key_bias ? 1 : 0;
  a.kb_start = key_bias_start;
  a.kb_end = key_bias_end;
  a.kb_value = key_bias_value;
  if ((rc = launch_sdpa(a, ctx->stream))) return rc;
  return after_launch("sdpa");
}

extern "C" int moe_layer(moe_ctx *ctx, const void *x, moe_dtype x_dtype, const float *w_router,
                         const float *b_router, const moe_expert_weight *glu,
                         const moe_expert_weight *lin, const moe_expert_weight *down,
                         const float *residual, int T, int d, int I, int E, int k, int bits,
                         int group_size_up, int group_size_down, float *route_out, float *out) {
  return moe_layer_batched(ctx, 1, nullptr, x, x_dtype, w_router, b_router, glu, lin, down,
                           residual, T, d, I, E, k, bits, group_size_up, group_size_down,
                           route_out, out);
}

extern "C" int moe_ctx_reserve(moe_ctx *ctx, int T, int d, int I, int E, int k) {
  return moe_ctx_reserve_batched(ctx, 1, T, d, I, E, k);
}

extern "C" int moe_ctx_reserve_batched(moe_ctx *ctx, int calls, int T, int d, int I, int E,
                                       int k) {
  int rc = check_ctx(ctx, "moe_ctx_reserve");
  if (rc) return rc;
  REQUIRE(calls >= 1 && T >= 1 && d >= 1 && I >= 1 && E >= 1 && k >= 1,
          "moe_ctx_reserve: sizes must be positive");
  LayerWs L;
  // y: room for down's two K parts (the grouped GEMM may split K).
  // act: room for the int8-limb form over padded rows (gemm_i8.hip).
  size_t act_floats = (size_t)T * k * I;
  const size_t limb_floats = (size_t)((gemm_i8_act_bytes(T * k, E, I) + 3) / 4);
  if (limb_floats > act_floats) act_floats = limb_floats;
  return plan_ws(ctx, calls, T, k, E, (size_t)T * 2 * k, router_partial_floats(T, d, E),
                 act_floats, (size_t)2 * T * k * (d > I ? d : I), L);
}

// ------------------------------------------------------------ weight upload

// An expert weight owned by the library (QuantExpertWeight's three device
// buffers). After moe_weights_dispose the handle stays valid and reports
// RESOURCE_DISPOSED until moe_weights_release frees it.
struct moe_weights {
  int device = 0;
  bool disposed = false;
  uint32_t *w = nullptr;
  float *scales = nullptr;
  float *bias = nullptr;
  int E = 0, K = 0, N = 0, bits = 0, g = 0;
};

static void weights_free(moe_weights *h) {
  if (h->w) (void)hipFree(h->w);
  if (h->scales) (void)hipFree(h->scales);
  if (h->bias) (void)hipFree(h->bias);
  h->w = nullptr;
  h->scales = nullptr;
  h->bias = nullptr;
}

extern "C" int moe_weights_upload(moe_ctx *ctx, const void *host, int raw_int8,
                                  const float *scales, const float *bias, int E, int K, int N,
                                  int bits, int group_size, moe_weights **out) {
  int rc = check_ctx(ctx, "upload");
  if (rc) return rc;
  REQUIRE(out, "upload: NULL handle");
  *out = nullptr;
  REQUIRE((long)E * K * N > 0 && E > 0 && K > 0 && N > 0, "upload: the shape has no elements");
  REQUIRE(host && scales, "upload: NULL tensor");
  REQUIRE(bits == 8 || bits == 4, "upload: bits must be 8 or 4, got " + S(bits));
  REQUIRE(K % 4 == 0 && N % 4 == 0,
          "upload: K " + S(K) + " and N " + S(N) + " must be multiples of 4");
  REQUIRE(group_size > 0 && group_size % 4 == 0 && K % group_size == 0,
          "upload: groupSize " + S(group_size) + " must be a multiple of 4 that divides K " + S(K));
  REQUIRE(E <= 1024, "upload: expert count must be in 1..1024, got " + S(E));
  moe_weights *h = new moe_weights;
  h->device = ctx->device;
  h->E = E;
  h->K = K;
  h->N = N;
  h->bits = bits;
  h->g = group_size;
  const size_t words = (size_t)E * K * N * bits / 32;
  const size_t n_scales = (size_t)E * K / group_size * N;
  const size_t n_bias = (size_t)E * N;
  int8_t *tmp = nullptr;
  auto fail = [&](hipError_t e, const char *what) {
    if (tmp) (void)hipFree(tmp);
    weights_free(h);
    delete h;
    return moe_fail(MOE_EXECUTION_FAILED, std::string("upload: ") + what + ": " + hipGetErrorString(e));
  };
  hipError_t e;
  if ((e = hipMalloc(&h->w, words * 4)) != hipSuccess) return fail(e, "hipMalloc");
  if ((e = hipMalloc(&h->scales, n_scales * 4)) != hipSuccess) return fail(e, "hipMalloc");
  if (bias && (e = hipMalloc(&h->bias, n_bias * 4)) != hipSuccess) return fail(e, "hipMalloc");
  hipStream_t s = ctx->stream;
  if (raw_int8) {
    // int8 [E][N][K] (output-first per expert, one value per byte) packed
    // on the device, as packQuantW per expert, experts concatenated.
    const size_t n_ints = (size_t)E * K * N;
    if ((e = hipMalloc(&tmp, n_ints)) != hipSuccess) return fail(e, "hipMalloc");
    if ((e = hipMemcpyAsync(tmp, host, n_ints, hipMemcpyHostToDevice, s)) != hipSuccess)
      return fail(e, "hipMemcpy");
    if ((rc = launch_pack_quantw(tmp, E, K, N, bits, h->w, s))) {
      (void)hipStreamSynchronize(s);
      (void)hipFree(tmp);
      weights_free(h);
      delete h;
      return rc;
    }
  } else if ((e = hipMemcpyAsync(h->w, host, words * 4, hipMemcpyHostToDevice, s)) != hipSuccess) {
    return fail(e, "hipMemcpy");
  }
  if ((e = hipMemcpyAsync(h->scales, scales, n_scales * 4, hipMemcpyHostToDevice, s)) != hipSuccess)
    return fail(e, "hipMemcpy");
  if (bias && (e = hipMemcpyAsync(h->bias, bias, n_bias * 4, hipMemcpyHostToDevice, s)) != hipSuccess)
    return fail(e, "hipMemcpy");
  // The host buffers may be released once this returns.
  if ((e = hipStreamSynchronize(s)) != hipSuccess) return fail(e, "hipStreamSynchronize");
  if (tmp) (void)hipFree(tmp);
  *out = h;
  return MOE_OK;
}

extern "C" int moe_weights_view(const moe_weights *h, moe_expert_weight *view) {
  if (!h) return moe_fail(MOE_NOT_INITIALIZED, "weights: handle is NULL");
  if (h->disposed) return moe_fail(MOE_RESOURCE_DISPOSED, "weights: used after dispose");
  REQUIRE(view, "weights: NULL view");
  view->w = h->w;
  view->scales = h->scales;
  view->bias = h->bias;
  return MOE_OK;
}

extern "C" int moe_weights_dispose(moe_weights *h) {
  if (!h) return moe_fail(MOE_NOT_INITIALIZED, "weights: handle is NULL");
  if (h->disposed) return MOE_OK;
  (void)hipSetDevice(h->device);
  // Work already enqueued on these buffers must finish before they go.
  MOE_HIP_CHECK(hipDeviceSynchronize());
  weights_free(h);
  h->disposed = true;
  return MOE_OK;
}

extern "C" int moe_weights_release(moe_weights *h) {
  if (!h) return MOE_OK;
  int rc = moe_weights_dispose(h);
  delete h;
  return rc;
}

// ------------------------------------------------- executor plumbing (host)

// checkExpertWeight (src/core/graph/ops/matmul.ts:274-315): the same checks
// in the same order with the same messages, which callers match by regex.
extern "C" int moe_check_expert_weight(const char *op_c, const moe_value_desc *w,
                                       const moe_value_desc *scales, const moe_value_desc *bias,
                                       const moe_value_desc *route, int64_t k, int64_t t,
                                       int slots, int bits, int group_size, int64_t *n_out,
                                       int64_t *experts_out) {
  const std::string op = op_c ? op_c : "moe";
  if (!w || !scales || !bias || !route)
    return moe_fail(MOE_INVALID_ARGUMENT, op + ": NULL value descriptor");
  REQUIRE(bits == 8 || bits == 4, op + ": bits must be 8 or 4, got " + S(bits));
  REQUIRE(k > 0 && w->dtype == MOE_VALUE_QUANTW && w->rank == 2 && w->dims[0] % k == 0,
          op + ": w must be a quantW [E·" + S(k) + ", N] weight");
  const int64_t r = w->dims[0], n = w->dims[1];
  const int64_t experts = r / k;
  // (r·n·bits)/32 as the reference computes it; a fraction never matches.
  REQUIRE((r * n * bits) % 32 == 0 && w->elems == r * n * bits / 32,
          op + ": quantW weight elems " + S(w->elems) + " != rows·cols·" + S(bits) + "/32");
  REQUIRE(k % 4 == 0 && n % 4 == 0,
          op + ": K " + S(k) + " and N " + S(n) + " must be multiples of 4");
  REQUIRE(group_size > 0 && group_size % 4 == 0 && k % group_size == 0,
          op + ": groupSize " + S(group_size) + " must be a multiple of 4 that divides K " + S(k));
  REQUIRE(scales->dtype == MOE_VALUE_F32 && scales->elems == experts * k * n / group_size,
          op + ": scales must be f32 [" + S(experts * k / group_size) + ", " + S(n) + "]");
  REQUIRE(bias->dtype == MOE_VALUE_F32 && bias->elems == experts * n,
          op + ": bias must be f32 [" + S(experts) + ", " + S(n) + "]");
  REQUIRE(route->dtype == MOE_VALUE_F32 && route->rank >= 2 && route->dims[0] == t &&
              route->dims[1] == 2 * (int64_t)slots,
          op + ": route must be topk's f32 [" + S(t) + ", " + S(2 * (int64_t)slots) + "] output");
  if (n_out) *n_out = n;
  if (experts_out) *experts_out = experts;
  return MOE_OK;
}

extern "C" int moe_buffer_alloc(moe_ctx *ctx, size_t bytes, void **out) {
  int rc = check_ctx(ctx, "moe_buffer_alloc");
  if (rc) return rc;
  REQUIRE(out, "moe_buffer_alloc: out is NULL");
  REQUIRE(bytes > 0, "upload: the shape has no elements");
  *out = nullptr;
  MOE_HIP_CHECK(hipMalloc(out, bytes));
  return MOE_OK;
}

extern "C" int moe_buffer_free(moe_ctx *ctx, void *ptr) {
  int rc = check_ctx(ctx, "moe_buffer_free");
  if (rc) return rc;
  if (!ptr) return MOE_OK;
  // Work queued on the context's stream may still use the buffer.
  MOE_HIP_CHECK(hipStreamSynchronize(ctx->stream));
  MOE_HIP_CHECK(hipFree(ptr));
  return MOE_OK;
}

extern "C" int moe_buffer_write(moe_ctx *ctx, void *dst, const void *host, size_t bytes) {
  int rc = check_ctx(ctx, "moe_buffer_write");
  if (rc) return rc;
  REQUIRE(dst && host, "moe_buffer_write: NULL pointer");
  REQUIRE(bytes > 0, "upload: the shape has no elements");
  MOE_HIP_CHECK(hipMemcpyAsync(dst, host, bytes, hipMemcpyHostToDevice, ctx->stream));
  MOE_HIP_CHECK(hipStreamSynchronize(ctx->stream));
  return MOE_OK;
}

extern "C" int moe_buffer_read(moe_ctx *ctx, void *host, const void *src, size_t bytes) {
  int rc = check_ctx(ctx, "moe_buffer_read");
  if (rc) return rc;
  REQUIRE(src && host, "moe_buffer_read: NULL pointer");
  if (bytes == 0) return MOE_OK;
  MOE_HIP_CHECK(hipMemcpyAsync(host, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  MOE_HIP_CHECK(hipStreamSynchronize(ctx->stream));
  return MOE_OK;
}
