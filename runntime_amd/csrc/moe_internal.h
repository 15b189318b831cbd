// Internal declarations shared by the HIP translation units of libmoe.so.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

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

struct moe_ctx {
  int device = 0;
  hipStream_t stream = nullptr;      // stream the calls enqueue on
  hipStream_t own_stream = nullptr;  // created by the context
  char *ws = nullptr;                // device workspace
  size_t ws_size = 0;
  bool disposed = false;
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

// Dispatch workspace views (all device pointers).
struct DispatchBufs {
  int32_t *blk_counts;  // [nblk, E]
  int32_t *blk_base;    // [nblk, E]
  int32_t *offsets;     // [E + 1]
  int32_t *tile_off;    // [E + 1] cumulative M-tiles per expert
  int32_t *active;      // [E] ids of experts with rows, ascending
  int32_t *meta;        // [META_N]
  int32_t *perm;        // [A] sorted position → assignment
};

// ---------------------------------------------------------- launchers

// Launchers refuse NULL device pointers: a kernel must never be handed one.
#define MOE_NONNULL(ptr)                                                                  \
  do {                                                                                    \
    if (!(ptr)) return moe_fail(MOE_EXECUTION_FAILED, std::string(__func__) + ": " #ptr " is NULL"); \
  } while (0)

int launch_topk(const void *logits, moe_dtype dt, int T, int E, int k, float *route,
                hipStream_t s);
int launch_router_topk(const void *x, moe_dtype dt, const float *w, const float *b, int T, int d,
                       int E, int k, float *partial, float *route, hipStream_t s);
int launch_dispatch(const float *route, int T, int E, int k, int tile_m, const DispatchBufs &db,
                    hipStream_t s);

enum ExpertMode { MODE_UP = 0, MODE_DOWN = 1 };

struct ExpertArgs {
  int mode;                 // ExpertMode
  const void *a;            // x [T, K] (up) or act [T·k, K] (down)
  moe_dtype a_dtype;
  int a_row_div;            // source row = assignment / a_row_div (k for up, 1 for down)
  const float *route;       // [T, 2k]
  int k;
  const moe_expert_weight *w0;  // glu (up) or down
  const moe_expert_weight *w1;  // lin (up) or null
  int K, N, E, bits, g;
  float *out;               // act [T·k, N] (up) or y [T·k, N] (down), row = assignment
  int A;                    // T·k
};

int launch_expert(const ExpertArgs &ea, const DispatchBufs &db, hipStream_t s);
// Fills n floats with 0 (a kernel, not hipMemsetAsync, so a captured graph
// replays it correctly).
int launch_zero(float *p, size_t n, hipStream_t s);
int launch_combine(const float *y, const float *route, const float *residual, int T, int N, int E,
                   int k, float *out, hipStream_t s);
