// Token dispatch for calls too large for the fused router kernel: a stable
// counting sort of assignments by expert (definition in dispatch_dev.h).
//
// Three kernels per batch of calls, all integer work:
//   k_dispatch_count   per 1024-assignment tile: LDS histogram
//   k_dispatch_scan    one block per call: offsets, M-tile offsets, active
//                      list, per-tile bases; marks unused perm slots −1
//   k_dispatch_scatter per tile: stable rank via wavefront ballots (one per id
//                      bit), then place
#include "dispatch_dev.h"

namespace {

using namespace moe_dev;
constexpr int DBLOCK = 256;

__global__ __launch_bounds__(DBLOCK) void k_dispatch_count(const float *__restrict__ route,
                                                           int64_t route_cs, int A, int k,
                                                           DispatchBufs db) {
  __shared__ int32_t hist[DISPATCH_MAX_E];
  const int call = blockIdx.y;
  const int E = db.E;
  route += call * route_cs;
  for (int e = threadIdx.x; e < E; e += DBLOCK) hist[e] = 0;
  __syncthreads();
  const int64_t a0 = (int64_t)blockIdx.x * DISPATCH_TILE;
  for (int i = threadIdx.x; i < DISPATCH_TILE; i += DBLOCK) {
    int64_t a = a0 + i;
    if (a >= A) break;
    int e = route_expert(route, a, k, E);
    if (e >= 0) atomicAdd(&hist[e], 1);
  }
  __syncthreads();
  int32_t *cnt = db.blk_counts + call * db.cnt_cs() + (int64_t)blockIdx.x * E;
  for (int e = threadIdx.x; e < E; e += DBLOCK) cnt[e] = hist[e];
}

// Block counts staged in LDS when they fit: every load is then out at once
// (summing them straight from memory waits one latency per few blocks).
constexpr int SCAN_LDS_COUNTS = 8192;

__global__ __launch_bounds__(1024) void k_dispatch_scan(DispatchBufs db, int tile_m) {
  __shared__ int32_t tot[DISPATCH_MAX_E];
  __shared__ int32_t off[DISPATCH_MAX_E + 1];
  __shared__ int32_t cl[SCAN_LDS_COUNTS];
  const int call = blockIdx.x;
  const int E = db.E, nblk = db.nblk;
  const int32_t *cnt = db.blk_counts + call * db.cnt_cs();
  const bool staged = nblk * E <= SCAN_LDS_COUNTS;
  if (staged) {
    // Up to eight counts a thread, all loaded before the first store (an
    // index past the end reloads the last count, which is not stored).
    const int n = nblk * E;
    for (int i0 = threadIdx.x; i0 < n; i0 += 8 * blockDim.x) {
      int32_t v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) v[u] = cnt[min(i0 + u * (int)blockDim.x, n - 1)];
#pragma unroll
      for (int u = 0; u < 8; u++)
        if (i0 + u * (int)blockDim.x < n) cl[i0 + u * blockDim.x] = v[u];
    }
    __syncthreads();
    cnt = cl;
  }
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int32_t c = 0;
    for (int b = 0; b < nblk; b++) c += cnt[(int64_t)b * E + e];
    tot[e] = c;
  }
  __syncthreads();
  if (threadIdx.x < WAVE)
    wave_scan_experts(tot, E, tile_m, threadIdx.x, db.offsets + call * db.off_cs(),
                      db.tile_off + call * db.off_cs(), db.active + call * db.act_cs(),
                      db.meta + call * db.meta_cs(), off);
  __syncthreads();
  int32_t *base = db.blk_base + call * db.cnt_cs();
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int32_t run = off[e];
    for (int b = 0; b < nblk; b++) {
      base[(int64_t)b * E + e] = run;
      run += cnt[(int64_t)b * E + e];
    }
  }
  int32_t *perm = db.perm + call * db.perm_cs();
  for (int i = off[E] + threadIdx.x; i < db.A; i += blockDim.x) perm[i] = -1;
}

__global__ __launch_bounds__(DBLOCK) void k_dispatch_scatter(const float *__restrict__ route,
                                                             int64_t route_cs, int A, int k,
                                                             DispatchBufs db) {
  __shared__ int32_t cursor[DISPATCH_MAX_E];
  __shared__ int32_t wc[4 * DISPATCH_MAX_E];
  const int call = blockIdx.y;
  const int E = db.E;
  route += call * route_cs;
  const int32_t *base = db.blk_base + call * db.cnt_cs() + (int64_t)blockIdx.x * E;
  for (int e = threadIdx.x; e < E; e += DBLOCK) cursor[e] = base[e];
  int32_t *perm = db.perm + call * db.perm_cs();
  const int64_t a0 = (int64_t)blockIdx.x * DISPATCH_TILE;
  for (int pass = 0; pass < DISPATCH_TILE / DBLOCK; pass++) {
    int64_t a = a0 + pass * DBLOCK + threadIdx.x;
    int e = (a < A) ? route_expert(route, a, k, E) : -1;
    block_place(e, a, E, cursor, wc, perm);
  }
}

}  // namespace

int launch_dispatch(const float *route, int64_t route_cs, int T, int E, int k, int calls,
                    int tile_m, const DispatchBufs &db, hipStream_t s) {
  MOE_NONNULL(route);
  MOE_NONNULL(db.blk_counts);
  MOE_NONNULL(db.blk_base);
  MOE_NONNULL(db.offsets);
  MOE_NONNULL(db.tile_off);
  MOE_NONNULL(db.active);
  MOE_NONNULL(db.meta);
  MOE_NONNULL(db.perm);
  if (E > DISPATCH_MAX_E) return moe_fail(MOE_INVALID_ARGUMENT, "dispatch: more than 1024 experts");
  const int A = T * k;
  if (db.E != E || db.A != A || db.nblk != (A + DISPATCH_TILE - 1) / DISPATCH_TILE)
    return moe_fail(MOE_EXECUTION_FAILED, "dispatch: workspace sized for another shape");
  hipLaunchKernelGGL(k_dispatch_count, dim3(db.nblk, calls), dim3(DBLOCK), 0, s, route, route_cs,
                     A, k, db);
  hipLaunchKernelGGL(k_dispatch_scan, dim3(calls), dim3(1024), 0, s, db, tile_m);
  hipLaunchKernelGGL(k_dispatch_scatter, dim3(db.nblk, calls), dim3(DBLOCK), 0, s, route,
                     route_cs, A, k, db);
  return 0;
}
