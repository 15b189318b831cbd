// Token dispatch: a stable counting sort of assignments by expert.
//
// The reference has no permutation: every (token, slot) row reads its own
// expert's weights (src/core/kernels/matmul/moeQuantW.ts:131-134). Grouping
// rows by expert lets the expert kernels stream each active expert's weights
// once. The sort is defined as: assignment a = t·k + s goes to expert
// e = route[t, s]; offsets[e] = Σ_{e' < e} count(e'); within an expert the
// assignments keep ascending a. An id that is not an expert index (negative,
// ≥ E, fractional, NaN) is left out.
//
// Three kernels, all integer work, none MFMA-shaped:
//   k_dispatch_count   per 1024-assignment tile: LDS histogram
//   k_dispatch_scan    one block: tile bases, offsets, active list, M-tiles
//   k_dispatch_scatter per tile: stable rank via wavefront ballots, then place
#include "moe_internal.h"

namespace {

constexpr int WAVE = 64;
constexpr int DBLOCK = 256;

__device__ __forceinline__ int route_expert(const float *route, int64_t a, int k, int E) {
  int64_t t = a / k;
  int s = (int)(a - t * k);
  float f = route[t * 2 * k + s];
  if (!(f >= 0.f) || f >= (float)E) return -1;
  int e = (int)f;
  return ((float)e == f) ? e : -1;
}

__global__ __launch_bounds__(DBLOCK) void k_dispatch_count(const float *__restrict__ route, int A,
                                                           int k, int E,
                                                           int32_t *__restrict__ blk_counts) {
  __shared__ int32_t hist[DISPATCH_MAX_E];
  for (int e = threadIdx.x; e < E; e += DBLOCK) hist[e] = 0;
  __syncthreads();
  int64_t a0 = (int64_t)blockIdx.x * DISPATCH_TILE;
  for (int i = threadIdx.x; i < DISPATCH_TILE; i += DBLOCK) {
    int64_t a = a0 + i;
    if (a >= A) break;
    int e = route_expert(route, a, k, E);
    if (e >= 0) atomicAdd(&hist[e], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += DBLOCK) blk_counts[(int64_t)blockIdx.x * E + e] = hist[e];
}

// One block. Thread e walks the tiles for expert e; a block-wide exclusive
// scan over experts gives the offsets.
__global__ __launch_bounds__(1024) void k_dispatch_scan(const int32_t *__restrict__ blk_counts,
                                                        int nblk, int E, int tile_m,
                                                        int32_t *__restrict__ blk_base,
                                                        int32_t *__restrict__ offsets,
                                                        int32_t *__restrict__ tile_off,
                                                        int32_t *__restrict__ active,
                                                        int32_t *__restrict__ meta) {
  __shared__ int32_t tot[DISPATCH_MAX_E];
  __shared__ int32_t tiles[DISPATCH_MAX_E];
  __shared__ int32_t act[DISPATCH_MAX_E];
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int32_t c = 0;
    for (int b = 0; b < nblk; b++) c += blk_counts[(int64_t)b * E + e];
    tot[e] = c;
    tiles[e] = (c + tile_m - 1) / tile_m;
    act[e] = c > 0 ? 1 : 0;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    // Sequential scans over E ≤ a few thousand: negligible next to the rest.
    int32_t run = 0, trun = 0, na = 0, mx = 0;
    for (int e = 0; e < E; e++) {
      int32_t c = tot[e];
      offsets[e] = run;
      tile_off[e] = trun;
      run += c;
      trun += tiles[e];
      if (c > 0) active[na++] = e;
      mx = c > mx ? c : mx;
      tot[e] = offsets[e];  // reuse: base of expert e
    }
    offsets[E] = run;
    tile_off[E] = trun;
    for (int i = na; i < E; i++) active[i] = -1;
    meta[META_VALID] = run;
    meta[META_ACTIVE] = na;
    meta[META_MAXCNT] = mx;
    meta[META_TILES] = trun;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int32_t base = tot[e];
    for (int b = 0; b < nblk; b++) {
      blk_base[(int64_t)b * E + e] = base;
      base += blk_counts[(int64_t)b * E + e];
    }
  }
}

// Stable placement inside one tile. Elements are taken 256 at a time, in
// order; within a wavefront the rank among equal experts comes from ballots,
// across the block's 4 wavefronts from per-wave counts in LDS.
__global__ __launch_bounds__(DBLOCK) void k_dispatch_scatter(const float *__restrict__ route, int A,
                                                             int k, int E,
                                                             const int32_t *__restrict__ blk_base,
                                                             int32_t *__restrict__ perm) {
  __shared__ int32_t cursor[DISPATCH_MAX_E];
  __shared__ int32_t wc[4 * DISPATCH_MAX_E];  // per-wave counts of this pass
  int lane = threadIdx.x & (WAVE - 1);
  int wave = threadIdx.x / WAVE;
  for (int e = threadIdx.x; e < E; e += DBLOCK) cursor[e] = blk_base[(int64_t)blockIdx.x * E + e];
  int64_t a0 = (int64_t)blockIdx.x * DISPATCH_TILE;
  for (int pass = 0; pass < DISPATCH_TILE / DBLOCK; pass++) {
    for (int i = threadIdx.x; i < 4 * E; i += DBLOCK) wc[i] = 0;
    __syncthreads();
    int64_t a = a0 + pass * DBLOCK + threadIdx.x;
    int e = (a < A) ? route_expert(route, a, k, E) : -1;
    // Rank among earlier lanes of this wavefront with the same expert.
    uint64_t pending = __ballot(e >= 0);
    int rank = 0;
    while (pending) {
      int leader = __ffsll((unsigned long long)pending) - 1;
      int el = __shfl(e, leader);
      uint64_t same = __ballot(e == el) & pending;
      if (e == el) {
        uint64_t below = same & ((1ull << lane) - 1ull);
        rank = __popcll(below);
        if (lane == leader) wc[wave * E + el] = __popcll(same);
      }
      pending &= ~same;
    }
    __syncthreads();
    if (e >= 0) {
      int32_t pos = cursor[e] + rank;
      for (int w = 0; w < wave; w++) pos += wc[w * E + e];
      perm[pos] = (int32_t)a;
    }
    __syncthreads();
    for (int ee = threadIdx.x; ee < E; ee += DBLOCK)
      cursor[ee] += wc[ee] + wc[E + ee] + wc[2 * E + ee] + wc[3 * E + ee];
    __syncthreads();
  }
}

// Marks perm entries past the valid count with −1.
__global__ void k_dispatch_tail(const int32_t *__restrict__ meta, int A, int32_t *__restrict__ perm) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < A && i >= meta[META_VALID]) perm[i] = -1;
}

}  // namespace

int launch_dispatch(const float *route, int T, int E, int k, int tile_m, const DispatchBufs &db,
                    hipStream_t s) {
  MOE_NONNULL(route);
  MOE_NONNULL(db.blk_counts);
  MOE_NONNULL(db.blk_base);
  MOE_NONNULL(db.offsets);
  MOE_NONNULL(db.tile_off);
  MOE_NONNULL(db.active);
  MOE_NONNULL(db.meta);
  MOE_NONNULL(db.perm);
  if (E > DISPATCH_MAX_E) return moe_fail(MOE_INVALID_ARGUMENT, "dispatch: more than 1024 experts");
  int A = T * k;
  int nblk = (A + DISPATCH_TILE - 1) / DISPATCH_TILE;
  hipLaunchKernelGGL(k_dispatch_count, dim3(nblk), dim3(DBLOCK), 0, s, route, A,
                     k, E, db.blk_counts);
  hipLaunchKernelGGL(k_dispatch_scan, dim3(1), dim3(1024), 0, s,
                     db.blk_counts, nblk, E, tile_m, db.blk_base, db.offsets, db.tile_off,
                     db.active, db.meta);
  hipLaunchKernelGGL(k_dispatch_scatter, dim3(nblk), dim3(DBLOCK), 0, s,
                     route, A, k, E, db.blk_base, db.perm);
  hipLaunchKernelGGL(k_dispatch_tail, dim3((A + 255) / 256), dim3(256), 0, s, db.meta, A, db.perm);
  return 0;
}
