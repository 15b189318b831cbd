// Device helpers of the dispatch (stable counting sort of assignments by
// expert), shared by the dispatch kernels and the fused router kernel.
//
// The sort: assignment a = t·k + s goes to expert e = route[t, s];
// offsets[e] = Σ_{e' < e} count(e'); within an expert assignments keep
// ascending a. An id that is not an expert index (negative, ≥ E, fractional,
// NaN) is left out. The reference has no such permutation: every (token,
// slot) row reads its expert's weights directly
// (src/core/kernels/matmul/moeQuantW.ts:131-134).
#pragma once
#include "moe_internal.h"

namespace moe_dev {

constexpr int WAVE = 64;

__device__ __forceinline__ int route_expert(const float *route, int64_t a, int k, int E) {
  int64_t t = a / k;
  int s = (int)(a - t * k);
  float f = route[t * 2 * k + s];
  if (!(f >= 0.f) || f >= (float)E) return -1;
  int e = (int)f;
  return ((float)e == f) ? e : -1;
}

// One wavefront turns per-expert counts (LDS) into the call's offsets,
// M-tile offsets, active-expert descriptors {e, first row, rows, first
// M-tile} and meta. lds_off receives a copy of offsets.
// Lane l scans a contiguous chunk of experts; chunk totals are combined with
// a shuffle prefix sum.
__device__ __forceinline__ void wave_scan_experts(const int32_t *hist, int E, int tile_m, int lane,
                                                  int32_t *offsets, int32_t *tile_off,
                                                  int32_t *active, int32_t *meta,
                                                  int32_t *lds_off) {
  const int chunk = (E + WAVE - 1) / WAVE;
  const int e0 = min(E, lane * chunk), e1 = min(E, e0 + chunk);
  int c = 0, tl = 0, na = 0, mx = 0;
  for (int e = e0; e < e1; e++) {
    int h = hist[e];
    c += h;
    tl += (h + tile_m - 1) / tile_m;
    na += h > 0;
    mx = h > mx ? h : mx;
  }
  int ic = c, it = tl, ia = na;
#pragma unroll
  for (int dlt = 1; dlt < WAVE; dlt <<= 1) {
    int oc = __shfl_up(ic, dlt), ot = __shfl_up(it, dlt), oa = __shfl_up(ia, dlt);
    if (lane >= dlt) {
      ic += oc;
      it += ot;
      ia += oa;
    }
  }
#pragma unroll
  for (int m = 1; m < WAVE; m <<= 1) {
    int o = __shfl_xor(mx, m);
    mx = o > mx ? o : mx;
  }
  int bc = ic - c, bt = it - tl, ba = ia - na;
  for (int e = e0; e < e1; e++) {
    int h = hist[e];
    offsets[e] = bc;
    lds_off[e] = bc;
    tile_off[e] = bt;
    if (h > 0) {
      active[4 * ba + 0] = e;
      active[4 * ba + 1] = bc;
      active[4 * ba + 2] = h;
      active[4 * ba + 3] = bt;
      ba++;
    }
    bc += h;
    bt += (h + tile_m - 1) / tile_m;
  }
  const int total = __shfl(ic, WAVE - 1), ttot = __shfl(it, WAVE - 1),
            atot = __shfl(ia, WAVE - 1);
  for (int i = atot + lane; i < E; i += WAVE) {
    active[4 * i + 0] = -1;
    active[4 * i + 1] = 0;
    active[4 * i + 2] = 0;
    active[4 * i + 3] = 0;
  }
  if (lane == 0) {
    offsets[E] = total;
    lds_off[E] = total;
    tile_off[E] = ttot;
    meta[META_VALID] = total;
    meta[META_ACTIVE] = atot;
    meta[META_MAXCNT] = mx;
    meta[META_TILES] = ttot;
  }
}

// Stable placement of up to 256 consecutive assignments (one per thread of
// wavefronts 0..3, a = a0 + threadIdx.x, expert e or −1). cursor[e] (LDS) is
// the next free position of expert e; wc is LDS scratch [4][E]. Every thread
// of the block must call it (barriers inside). Advances cursor.
__device__ __forceinline__ void block_place(int e, int64_t a, int E, int32_t *cursor, int32_t *wc,
                                            int32_t *perm) {
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = threadIdx.x / WAVE;
  for (int i = threadIdx.x; i < 4 * E; i += blockDim.x) wc[i] = 0;
  __syncthreads();
  int rank = 0;
  if (wave < 4) {
    // The lanes of this wavefront with the same expert, from one ballot per
    // bit of the id (lanes whose bit agrees), then the rank among the
    // earlier ones; the first such lane records the wavefront's count.
    uint64_t same = __ballot(e >= 0);
    for (int bit = 0; (1 << bit) < E; bit++) {
      const uint64_t ones = __ballot(e >= 0 && ((e >> bit) & 1));
      same &= ((e >> bit) & 1) ? ones : ~ones;
    }
    if (e >= 0) {
      rank = __popcll(same & ((1ull << lane) - 1ull));
      if (rank == 0) wc[wave * E + e] = __popcll(same);
    }
  }
  __syncthreads();
  if (wave < 4 && e >= 0) {
    int32_t pos = cursor[e] + rank;
    for (int w = 0; w < wave; w++) pos += wc[w * E + e];
    perm[pos] = (int32_t)a;
  }
  __syncthreads();
  for (int ee = threadIdx.x; ee < E; ee += blockDim.x)
    cursor[ee] += wc[ee] + wc[E + ee] + wc[2 * E + ee] + wc[3 * E + ee];
  __syncthreads();
}

}  // namespace moe_dev
