// Router GEMV/GEMM and top-k gating for gfx950.
//
// Reference: src/core/kernels/reduce/topkSelect.ts:21-92 (selection and
// softmax), src/zoo/privacy-filter/moeMlp.ts:83 (topk(gate.forward(xn), 4)),
// src/core/nn/layers.ts:252-263 (the router is a Linear, W stored [d, E]).
//
// Logits follow this library's canonical f32 order so expert ids are
// reproducible bit for bit on the CPU:
//   c_j = fma chain over k ascending in chunk j (64 wide), from 0
//   S   = ((c_0 + c_1) + c_2) + …;   logit = S + b
// This file is compiled with -ffp-contract=off; the only fused operations
// are the explicit fmaf() calls.
//
// Top-k runs one 64-wide wavefront per token. Each lane owns experts
// lane, lane+64, …; k rounds of a butterfly arg-max (ties → lower id) pick
// the winners. This is the reference's bubble insertion restated for a
// wavefront: a logit is a candidate only if it is strictly above the
// reference's −3.4e38 start value (so NaN never enters), and a slot no
// candidate fills keeps (−3.4e38, id 0), as the reference's does.
#include "norm_dev.h"
#include "router_dev.h"

namespace {

typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float floatx4_r __attribute__((ext_vector_type(4)));
constexpr int WAVE = 64;
using moe_dev::wave_topk_route;

__device__ __forceinline__ float load_as_f32(const float *p, int64_t i) { return p[i]; }
__device__ __forceinline__ float load_as_f32(const _Float16 *p, int64_t i) { return (float)p[i]; }

// ------------------------------------------------------- standalone topk

template <int NI, typename T>
__global__ __launch_bounds__(256) void k_topk(const T *__restrict__ logits, int Tn, int E, int k,
                                              float *__restrict__ route) {
  int lane = threadIdx.x & (WAVE - 1);
  int t = blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE;
  if (t >= Tn) return;  // whole wavefront exits together
  float vals[NI];
#pragma unroll
  for (int i = 0; i < NI; i++) {
    int e = lane + WAVE * i;
    vals[i] = (e < E) ? load_as_f32(logits, (int64_t)t * E + e) : -INFINITY;
  }
  wave_topk_route<NI>(vals, E, k, lane, route + (int64_t)t * 2 * k);
}

// --------------------------------------------------------- fused router

// Per (token tile, d chunk, expert tile, call): c_j for every (token,
// expert). The x tile [16, 64] and the W chunk [64, 128] sit in LDS.
constexpr int RT_TOKENS = 16;
constexpr int RT_EXPERTS = 128;

// Inverse RMS of 1-4 rows (x, x + stride, …) in the canonical order, their
// loads issued together (wave_rows_inv) for rows up to 2048 long.
template <typename T>
__device__ __forceinline__ void tile_rows_inv(const T *x, int64_t stride, int count, int n, float eps,
                                              int lane, float (&inv)[4]) {
  if (n <= 256) {
    moe_dev::wave_rows_inv<T, 4, 1>(x, stride, count, n, eps, lane, inv);
  } else if (n <= 512) {
    moe_dev::wave_rows_inv<T, 4, 2>(x, stride, count, n, eps, lane, inv);
  } else if (n <= 1024) {
    moe_dev::wave_rows_inv<T, 4, 4>(x, stride, count, n, eps, lane, inv);
  } else if (n <= 2048) {
    float a[2], b[2];
    moe_dev::wave_rows_inv<T, 2, 8>(x, stride, min(count, 2), n, eps, lane, a);
    b[0] = b[1] = 0.f;
    if (count > 2) moe_dev::wave_rows_inv<T, 2, 8>(x + 2 * stride, stride, count - 2, n, eps, lane, b);
    inv[0] = a[0], inv[1] = a[1], inv[2] = b[0], inv[3] = b[1];
  } else {
#pragma unroll
    for (int r = 0; r < 4; r++)
      inv[r] = r < count ? moe_dev::wave_row_inv(x + r * stride, n, eps, lane) : 0.f;
  }
}

// NORM: moe_block's pre-norm applied while staging (ra.norm_w); a template
// flag, so that the plain instance keeps its few registers (occupancy).
// EXB experts per block: 128, or fewer for launches with few blocks (a
// single-token call has one block per chunk and expert tile: more, smaller
// tiles spread its router weights over more CUs).
// VEC (E a multiple of 4): W comes in 16-byte loads, four experts a lane.
// One CU's load instructions, not bytes, bound this kernel: 4-byte loads
// move ~23 GB/s per CU (256 B per wavefront instruction).
template <typename T, bool NORM, bool VEC, int EXB>
__global__ __launch_bounds__(256) void k_router_chunks(RouterArgs ra) {
  __shared__ float xs[RT_TOKENS * ROUTER_CHUNK];
  __shared__ float ws[ROUTER_CHUNK * EXB];
  const int Tn = ra.T, d = ra.d, E = ra.E;
  const int J = (d + ROUTER_CHUNK - 1) / ROUTER_CHUNK;
  const int etiles = (E + EXB - 1) / EXB;
  const int call = blockIdx.z / etiles;
  const T *x = (const T *)ra.x + call * ra.x_cs;
  const float *w = ra.w + call * ra.w_cs;
  float *partial = ra.partial + call * ((int64_t)Tn * J * E);
  const int t0 = blockIdx.x * RT_TOKENS;
  const int j = blockIdx.y;
  const int e0 = (blockIdx.z % etiles) * EXB;
  const int et = min(EXB, E - e0);
  const int k0 = j * ROUTER_CHUNK;
  const int len = min(ROUTER_CHUNK, d - k0);
  // Staging: every load of the tile is issued before the first LDS store.
  constexpr int XPER = RT_TOKENS * ROUTER_CHUNK / 256, WPER = ROUTER_CHUNK * EXB / 256;
  const T *nw = NORM ? (const T *)ra.norm_w : nullptr;
  float xv[XPER], nv[NORM ? XPER : 1];
  floatx4_r wv[WPER / 4];
#pragma unroll
  for (int r = 0; r < XPER; r++) {
    int i = threadIdx.x + 256 * r;
    int tt = i / ROUTER_CHUNK, kk = i % ROUTER_CHUNK;
    int t = t0 + tt;
    xv[r] = (t < Tn && kk < len) ? load_as_f32(x, (int64_t)t * d + k0 + kk) : 0.f;
    if constexpr (NORM) nv[r] = kk < len ? load_as_f32(nw, k0 + kk) : 0.f;
  }
  if constexpr (VEC) {
    // Lane i: experts 4(i mod 32) .. + 3 of k row i / 32 (et is a multiple of 4).
#pragma unroll
    for (int r = 0; r < WPER / 4; r++) {
      int i = threadIdx.x + 256 * r;
      int kk = i / (EXB / 4), ee = 4 * (i % (EXB / 4));
      wv[r] = (kk < len && ee < et)
                  ? __builtin_nontemporal_load((const floatx4_r *)(w + (int64_t)(k0 + kk) * E + e0 + ee))
                  : floatx4_r{0.f, 0.f, 0.f, 0.f};
    }
  } else {
#pragma unroll
    for (int r = 0; r < WPER / 4; r++)
#pragma unroll
      for (int c = 0; c < 4; c++) {
        int i = threadIdx.x + 256 * (4 * r + c);
        int kk = i / EXB, ee = i % EXB;
        wv[r][c] = (kk < len && ee < et)
                       ? __builtin_nontemporal_load(w + (int64_t)(k0 + kk) * E + e0 + ee)
                       : 0.f;
      }
  }
  // moe_block's pre-norm, while the tile's loads are in flight: wavefront w
  // takes the inverse RMS of the tile's tokens w, w + 4, w + 8, w + 12 (the
  // canonical order), the loads of all four rows out at once; the first
  // chunk's blocks store it.
  static_assert(RT_TOKENS == 4 * (256 / WAVE), "four tokens per wavefront");
  __shared__ float sinv[RT_TOKENS];
  if constexpr (NORM) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int w4 = threadIdx.x / WAVE;
    const int count = min(4, max(0, (Tn - t0 - w4 + 3) / 4));
    float inv[4] = {0.f, 0.f, 0.f, 0.f};
    if (count > 0) tile_rows_inv(x + (int64_t)(t0 + w4) * d, 4 * (int64_t)d, count, d, ra.norm_eps, lane, inv);
    if (lane == 0) {
#pragma unroll
      for (int b = 0; b < 4; b++) {
        if (b >= count) break;
        const int tt = w4 + 4 * b;
        sinv[tt] = inv[b];
        if (j == 0 && blockIdx.z % etiles == 0) ra.inv[t0 + tt] = inv[b];
      }
    }
    __syncthreads();
  }
  // The pre-norm after every load of the tile is out (a norm right after
  // its load would wait for that load before the next one went out).
  if constexpr (NORM) {
#pragma unroll
    for (int r = 0; r < XPER; r++) {
      int i = threadIdx.x + 256 * r;
      int tt = i / ROUTER_CHUNK, kk = i % ROUTER_CHUNK;
      if (t0 + tt < Tn && kk < len) xv[r] = moe_dev::norm_value<T>(xv[r], sinv[tt], nv[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < XPER; r++) xs[threadIdx.x + 256 * r] = xv[r];
  if constexpr (VEC) {
#pragma unroll
    for (int r = 0; r < WPER / 4; r++) ((floatx4_r *)ws)[threadIdx.x + 256 * r] = wv[r];
  } else {
#pragma unroll
    for (int r = 0; r < WPER / 4; r++)
#pragma unroll
      for (int c = 0; c < 4; c++) ws[threadIdx.x + 256 * (4 * r + c)] = wv[r][c];
  }
  __syncthreads();
  for (int p = threadIdx.x; p < RT_TOKENS * EXB; p += blockDim.x) {
    int tt = p / EXB, ee = p % EXB;
    int t = t0 + tt;
    if (t >= Tn) break;
    if (ee >= et) continue;
    const float *xr = xs + tt * ROUTER_CHUNK;
    float c = 0.f;
    for (int kk = 0; kk < len; kk++) c = fmaf(xr[kk], ws[kk * EXB + ee], c);
    partial[((int64_t)t * J + j) * E + e0 + ee] = c;
  }
}

// S = ((c_0 + c_1) + c_2) + … + b for the wavefront's experts. The
// partials come from blocks on every XCD, so each batch of loads waits a
// full memory latency: the loads go out FB at a time (the launch sizes FB
// to J, up to 32: d ≤ 2048 in one batch), the adds stay in chunk order.
template <int NI, int FB>
__device__ __forceinline__ void fold_logits(const float *partial, const float *b, int t, int J,
                                            int E, int lane, float (&vals)[NI]) {
#pragma unroll
  for (int i = 0; i < NI; i++) {
    const int e = lane + moe_dev::WAVE * i;
    float s = -INFINITY;
    if (e < E) {
      const float *p = partial + (int64_t)t * J * E + e;
      for (int j0 = 0; j0 < J; j0 += FB) {
        float v[FB];
#pragma unroll
        for (int u = 0; u < FB; u++) v[u] = p[(int64_t)min(j0 + u, J - 1) * E];  // in bounds
#pragma unroll
        for (int u = 0; u < FB; u++)
          if (j0 + u < J) s = j0 + u == 0 ? v[u] : s + v[u];
      }
      if (b) s = s + b[e];
    }
    vals[i] = s;
  }
}

// fold_logits in two halves, so that a wavefront that takes several tokens
// can issue the next token's loads before the current token's top-k.
template <int NI, int FB>
struct FoldLoads {
  float v[NI][FB];
};
template <int NI, int FB>
__device__ __forceinline__ void fold_load(const float *partial, int t, int J, int E, int lane,
                                          FoldLoads<NI, FB> &L) {
#pragma unroll
  for (int i = 0; i < NI; i++) {
    const int e = min(lane + moe_dev::WAVE * i, E - 1);  // in bounds; lanes past E unused
    const float *p = partial + (int64_t)t * J * E + e;
#pragma unroll
    for (int u = 0; u < FB; u++) L.v[i][u] = p[(int64_t)min(u, J - 1) * E];
  }
}
// The same sum as fold_logits (chunk order, then + b) from loads already in
// registers; J ≤ FB.
template <int NI, int FB>
__device__ __forceinline__ void fold_sum(const FoldLoads<NI, FB> &L, const float *b, int J, int E,
                                         int lane, float (&vals)[NI]) {
#pragma unroll
  for (int i = 0; i < NI; i++) {
    const int e = lane + moe_dev::WAVE * i;
    float s = L.v[i][0];
#pragma unroll
    for (int u = 1; u < FB; u++)
      if (u < J) s = s + L.v[i][u];
    if (b && e < E) s = s + b[e];
    vals[i] = e < E ? s : -INFINITY;
  }
}

// One wavefront per token: fold, top-k, route row.
template <int NI, int FB>
__global__ __launch_bounds__(256) void k_router_fold_topk(RouterArgs ra) {
  const int lane = threadIdx.x & (moe_dev::WAVE - 1);
  const int t = blockIdx.x * (blockDim.x / moe_dev::WAVE) + threadIdx.x / moe_dev::WAVE;
  if (t >= ra.T) return;
  const int call = blockIdx.y;
  const int J = (ra.d + ROUTER_CHUNK - 1) / ROUTER_CHUNK;
  const float *partial = ra.partial + call * ((int64_t)ra.T * J * ra.E);
  const float *b = ra.b ? ra.b + call * ra.b_cs : nullptr;
  float vals[NI];
  fold_logits<NI, FB>(partial, b, t, J, ra.E, lane, vals);
  wave_topk_route<NI>(vals, ra.E, ra.k, lane, ra.route + call * ra.route_cs + (int64_t)t * 2 * ra.k);
}

// Small calls (T ≤ 64): one block per call (a wavefront per token, up to 16
// wavefronts that then take several tokens each, and at least one thread per
// assignment: 64·max(min(T, 16), ⌈T·k / 64⌉) threads) does the fold
// and top-k of every token, then the call's dispatch (dispatch_dev.h) from
// the ids it just chose — no second pass over the route. An assignment's
// place within its expert is its rank among the earlier assignments with
// that expert, counted over the ids in LDS (at most 256, read by every
// thread at once).
template <int NI, int FB>
__global__ __launch_bounds__(1024) void k_router_fold_topk_dispatch(RouterArgs ra, DispatchBufs db,
                                                                    int tile_m) {
  __shared__ __align__(16) int32_t sid[FUSED_T * MAX_K];
  __shared__ int32_t hist[DISPATCH_MAX_E];
  __shared__ int32_t cursor[DISPATCH_MAX_E + 1];
  const int lane = threadIdx.x & (moe_dev::WAVE - 1);
  const int nwaves = blockDim.x / moe_dev::WAVE;
  const int call = blockIdx.x;
  const int E = ra.E, k = ra.k, A = ra.T * ra.k;
  for (int e = threadIdx.x; e < E; e += blockDim.x) hist[e] = 0;
  const int J = (ra.d + ROUTER_CHUNK - 1) / ROUTER_CHUNK;
  const float *partial = ra.partial + call * ((int64_t)ra.T * J * E);
  const float *b = ra.b ? ra.b + call * ra.b_cs : nullptr;
  // Two tokens' loads live at once: only while they take ≤ 64 registers.
  if (NI * FB <= 32 && J <= FB) {
    // Tokens t, t + nwaves, …: the next token's partials (its index
    // clamped to the last token, so no load sits under a branch) are in
    // flight during this token's top-k.
    int t = threadIdx.x / moe_dev::WAVE;
    FoldLoads<NI, FB> cur;
    fold_load<NI, FB>(partial, min(t, ra.T - 1), J, E, lane, cur);
    for (; t < ra.T; t += nwaves) {
      FoldLoads<NI, FB> nxt;
      fold_load<NI, FB>(partial, min(t + nwaves, ra.T - 1), J, E, lane, nxt);
      float vals[NI];
      fold_sum<NI, FB>(cur, b, J, E, lane, vals);
      int id = wave_topk_route<NI>(vals, E, k, lane,
                                   ra.route + call * ra.route_cs + (int64_t)t * 2 * k);
      if (lane < k) sid[t * k + lane] = id;
      cur = nxt;
    }
  } else {
    for (int t = threadIdx.x / moe_dev::WAVE; t < ra.T; t += nwaves) {
      float vals[NI];
      fold_logits<NI, FB>(partial, b, t, J, E, lane, vals);
      int id = wave_topk_route<NI>(vals, E, k, lane,
                                   ra.route + call * ra.route_cs + (int64_t)t * 2 * k);
      if (lane < k) sid[t * k + lane] = id;
    }
  }
  __syncthreads();
  const int a = threadIdx.x;
  const int e = (a < A) ? sid[a] : -1;
  if (e >= 0) atomicAdd(&hist[e], 1);
  __syncthreads();
  if (threadIdx.x < moe_dev::WAVE)
    moe_dev::wave_scan_experts(hist, E, tile_m, lane, db.offsets + call * db.off_cs(),
                               db.tile_off + call * db.off_cs(), db.active + call * db.act_cs(),
                               db.meta + call * db.meta_cs(), cursor);
  __syncthreads();
  if (e >= 0) {
    // Four ids per LDS read (the same address for every thread); ids past a
    // (including the unwritten tail past A) are not counted.
    const int4 *s4 = (const int4 *)sid;
    int rank = 0;
#pragma unroll 4
    for (int j = 0; j < (A + 3) / 4; j++) {
      const int4 q = s4[j];
      rank += (4 * j < a && q.x == e) + (4 * j + 1 < a && q.y == e) + (4 * j + 2 < a && q.z == e) +
              (4 * j + 3 < a && q.w == e);
    }
    db.perm[call * db.perm_cs() + cursor[e] + rank] = a;
  }
}

// ---------------------------------------- chunk partials for many tokens

// The same c_j as k_router_chunks, register-tiled: a block of 256 threads
// takes TB tokens × EB experts of one chunk, each thread 4 tokens × 4
// experts from two 16-byte LDS reads per k (x^T [64][TB], W [64][EB]).
// For calls with more tokens than the one-block-per-call fused path.
constexpr int RC_EB = 64;  // experts per block (E ≥ 64); TB = 64 tokens

template <typename T, int EB>
__global__ __launch_bounds__(256) void k_router_chunks_tiled(RouterArgs ra) {
  constexpr int EGN = EB / 4, TGN = 256 / EGN, TB = 4 * TGN;
  __shared__ __align__(16) float xs[ROUTER_CHUNK * TB];  // [k][token]
  __shared__ __align__(16) float ws[ROUTER_CHUNK * EB];  // [k][expert]
  const int Tn = ra.T, d = ra.d, E = ra.E;
  const int J = (d + ROUTER_CHUNK - 1) / ROUTER_CHUNK;
  const int etiles = (E + EB - 1) / EB;
  const int call = blockIdx.z / etiles;
  const T *x = (const T *)ra.x + call * ra.x_cs;
  const float *w = ra.w + call * ra.w_cs;
  float *partial = ra.partial + call * ((int64_t)Tn * J * E);
  const int t0 = blockIdx.x * TB;
  const int j = blockIdx.y;
  const int e0 = (blockIdx.z % etiles) * EB;
  const int k0 = j * ROUTER_CHUNK;
  const int len = min(ROUTER_CHUNK, d - k0);
  const int tid = threadIdx.x;
  // Staging in 16-byte loads where the chunk is whole and aligned: x as
  // 8-element runs of a token's row (stored transposed), W as 4-expert runs.
  const bool vec = len == ROUTER_CHUNK && (d & 7) == 0 && (E & 3) == 0 && e0 + EB <= E;
  if (vec) {
    // Every load of the tile before the first LDS store (a loop of load,
    // store pairs waits one memory latency per iteration). A token past T
    // reads token T − 1 and stores zeros.
    constexpr int XR = ROUTER_CHUNK / 8;  // runs per token row
    constexpr int XN = TB * XR / 256, WN = ROUTER_CHUNK * EB / 4 / 256;
    static_assert(TB * XR % 256 == 0 && ROUTER_CHUNK * EB / 4 % 256 == 0, "whole passes");
    typedef float f8 __attribute__((ext_vector_type(8)));
    f8 xv[XN];
    float4 wv[WN];
#pragma unroll
    for (int r = 0; r < XN; r++) {
      const int i = tid + 256 * r;
      const int tt = i / XR, kk = (i % XR) * 8, t = min(t0 + tt, Tn - 1);
      if constexpr (sizeof(T) == 2) {
        const half8v h = *(const half8v *)((const _Float16 *)x + (int64_t)t * d + k0 + kk);
#pragma unroll
        for (int q = 0; q < 8; q++) xv[r][q] = (float)h[q];
      } else {
        const float4 a = *(const float4 *)((const float *)x + (int64_t)t * d + k0 + kk);
        const float4 b = *(const float4 *)((const float *)x + (int64_t)t * d + k0 + kk + 4);
        xv[r] = f8{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      }
    }
#pragma unroll
    for (int r = 0; r < WN; r++) {
      const int i = tid + 256 * r;
      const int kk = i / (EB / 4), ee = (i % (EB / 4)) * 4;
      wv[r] = *(const float4 *)&w[(int64_t)(k0 + kk) * E + e0 + ee];
    }
#pragma unroll
    for (int r = 0; r < XN; r++) {
      const int i = tid + 256 * r;
      const int tt = i / XR, kk = (i % XR) * 8;
      const bool ok = t0 + tt < Tn;
#pragma unroll
      for (int q = 0; q < 8; q++) xs[(kk + q) * TB + tt] = ok ? xv[r][q] : 0.f;
    }
#pragma unroll
    for (int r = 0; r < WN; r++) {
      const int i = tid + 256 * r;
      const int kk = i / (EB / 4), ee = (i % (EB / 4)) * 4;
      *(float4 *)&ws[kk * EB + ee] = wv[r];
    }
  } else {
    for (int i = tid; i < ROUTER_CHUNK * TB; i += 256) {
      const int tt = i / ROUTER_CHUNK, kk = i % ROUTER_CHUNK, t = t0 + tt;
      xs[kk * TB + tt] = (t < Tn && kk < len) ? load_as_f32(x, (int64_t)t * d + k0 + kk) : 0.f;
    }
    for (int i = tid; i < ROUTER_CHUNK * EB; i += 256) {
      const int kk = i / EB, ee = i % EB, e = e0 + ee;
      ws[i] = (kk < len && e < E) ? w[(int64_t)(k0 + kk) * E + e] : 0.f;
    }
  }
  __syncthreads();
  const int eg = tid % EGN, tg = tid / EGN;
  float c[4][4] = {};
  for (int kk = 0; kk < len; kk++) {
    const float4 xv = *(const float4 *)&xs[kk * TB + 4 * tg];
    const float4 wv = *(const float4 *)&ws[kk * EB + 4 * eg];
    const float xa[4] = {xv.x, xv.y, xv.z, xv.w}, wa[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
      for (int q = 0; q < 4; q++) c[a][q] = fmaf(xa[a], wa[q], c[a][q]);
  }
#pragma unroll
  for (int a = 0; a < 4; a++) {
    const int t = t0 + 4 * tg + a;
    if (t >= Tn) break;
    float *row = partial + ((int64_t)t * J + j) * E + e0 + 4 * eg;
    if (e0 + 4 * eg + 3 < E && (E & 3) == 0) {
      *(float4 *)row = make_float4(c[a][0], c[a][1], c[a][2], c[a][3]);
    } else {
#pragma unroll
      for (int q = 0; q < 4; q++)
        if (e0 + 4 * eg + q < E) row[q] = c[a][q];
    }
  }
}

template <typename T>
int topk_launch(const T *logits, int Tn, int E, int k, float *route, hipStream_t s) {
  dim3 grid((Tn + 3) / 4), block(256);
  int ni = (E + WAVE - 1) / WAVE;
#define TOPK_NI(N)                                                                    \
  if (ni <= N) {                                                                      \
    hipLaunchKernelGGL((k_topk<N, T>), grid, block, 0, s, logits, Tn, E, k, route);   \
    return 0;                                                                         \
  }
  TOPK_NI(1) TOPK_NI(2) TOPK_NI(4) TOPK_NI(8) TOPK_NI(16) TOPK_NI(32) TOPK_NI(64)
#undef TOPK_NI
  return moe_fail(MOE_INVALID_ARGUMENT, "topk: more than 4096 experts");
}

}  // namespace

int launch_topk(const void *logits, moe_dtype dt, int T, int E, int k, float *route,
                hipStream_t s) {
  MOE_NONNULL(logits);
  MOE_NONNULL(route);
  if (dt == MOE_F16) return topk_launch((const _Float16 *)logits, T, E, k, route, s);
  return topk_launch((const float *)logits, T, E, k, route, s);
}

int launch_router_topk(const RouterArgs &ra, const DispatchBufs *db, int tile_m, bool *dispatched,
                       hipStream_t s) {
  MOE_NONNULL(ra.x);
  MOE_NONNULL(ra.w);
  MOE_NONNULL(ra.partial);
  MOE_NONNULL(ra.route);
  if (ra.E > ROUTER_MAX_E) return moe_fail(MOE_INVALID_ARGUMENT, "router: more than 512 experts");
  const bool fuse = db && ra.T <= FUSED_T && ra.T * ra.k <= FUSED_T * MAX_K;
  // Many tokens: the register-tiled chunk kernel (64 or 32 experts a block).
  if (!fuse && ra.T > SMALL_T && ra.E >= 32) {
    if (ra.norm_w)
      return moe_fail(MOE_EXECUTION_FAILED, "router: the staged pre-norm runs on calls of at most 64 tokens");
    const int J = (ra.d + ROUTER_CHUNK - 1) / ROUTER_CHUNK;
    if (ra.E >= 64) {
      const int tb = 4 * (256 / (64 / 4)), et = (ra.E + 63) / 64;
      dim3 g((ra.T + tb - 1) / tb, J, et * ra.calls);
      if (ra.x_dtype == MOE_F16) hipLaunchKernelGGL((k_router_chunks_tiled<_Float16, 64>), g, dim3(256), 0, s, ra);
      else hipLaunchKernelGGL((k_router_chunks_tiled<float, 64>), g, dim3(256), 0, s, ra);
    } else {
      const int tb = 4 * (256 / (32 / 4)), et = (ra.E + 31) / 32;
      dim3 g((ra.T + tb - 1) / tb, J, et * ra.calls);
      if (ra.x_dtype == MOE_F16) hipLaunchKernelGGL((k_router_chunks_tiled<_Float16, 32>), g, dim3(256), 0, s, ra);
      else hipLaunchKernelGGL((k_router_chunks_tiled<float, 32>), g, dim3(256), 0, s, ra);
    }
  } else {
    const int J = (ra.d + ROUTER_CHUNK - 1) / ROUTER_CHUNK;
    // Expert tiles of 128, or 64 / 32 while the launch has under 256 blocks.
    const long tt = ((long)ra.T + RT_TOKENS - 1) / RT_TOKENS * J * ra.calls;
    const int exb = tt * ((ra.E + 127) / 128) >= 256 ? 128 : tt * ((ra.E + 63) / 64) >= 256 ? 64 : 32;
    const int etiles = (ra.E + exb - 1) / exb;
    dim3 grid((ra.T + RT_TOKENS - 1) / RT_TOKENS, J, etiles * ra.calls), block(256);
    // 16-byte W loads need every row of W 16-byte aligned.
    const bool vec = ra.E % 4 == 0 && ((uintptr_t)ra.w & 15) == 0 && ra.w_cs % 4 == 0;
#define RC_EXB(T_, N_, V_)                                                                       \
  do {                                                                                           \
    if (exb == 128) hipLaunchKernelGGL((k_router_chunks<T_, N_, V_, 128>), grid, block, 0, s, ra); \
    else if (exb == 64) hipLaunchKernelGGL((k_router_chunks<T_, N_, V_, 64>), grid, block, 0, s, ra); \
    else hipLaunchKernelGGL((k_router_chunks<T_, N_, V_, 32>), grid, block, 0, s, ra);           \
  } while (0)
#define RC_LAUNCH(T_, N_)                 \
  do {                                    \
    if (vec) RC_EXB(T_, N_, true);        \
    else RC_EXB(T_, N_, false);           \
  } while (0)
    if (ra.x_dtype == MOE_F16) {
      if (ra.norm_w) RC_LAUNCH(_Float16, true); else RC_LAUNCH(_Float16, false);
    } else {
      if (ra.norm_w) RC_LAUNCH(float, true); else RC_LAUNCH(float, false);
    }
#undef RC_LAUNCH
#undef RC_EXB
  }
  if (ra.chunks_only) {
    if (dispatched) *dispatched = true;
    return 0;
  }
  const int ni = (ra.E + WAVE - 1) / WAVE;
  // Fold batch: the chunk count J, rounded up to 8, 16 or 32 (8 with more
  // than two experts a lane).
  const int Jc = (ra.d + ROUTER_CHUNK - 1) / ROUTER_CHUNK;
  const int fb = ni > 2 || Jc <= 8 ? 8 : Jc <= 16 ? 16 : 32;
  if (dispatched) *dispatched = fuse;
  if (fuse) {
    // A wavefront per token up to 16 (more tokens loop), and at least one
    // thread per assignment (T·k ≤ 1024).
    const int fused_waves = std::max(std::min(ra.T, 16), (ra.T * ra.k + WAVE - 1) / WAVE);
    const int fused_threads = WAVE * fused_waves;  // ≤ 1024
    MOE_NONNULL(db->offsets);
    MOE_NONNULL(db->perm);
    if (db->E != ra.E || db->A != ra.T * ra.k)
      return moe_fail(MOE_EXECUTION_FAILED, "router: dispatch workspace sized for another shape");
#define FB_SWITCH(KERNEL, N, GRID, BLOCK, ...)                                                   \
  do {                                                                                           \
    if (N > 2 || fb == 8) hipLaunchKernelGGL((KERNEL<N, 8>), GRID, BLOCK, 0, s, __VA_ARGS__);    \
    else if (fb == 16) hipLaunchKernelGGL((KERNEL<N, 16>), GRID, BLOCK, 0, s, __VA_ARGS__);      \
    else hipLaunchKernelGGL((KERNEL<N, 32>), GRID, BLOCK, 0, s, __VA_ARGS__);                    \
  } while (0)
#define FUSED_NI(N)                                                                        \
  if (ni <= N) {                                                                           \
    FB_SWITCH(k_router_fold_topk_dispatch, N, dim3(ra.calls), dim3(fused_threads), ra, *db, tile_m); \
    return 0;                                                                              \
  }
    FUSED_NI(1) FUSED_NI(2) FUSED_NI(4) FUSED_NI(8)
#undef FUSED_NI
  }
  dim3 g2((ra.T + 3) / 4, ra.calls);
#define FOLD_NI(N)                                                                      \
  if (ni <= N) {                                                                        \
    FB_SWITCH(k_router_fold_topk, N, g2, dim3(256), ra);                                \
    return 0;                                                                           \
  }
  FOLD_NI(1) FOLD_NI(2) FOLD_NI(4) FOLD_NI(8)
#undef FOLD_NI
#undef FB_SWITCH
  return moe_fail(MOE_INVALID_ARGUMENT, "router: more than 512 experts");
}
