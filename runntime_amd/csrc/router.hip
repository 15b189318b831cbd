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
#include "moe_internal.h"

namespace {

constexpr float NEG_START = -3.4e38f;
constexpr int WAVE = 64;

__device__ __forceinline__ float load_as_f32(const float *p, int64_t i) { return p[i]; }
__device__ __forceinline__ float load_as_f32(const _Float16 *p, int64_t i) { return (float)p[i]; }

// (v, e) butterfly arg-max over the wavefront; larger v wins, equal v → lower e.
__device__ __forceinline__ void wave_argmax(float &v, int &e) {
#pragma unroll
  for (int m = 1; m < WAVE; m <<= 1) {
    float ov = __shfl_xor(v, m);
    int oe = __shfl_xor(e, m);
    bool take = (ov > v) || (ov == v && oe < e);
    v = take ? ov : v;
    e = take ? oe : e;
  }
}

// Selects the top k of the wavefront's logits and writes the route row.
// vals[i] is expert lane + 64·i (i < NI). Round r's winner is kept by lane r.
// Then w_i = exp(v_i − v_0) / Σ_j exp(v_j − v_0), the sum taken left to right
// (topkSelect.ts:142-156); lane i < k writes slot i.
template <int NI>
__device__ __forceinline__ void wave_topk_route(const float (&vals)[NI], int E, int k, int lane,
                                                float *row) {
  uint64_t taken = 0;
  float my_v = NEG_START;
  int my_id = 0;
#pragma unroll 1
  for (int r = 0; r < k; r++) {
    float bv = -INFINITY;
    int be = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < NI; i++) {
      int e = lane + WAVE * i;
      float v = vals[i];
      bool cand = (e < E) && !((taken >> i) & 1ull) && (v > NEG_START);
      if (cand && v > bv) {  // ascending e and strict > keep the lower id
        bv = v;
        be = e;
      }
    }
    wave_argmax(bv, be);
    float sv = NEG_START;  // no candidate left: the reference's untouched slot
    int si = 0;
    if (be != 0x7fffffff) {
      sv = bv;
      si = be;
      if ((be & (WAVE - 1)) == lane) taken |= 1ull << (be / WAVE);
    }
    if (lane == r) {
      my_v = sv;
      my_id = si;
    }
  }
  float m = __shfl(my_v, 0);
  float ex = expf(my_v - m);
  float z = __shfl(ex, 0);
#pragma unroll 1
  for (int i = 1; i < k; i++) z = z + __shfl(ex, i);
  if (lane < k) {
    row[lane] = (float)my_id;
    row[k + lane] = ex / z;
  }
}

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

// Per (token tile, d chunk, expert tile): c_j for every (token, expert). The
// x tile [16, 64] and the W chunk [64, 128] sit in LDS.
constexpr int RT_TOKENS = 16;
constexpr int RT_EXPERTS = 128;

template <typename T>
__global__ __launch_bounds__(256) void k_router_chunks(const T *__restrict__ x,
                                                       const float *__restrict__ w, int Tn, int d,
                                                       int E, float *__restrict__ partial) {
  __shared__ float xs[RT_TOKENS * ROUTER_CHUNK];
  __shared__ float ws[ROUTER_CHUNK * RT_EXPERTS];
  int J = (d + ROUTER_CHUNK - 1) / ROUTER_CHUNK;
  int t0 = blockIdx.x * RT_TOKENS;
  int j = blockIdx.y;
  int e0 = blockIdx.z * RT_EXPERTS;
  int et = min(RT_EXPERTS, E - e0);
  int k0 = j * ROUTER_CHUNK;
  int len = min(ROUTER_CHUNK, d - k0);
  for (int i = threadIdx.x; i < RT_TOKENS * ROUTER_CHUNK; i += blockDim.x) {
    int tt = i / ROUTER_CHUNK, kk = i % ROUTER_CHUNK;
    int t = t0 + tt;
    xs[i] = (t < Tn && kk < len) ? load_as_f32(x, (int64_t)t * d + k0 + kk) : 0.f;
  }
  for (int i = threadIdx.x; i < ROUTER_CHUNK * RT_EXPERTS; i += blockDim.x) {
    int kk = i / RT_EXPERTS, ee = i % RT_EXPERTS;
    ws[i] = (kk < len && ee < et) ? w[(int64_t)(k0 + kk) * E + e0 + ee] : 0.f;
  }
  __syncthreads();
  for (int p = threadIdx.x; p < RT_TOKENS * RT_EXPERTS; p += blockDim.x) {
    int tt = p / RT_EXPERTS, ee = p % RT_EXPERTS;
    int t = t0 + tt;
    if (t >= Tn) break;
    if (ee >= et) continue;
    const float *xr = xs + tt * ROUTER_CHUNK;
    float c = 0.f;
    for (int kk = 0; kk < len; kk++) c = fmaf(xr[kk], ws[kk * RT_EXPERTS + ee], c);
    partial[((int64_t)t * J + j) * E + e0 + ee] = c;
  }
}

// Folds the chunk partials in order, adds the bias and runs the top-k.
template <int NI>
__global__ __launch_bounds__(256) void k_router_fold_topk(const float *__restrict__ partial,
                                                          const float *__restrict__ b, int Tn,
                                                          int J, int E, int k,
                                                          float *__restrict__ route) {
  int lane = threadIdx.x & (WAVE - 1);
  int t = blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE;
  if (t >= Tn) return;
  float vals[NI];
#pragma unroll
  for (int i = 0; i < NI; i++) {
    int e = lane + WAVE * i;
    float s = -INFINITY;
    if (e < E) {
      const float *p = partial + (int64_t)t * J * E + e;
      s = p[0];
      for (int jj = 1; jj < J; jj++) s = s + p[(int64_t)jj * E];
      if (b) s = s + b[e];
    }
    vals[i] = s;
  }
  wave_topk_route<NI>(vals, E, k, lane, route + (int64_t)t * 2 * k);
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

int fold_launch(const float *partial, const float *b, int Tn, int J, int E, int k, float *route,
                hipStream_t s) {
  dim3 grid((Tn + 3) / 4), block(256);
  int ni = (E + WAVE - 1) / WAVE;
#define FOLD_NI(N)                                                                          \
  if (ni <= N) {                                                                            \
    hipLaunchKernelGGL((k_router_fold_topk<N>), grid, block, 0, s, partial, b, Tn, J, E, k, \
                       route);                                                              \
    return 0;                                                                               \
  }
  FOLD_NI(1) FOLD_NI(2) FOLD_NI(4) FOLD_NI(8)
#undef FOLD_NI
  return moe_fail(MOE_INVALID_ARGUMENT, "router: more than 512 experts");
}

}  // namespace

int launch_topk(const void *logits, moe_dtype dt, int T, int E, int k, float *route,
                hipStream_t s) {
  MOE_NONNULL(logits);
  MOE_NONNULL(route);
  if (dt == MOE_F16) return topk_launch((const _Float16 *)logits, T, E, k, route, s);
  return topk_launch((const float *)logits, T, E, k, route, s);
}

int launch_router_topk(const void *x, moe_dtype dt, const float *w, const float *b, int T, int d,
                       int E, int k, float *partial, float *route, hipStream_t s) {
  MOE_NONNULL(x);
  MOE_NONNULL(w);
  MOE_NONNULL(partial);
  MOE_NONNULL(route);
  int J = (d + ROUTER_CHUNK - 1) / ROUTER_CHUNK;
  dim3 grid((T + RT_TOKENS - 1) / RT_TOKENS, J, (E + RT_EXPERTS - 1) / RT_EXPERTS), block(256);
  if (dt == MOE_F16)
    hipLaunchKernelGGL(k_router_chunks<_Float16>, grid, block, 0, s, (const _Float16 *)x, w, T,
                       d, E, partial);
  else
    hipLaunchKernelGGL(k_router_chunks<float>, grid, block, 0, s, (const float *)x, w, T, d, E,
                       partial);
  return fold_launch(partial, b, T, J, E, k, route, s);
}
