// RMSNorm for gfx950: x · rsqrt(mean(x²) + eps) · weight, optionally
// (residual + that) · scale, over each run of `group` columns of a row.
//
// Reference: src/core/graph/ops/reduce.ts:61-92 (rmsNorm op and its
// options), src/core/kernels/reduce/rmsNorm.ts:84-140 (kernel: f32 sums,
// v = x·inv·w, then + residual, then · outScale, stored in the input dtype),
// src/zoo/privacy-filter/moeMlp.ts:23,82 (the MoE block's pre-norm, eps 1e-5).
//
// One 64-wide wavefront per (row, run). The sum of squares follows this
// library's canonical f32 order, so a CPU restatement reproduces it bit for
// bit (the normalised row feeds the router, whose expert ids are compared
// bit for bit):
//   lane l sums the quads q ≡ l (mod 64) of the run in ascending q, each
//   quad's elements in ascending order: s = s + x·x (no fused multiply-add:
//   this file is compiled with -ffp-contract=off);
//   the 64 lane sums meet in an xor butterfly, strides 32, 16, …, 1 (IEEE
//   addition commutes, so every lane ends with the same bits);
//   inv = 1 / sqrt(total / group + eps), both operations correctly rounded.
// The reference sums with a 32-lane subgroup or a 64-thread tree
// (rmsNorm.ts:26-45,115-118); its tests allow a few ulp (atol 1e-6, rtol
// 1e-5 for f32), which this order meets.
#include "moe_internal.h"

namespace {

constexpr int WAVE = 64;
constexpr int NORM_BLOCK = 256;  // four wavefronts, four (row, run) items

template <typename T>
__device__ __forceinline__ float ld(const T *p, int64_t i) {
  return (float)p[i];
}

template <typename T>
__global__ __launch_bounds__(NORM_BLOCK) void k_rmsnorm(NormArgs a) {
  const int lane = threadIdx.x & (WAVE - 1);
  const int runs = a.cols / a.group;
  const int64_t item = (int64_t)blockIdx.x * (NORM_BLOCK / WAVE) + threadIdx.x / WAVE;
  if (item >= (int64_t)a.rows * runs) return;  // the whole wavefront together
  const int64_t row = item / runs;
  const int g0 = (int)(item - row * runs) * a.group;
  const int64_t base = row * a.cols + g0;
  const T *x = (const T *)a.x;

  float s = 0.f;
  for (int q = lane; 4 * q < a.group; q += WAVE) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int i = 4 * q + j;
      if (i < a.group) {
        const float v = ld(x, base + i);
        s = s + v * v;
      }
    }
  }
#pragma unroll
  for (int m = WAVE / 2; m >= 1; m >>= 1) s = s + __shfl_xor(s, m);
  const float inv = 1.0f / sqrtf(s / (float)a.group + a.eps);

  const T *w = (const T *)a.weight;
  const T *r = (const T *)a.residual;
  T *out = (T *)a.out;
  const int woff = a.weight_len == a.group ? 0 : g0;  // shared weight, or a slice per run
  for (int i = lane; i < a.group; i += WAVE) {
    float v = ld(x, base + i) * inv * ld(w, woff + i);
    if (r) v = v + ld(r, base + i);
    v = v * a.scale;
    out[base + i] = (T)v;
  }
}

// The same item with every load issued at once: runs of whole quads (group
// % 4 == 0, 16-byte f32 / 8-byte f16 alignment) of at most 256·MQ columns.
// Lane l holds quads l, l + 64, … of x, the weight and the residual in
// registers; the sum, the butterfly, inv and the outputs are the scalar
// kernel's, in the same order.
template <typename T> struct Quad;
template <> struct Quad<float> {
  typedef float4 raw;
  static __device__ __forceinline__ raw load(const float *p) { return *(const float4 *)p; }
  static __device__ __forceinline__ float get(raw v, int j) {
    return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
  }
  static __device__ __forceinline__ void store(float *p, const float (&v)[4]) {
    *(float4 *)p = make_float4(v[0], v[1], v[2], v[3]);
  }
};
typedef _Float16 half4n __attribute__((ext_vector_type(4)));
template <> struct Quad<_Float16> {
  typedef half4n raw;
  static __device__ __forceinline__ raw load(const _Float16 *p) { return *(const half4n *)p; }
  static __device__ __forceinline__ float get(raw v, int j) { return (float)v[j]; }
  static __device__ __forceinline__ void store(_Float16 *p, const float (&v)[4]) {
    *(half4n *)p = half4n{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
  }
};

template <typename T, int MQ>
__global__ __launch_bounds__(NORM_BLOCK) void k_rmsnorm_quads(NormArgs a) {
  typedef Quad<T> Q;
  const int lane = threadIdx.x & (WAVE - 1);
  const int runs = a.cols / a.group;
  const int64_t item = (int64_t)blockIdx.x * (NORM_BLOCK / WAVE) + threadIdx.x / WAVE;
  if (item >= (int64_t)a.rows * runs) return;  // the whole wavefront together
  const int64_t row = item / runs;
  const int g0 = (int)(item - row * runs) * a.group;
  const int64_t base = row * a.cols + g0;
  const int nq = a.group / 4;
  const int woff = a.weight_len == a.group ? 0 : g0;
  const T *x = (const T *)a.x;
  const T *w = (const T *)a.weight;
  const T *r = (const T *)a.residual;
  typename Q::raw xv[MQ], wv[MQ], rv[MQ];
#pragma unroll
  for (int j = 0; j < MQ; j++) {
    const int q = lane + WAVE * j;
    const int qc = q < nq ? q : 0;  // in bounds; unused past the run
    xv[j] = Q::load(x + base + 4 * qc);
    wv[j] = Q::load(w + woff + 4 * qc);
    rv[j] = r ? Q::load(r + base + 4 * qc) : xv[j];
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < MQ; j++) {
    if (lane + WAVE * j < nq) {
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const float v = Q::get(xv[j], c);
        s = s + v * v;
      }
    }
  }
#pragma unroll
  for (int m = WAVE / 2; m >= 1; m >>= 1) s = s + __shfl_xor(s, m);
  const float inv = 1.0f / sqrtf(s / (float)a.group + a.eps);
  T *out = (T *)a.out;
#pragma unroll
  for (int j = 0; j < MQ; j++) {
    const int q = lane + WAVE * j;
    if (q >= nq) continue;
    float o[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      float v = Q::get(xv[j], c) * inv * Q::get(wv[j], c);
      if (r) v = v + Q::get(rv[j], c);
      o[c] = v * a.scale;
    }
    Q::store(out + base + 4 * q, o);
  }
}

}  // namespace

int launch_rmsnorm(const NormArgs &a, hipStream_t s) {
  MOE_NONNULL(a.x);
  MOE_NONNULL(a.weight);
  MOE_NONNULL(a.out);
  if (a.rows < 1 || a.cols < 1 || a.group < 1 || a.cols % a.group)
    return moe_fail(MOE_EXECUTION_FAILED, "rmsNorm: bad launch shape");
  const int64_t items = (int64_t)a.rows * (a.cols / a.group);
  const int64_t blocks = (items + NORM_BLOCK / WAVE - 1) / (NORM_BLOCK / WAVE);
  if (blocks > 0x7fffffff) return moe_fail(MOE_EXECUTION_FAILED, "rmsNorm: too many rows");
  const size_t al = a.dtype == MOE_F16 ? 8 : 16;
  const bool aligned = ((uintptr_t)a.x % al == 0) && ((uintptr_t)a.weight % al == 0) &&
                       ((uintptr_t)a.out % al == 0) &&
                       (!a.residual || (uintptr_t)a.residual % al == 0);
  const int mq = (a.group / 4 + WAVE - 1) / WAVE;  // quads per lane
  const bool quads = aligned && a.group % 4 == 0 && a.cols % 4 == 0 && mq <= 8;
  dim3 g((unsigned)blocks), b(NORM_BLOCK);
  if (quads) {
    if (a.dtype == MOE_F16) {
      if (mq <= 4) hipLaunchKernelGGL((k_rmsnorm_quads<_Float16, 4>), g, b, 0, s, a);
      else hipLaunchKernelGGL((k_rmsnorm_quads<_Float16, 8>), g, b, 0, s, a);
    } else {
      if (mq <= 4) hipLaunchKernelGGL((k_rmsnorm_quads<float, 4>), g, b, 0, s, a);
      else hipLaunchKernelGGL((k_rmsnorm_quads<float, 8>), g, b, 0, s, a);
    }
  } else if (a.dtype == MOE_F16) {
    hipLaunchKernelGGL(k_rmsnorm<_Float16>, g, b, 0, s, a);
  } else {
    hipLaunchKernelGGL(k_rmsnorm<float>, g, b, 0, s, a);
  }
  return 0;
}
