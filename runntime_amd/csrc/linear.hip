// Dense Linear for the privacy filter's attention projections and head:
// y [T, N] = x [T, K] · W [K, N] + bias (+ addend), f32, W row-major.
//
// Reference: src/core/nn/layers.ts:166-263 (Linear: y = x·W + bias +
// addend, W stored [in, out]), src/core/graph/compose.ts:45-53. A quantized
// checkpoint weight is dequantized once at load (q · scale per group of
// inputs, the values the reference's kernel multiplies by), so float and
// quantized Linears share this kernel.
//
// The projections are small (≤ 1152 × 896) and the texts short (tens of
// rows), so the work is spread over columns and K: block (column tile of
// 256, K slice of LKS) stages its rows' K slice in LDS and writes a
// partial product; a second kernel adds the slices in slice order, then the
// bias and the addend. Each thread owns one column and LRB rows at a time.
#include "moe_internal.h"

namespace {

constexpr int LCOLS = 256;  // columns per block (one per thread)
constexpr int LKS = 64;     // K per slice
constexpr int LRB = 16;     // rows per pass

__global__ __launch_bounds__(LCOLS) void k_linear_partial(const float *__restrict__ x,
                                                          const float *__restrict__ w,
                                                          float *__restrict__ part, int T, int K,
                                                          int N) {
  __shared__ float xs[LRB][LKS];
  const int n = blockIdx.x * LCOLS + threadIdx.x;
  const int s = blockIdx.y;
  const int k0 = s * LKS, kl = min(LKS, K - k0);
  const bool col = n < N;
  float *out = part + (int64_t)s * T * N;
  for (int r0 = 0; r0 < T; r0 += LRB) {
    const int rows = min(LRB, T - r0);
    __syncthreads();
    for (int i = threadIdx.x; i < LRB * LKS; i += LCOLS) {
      const int r = i / LKS, kk = i % LKS;
      xs[r][kk] = (r < rows && kk < kl) ? x[(int64_t)(r0 + r) * K + k0 + kk] : 0.f;
    }
    __syncthreads();
    float acc[LRB];
#pragma unroll
    for (int r = 0; r < LRB; r++) acc[r] = 0.f;
    if (col) {
      const float *wp = w + (int64_t)k0 * N + n;
      int kk = 0;
      for (; kk + 4 <= kl; kk += 4) {
        const float w0 = wp[(int64_t)kk * N], w1 = wp[(int64_t)(kk + 1) * N];
        const float w2 = wp[(int64_t)(kk + 2) * N], w3 = wp[(int64_t)(kk + 3) * N];
#pragma unroll
        for (int r = 0; r < LRB; r++) {
          const float4 xv = *(const float4 *)&xs[r][kk];
          acc[r] = fmaf(xv.x, w0, acc[r]);
          acc[r] = fmaf(xv.y, w1, acc[r]);
          acc[r] = fmaf(xv.z, w2, acc[r]);
          acc[r] = fmaf(xv.w, w3, acc[r]);
        }
      }
      for (; kk < kl; kk++) {
        const float wv = wp[(int64_t)kk * N];
#pragma unroll
        for (int r = 0; r < LRB; r++) acc[r] = fmaf(xs[r][kk], wv, acc[r]);
      }
#pragma unroll
      for (int r = 0; r < LRB; r++)
        if (r < rows) out[(int64_t)(r0 + r) * N + n] = acc[r];
    }
  }
}

__global__ void k_linear_reduce(const float *__restrict__ part, int S, const float *__restrict__ bias,
                                const float *__restrict__ addend, float *__restrict__ y, int T,
                                int N) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)T * N) return;
  const int n = (int)(i % N);
  float v = part[i];
  for (int s = 1; s < S; s++) v += part[(int64_t)s * T * N + i];
  if (bias) v += bias[n];
  if (addend) v += addend[i];
  y[i] = v;
}

}  // namespace

size_t linear_ws_bytes(int T, int K, int N) {
  return (size_t)((K + LKS - 1) / LKS) * T * N * 4;
}

int launch_linear(const float *x, const float *w, const float *bias, const float *addend, float *y,
                  float *part, int T, int K, int N, hipStream_t s) {
  MOE_NONNULL(x);
  MOE_NONNULL(w);
  MOE_NONNULL(y);
  MOE_NONNULL(part);
  const int S = (K + LKS - 1) / LKS;
  dim3 grid((N + LCOLS - 1) / LCOLS, S);
  hipLaunchKernelGGL(k_linear_partial, grid, dim3(LCOLS), 0, s, x, w, part, T, K, N);
  const int64_t n = (int64_t)T * N;
  hipLaunchKernelGGL(k_linear_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, part, S,
                     bias, addend, y, T, N);
  return 0;
}
