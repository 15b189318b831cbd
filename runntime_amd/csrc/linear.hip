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
// rows), so the work is spread over columns, K and rows: block (column
// tile of 64, K slice of LKS, chunk of LRB rows) is one wavefront; it
// stages its rows' K slice in LDS and writes a partial product, and a second
// kernel adds the slices in slice order, then the bias and the addend. Each
// lane owns one column, its K slice held in registers.
#include "moe_internal.h"

namespace {

constexpr int LCOLS = 64;   // columns per block (one per lane)
constexpr int LKS = 64;     // K per slice
constexpr int LRB = 16;     // rows per pass

__global__ __launch_bounds__(LCOLS) void k_linear_partial(const float *__restrict__ x,
                                                          const float *__restrict__ w,
                                                          float *__restrict__ part, int T, int K,
                                                          int N) {
  __shared__ float xs[LRB][LKS];
  const int n = blockIdx.x * LCOLS + threadIdx.x;
  const int s = blockIdx.y;
  const int r_first = blockIdx.z * LRB;
  const int k0 = s * LKS, kl = min(LKS, K - k0);
  const bool col = n < N;
  float *out = part + (int64_t)s * T * N;
  // The column's K slice in registers, every load issued at once.
  float wr[LKS];
#pragma unroll
  for (int kk = 0; kk < LKS; kk++)
    wr[kk] = (col && kk < kl) ? w[(int64_t)(k0 + kk) * N + n] : 0.f;
  const int rows = min(LRB, T - r_first);
  for (int i = threadIdx.x; i < LRB * LKS; i += LCOLS) {
    const int r = i / LKS, kk = i % LKS;
    xs[r][kk] = (r < rows && kk < kl) ? x[(int64_t)(r_first + r) * K + k0 + kk] : 0.f;
  }
  __syncthreads();
  if (!col) return;
  // One row at a time over the unrolled slice (register indices stay
  // static), two chains per row.
  for (int r = 0; r < rows; r++) {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int kk = 0; kk < LKS; kk += 4) {
      const float4 xv = *(const float4 *)&xs[r][kk];
      a0 = fmaf(xv.x, wr[kk], a0);
      a1 = fmaf(xv.y, wr[kk + 1], a1);
      a0 = fmaf(xv.z, wr[kk + 2], a0);
      a1 = fmaf(xv.w, wr[kk + 3], a1);
    }
    out[(int64_t)(r_first + r) * N + n] = a0 + a1;
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
  if ((T + LRB - 1) / LRB > 65535)
    return moe_fail(MOE_INVALID_ARGUMENT, "linear: more than " + std::to_string(65535 * LRB) + " rows");
  dim3 grid((N + LCOLS - 1) / LCOLS, S, (T + LRB - 1) / LRB);
  hipLaunchKernelGGL(k_linear_partial, grid, dim3(LCOLS), 0, s, x, w, part, T, K, N);
  const int64_t n = (int64_t)T * N;
  hipLaunchKernelGGL(k_linear_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, part, S,
                     bias, addend, y, T, N);
  return 0;
}
