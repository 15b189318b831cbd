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
constexpr int LKS = 32;     // K per slice
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
  // The column's K slice in registers, every load issued at once. The
  // addresses are clamped into the matrix and the values past it zeroed,
  // so no load sits under a branch.
  float wr[LKS];
  const int nc = min(n, N - 1);
#pragma unroll
  for (int kk = 0; kk < LKS; kk++) {
    const float v = w[(int64_t)min(k0 + kk, K - 1) * N + nc];
    wr[kk] = kk < kl ? v : 0.f;
  }
  const int rows = min(LRB, T - r_first);
  // x slab, every load issued before the first LDS store (a load-store
  // pair per iteration waits out each load's latency in turn).
  constexpr int PER = LRB * LKS / LCOLS;
  float xv[PER];
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int i = threadIdx.x + LCOLS * j, r = i / LKS, kk = i % LKS;
    xv[j] = (r < rows && kk < kl) ? x[(int64_t)(r_first + r) * K + k0 + kk] : 0.f;
  }
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int i = threadIdx.x + LCOLS * j;
    xs[i / LKS][i % LKS] = xv[j];
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
  // Slices added in order, their loads issued 8 at a time.
  const int64_t sl = (int64_t)T * N;
  float v = 0.f;
  int s = 0;
  for (; s + 8 <= S; s += 8) {
    float q[8];
#pragma unroll
    for (int j = 0; j < 8; j++) q[j] = part[(s + j) * sl + i];
#pragma unroll
    for (int j = 0; j < 8; j++) v = (s + j == 0) ? q[j] : v + q[j];
  }
  for (; s < S; s++) v = s == 0 ? part[i] : v + part[s * sl + i];
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
