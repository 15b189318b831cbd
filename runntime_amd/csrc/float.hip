// Float-weight expert products (f32 or f16 weights) for gfx950: the
// privacy filter's float branch.
//
// Reference: src/core/kernels/matmul/matmulGather.ts:38-103 (out[i] =
// a[i]·W[e_i] + bias[e_i], W = rows [e·K, (e+1)·K) of w [E·K, N]),
// src/core/graph/ops/matmul.ts:180-210 (the op), src/zoo/privacy-filter/
// moeMlp.ts:85-100 (the float forward: glu and lin gathers, clamped
// SwiGLU, the out gather, gate-weighted sum over the slots, + x).
//
// Rows arrive grouped by expert (dispatch.hip), so each expert's weight
// rows stream once per chunk of its rows, where the reference reads them
// once per (row, slot). The weights are row-major [K, N] per expert: a
// lane owns 4 consecutive columns (one 8- or 16-byte load per weight row,
// 64 lanes reading one contiguous stretch), and the block's 4 wavefronts
// split K; their partial sums meet in LDS, added in wavefront order. The
// arithmetic is f32 VALU fma: at decode sizes the kernel streams weights,
// and MFMA would need the weights transposed first.
#include "moe_internal.h"

namespace {

constexpr int WAVE = 64;
constexpr int FCOLS = 4 * WAVE;  // columns per block

__device__ __forceinline__ float swiglu(float glu, float lin) {
  // activations.ts:127-133, exp via the hardware 2^x and the quotient via
  // the hardware reciprocal (each within 1 ulp), as the int8 path does.
  const float g = fminf(glu, 7.0f);
  const float l = fminf(fmaxf(lin, -7.0f), 7.0f);
  const float e = __builtin_amdgcn_exp2f(g * (-1.702f * 1.4426950408889634f));
  return g * __builtin_amdgcn_rcpf(1.0f + e) * (l + 1.0f);
}

__device__ __forceinline__ float4 load4w(const float *p) { return *(const float4 *)p; }
__device__ __forceinline__ float4 load4w(const _Float16 *p) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  const h4 v = *(const h4 *)p;
  return make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
}
__device__ __forceinline__ void store4(float *p, float4 v) { *(float4 *)p = v; }
__device__ __forceinline__ void store4(_Float16 *p, float4 v) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  *(h4 *)p = h4{(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
}
__device__ __forceinline__ float4 fma4(float a, float4 w, float4 c) {
  return make_float4(fmaf(a, w.x, c.x), fmaf(a, w.y, c.y), fmaf(a, w.z, c.z), fmaf(a, w.w, c.w));
}
__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// MODE_UP: act[a] = swiglu(x·glu[e] + bias_glu[e], x·lin[e] + bias_lin[e]).
// MODE_DOWN (and the plain gather): out[a] = x·w[e] + bias[e].
// AT: activation type, WT: weight and bias type, OT: output type.
// FW wavefronts split K; FRC rows per chunk. Decode (experts with a row or
// two) runs 8 × 2: twice the wavefronts and loads in flight of 4 × 4, whose
// larger chunks suit experts with more rows (fewer passes over the weights).
// FU weight rows per loop iteration are in flight: 8 with 2 rows per chunk,
// 4 with 4 (where 8 costs more registers than it gains).
template <int MODE, typename AT, typename WT, typename OT, int FW, int FRC, int FU>
__global__ __launch_bounds__(FW * WAVE) void k_float_expert(FloatArgs p) {
  constexpr int NS = MODE == MODE_UP ? 2 : 1;
  extern __shared__ __align__(16) unsigned char smem[];
  float *xs = (float *)smem;                                  // [FRC][K]
  float4 *red = (float4 *)(smem + (size_t)FRC * p.K * 4);     // [FW][NS][FRC][WAVE]

  const int call = blockIdx.z;
  const int4 desc = ((const int4 *)(p.db.active + call * p.db.act_cs()))[blockIdx.y];
  const int e = desc.x;
  if (e < 0) return;
  const int p0 = desc.y, cnt = desc.z;
  const int32_t *perm = p.db.perm + call * p.db.perm_cs();
  const AT *abase = (const AT *)p.a + call * p.a_cs;
  OT *out = (OT *)p.out + call * p.out_cs;
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
  const int c0 = blockIdx.x * FCOLS + 4 * lane;
  const bool col_ok = c0 < p.N;
  const int kq = (p.K + FW - 1) / FW;
  const int kb = wave * kq, ke = min(p.K, kb + kq);
  const WT *w[NS];
  const WT *b[NS];
#pragma unroll
  for (int s = 0; s < NS; s++) {
    w[s] = (const WT *)(s == 0 ? p.w0 : p.w1) + call * (s == 0 ? p.w0_cs : p.w1_cs) +
           (int64_t)e * p.K * p.N + (col_ok ? c0 : 0);
    const WT *bb = (const WT *)(s == 0 ? p.b0 : p.b1);
    b[s] = bb ? bb + call * (s == 0 ? p.b0_cs : p.b1_cs) + (int64_t)e * p.N + (col_ok ? c0 : 0)
              : nullptr;
  }

  for (int r0 = 0; r0 < cnt; r0 += FRC) {
    const int rows = min(FRC, cnt - r0);
    for (int i = threadIdx.x; i < FRC * p.K; i += FW * WAVE) {
      const int r = i / p.K, kk = i - r * p.K;
      float v = 0.f;
      if (r < rows) v = (float)abase[(int64_t)(perm[p0 + r0 + r] / p.a_row_div) * p.K + kk];
      xs[i] = v;
    }
    __syncthreads();
    float4 acc[NS][FRC];
#pragma unroll
    for (int s = 0; s < NS; s++)
#pragma unroll
      for (int r = 0; r < FRC; r++) acc[s][r] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (col_ok) {
      // FU weight rows per iteration, every load issued before the fmas.
      int kk = kb;
      for (; kk + FU <= ke; kk += FU) {
        float4 wv[NS][FU];
#pragma unroll
        for (int s = 0; s < NS; s++)
#pragma unroll
          for (int u = 0; u < FU; u++) wv[s][u] = load4w(w[s] + (int64_t)(kk + u) * p.N);
#pragma unroll
        for (int u = 0; u < FU; u++)
#pragma unroll
          for (int r = 0; r < FRC; r++) {
            const float xv = xs[r * p.K + kk + u];
#pragma unroll
            for (int s = 0; s < NS; s++) acc[s][r] = fma4(xv, wv[s][u], acc[s][r]);
          }
      }
      for (; kk < ke; kk++) {
#pragma unroll
        for (int s = 0; s < NS; s++) {
          const float4 wv = load4w(w[s] + (int64_t)kk * p.N);
#pragma unroll
          for (int r = 0; r < FRC; r++) acc[s][r] = fma4(xs[r * p.K + kk], wv, acc[s][r]);
        }
      }
    }
#pragma unroll
    for (int s = 0; s < NS; s++)
#pragma unroll
      for (int r = 0; r < FRC; r++) red[((wave * NS + s) * FRC + r) * WAVE + lane] = acc[s][r];
    __syncthreads();
    // Wavefront 0 adds the K quarters in order, then the bias and (up) the
    // SwiGLU, and writes each row.
    if (wave == 0 && col_ok) {
      for (int r = 0; r < rows; r++) {
        float4 v[NS];
#pragma unroll
        for (int s = 0; s < NS; s++) {
          float4 t = red[((0 * NS + s) * FRC + r) * WAVE + lane];
#pragma unroll
          for (int q = 1; q < FW; q++) t = add4(t, red[((q * NS + s) * FRC + r) * WAVE + lane]);
          if (b[s]) t = add4(t, load4w(b[s]));
          v[s] = t;
        }
        float4 o = v[0];
        if (MODE == MODE_UP)
          o = make_float4(swiglu(v[0].x, v[1].x), swiglu(v[0].y, v[1].y), swiglu(v[0].z, v[1].z),
                          swiglu(v[0].w, v[1].w));
        store4(out + (int64_t)perm[p0 + r0 + r] * p.N + c0, o);
      }
    }
    __syncthreads();  // xs and red are rewritten by the next chunk
  }
}

__global__ void k_idx_route(const float *__restrict__ idx, int M, float *__restrict__ route) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < M) {
    route[2 * i] = idx[i];
    route[2 * i + 1] = 1.0f;
  }
}

}  // namespace

int launch_idx_route(const float *idx, int M, float *route, hipStream_t s) {
  MOE_NONNULL(idx);
  MOE_NONNULL(route);
  hipLaunchKernelGGL(k_idx_route, dim3((M + 255) / 256), dim3(256), 0, s, idx, M, route);
  return 0;
}

size_t float_expert_lds(int K, int mode, int fw, int frc) {
  return (size_t)frc * K * 4 + (size_t)fw * (mode == MODE_UP ? 2 : 1) * frc * WAVE * 16;
}

int launch_float_expert(const FloatArgs &p, int mode, moe_dtype a_dt, moe_dtype w_dt,
                        moe_dtype o_dt, int max_active, int calls, hipStream_t s) {
  MOE_NONNULL(p.a);
  MOE_NONNULL(p.w0);
  MOE_NONNULL(p.out);
  MOE_NONNULL(p.db.perm);
  MOE_NONNULL(p.db.active);
  if (mode == MODE_UP) MOE_NONNULL(p.w1);
  // Experts with at most ~2 rows on average (decode): 8 wavefronts × 2 rows.
  const bool small = (long)p.db.A <= 2l * max_active;
  const int fw = small ? 8 : 4, frc = small ? 2 : 4;
  const size_t lds = float_expert_lds(p.K, mode, fw, frc);
  if (lds > 64 * 1024)
    return moe_fail(MOE_INVALID_ARGUMENT, "float expert: K " + std::to_string(p.K) +
                                              " is too long for the 64 KB row stage");
  dim3 grid((p.N + FCOLS - 1) / FCOLS, max_active, calls), block(fw * WAVE);
#define FLT(M_, A_, W_, O_)                                                                   \
  do {                                                                                        \
    if (small) hipLaunchKernelGGL((k_float_expert<M_, A_, W_, O_, 8, 2, 8>), grid, block, lds, s, p); \
    else hipLaunchKernelGGL((k_float_expert<M_, A_, W_, O_, 4, 4, 4>), grid, block, lds, s, p);       \
  } while (0)
  const bool af = a_dt == MOE_F16, wf = w_dt == MOE_F16, of = o_dt == MOE_F16;
  if (mode == MODE_UP) {
    // act is f32 (the layer keeps its intermediates in f32)
    if (af && wf) FLT(MODE_UP, _Float16, _Float16, float);
    else if (!af && !wf) FLT(MODE_UP, float, float, float);
    else return moe_fail(MOE_INVALID_ARGUMENT, "float expert: x and weights need one dtype");
  } else {
    if (wf) {
      if (af && of) FLT(MODE_DOWN, _Float16, _Float16, _Float16);
      else if (!af && !of) FLT(MODE_DOWN, float, _Float16, float);
      else if (!af && of) FLT(MODE_DOWN, float, _Float16, _Float16);
      else FLT(MODE_DOWN, _Float16, _Float16, float);
    } else {
      if (!af && !of) FLT(MODE_DOWN, float, float, float);
      else return moe_fail(MOE_INVALID_ARGUMENT, "float expert: f32 weights need f32 rows");
    }
  }
#undef FLT
  return 0;
}
