// Grouped expert products (gate/up + clamped SwiGLU, and down) for gfx950.
//
// Reference: src/core/kernels/matmul/moeQuantW.ts:122-175 (moeUp) and
// :188-237 (moeDown), src/core/kernels/activations.ts:120-133 (SwiGLU),
// src/core/kernels/quantCommon.ts:8-31 (quantW layout).
//
// Rows arrive grouped by expert (dispatch.hip), so one block streams one
// active expert's int8 weights once for all of that expert's rows, instead
// of once per (token, slot) row as the reference does.
//
// k_expert_skinny — the MFMA path (bits = 8, groupSize a multiple of 32 or
// equal to K). One block = one active expert × 64 output columns (16 quantW
// units of 4 columns); its 4 wavefronts split K. Per 32-wide K step a lane
// loads two consecutive 16-byte quantW tiles of its unit (32 contiguous
// bytes; the 4 lanes of a unit cover 128 contiguous bytes), which hold 8
// consecutive k values for each of the unit's 4 columns. Column i of the
// unit feeds MFMA i: v_mfma_f32_16x16x32_f16 with A = 16 rows of the input,
// B = 16 units' column i. int8 → f16 is exact (1024-bias trick with v_perm),
// so the products are exact and sums are f32. An f32 input is split into
// f16 hi + lo parts (two MFMAs), which keeps it to ~2^-22 relative.
// Scales (per column and K group) multiply the f32 partial sums; biases and
// the SwiGLU run in the epilogue.
//
// k_expert_simple — VALU fallback for every other case (int4, small
// groups): one thread per (row, column), f32 fma per group, then × scale.
#include "moe_internal.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;

struct ExpertKArgs {
  const void *a;
  int64_t a_cs;
  int a_row_div;
  const float *route;
  int64_t route_cs;
  int k;
  const uint32_t *w0;
  const float *s0;
  const float *b0;
  const uint32_t *w1;
  const float *s1;
  const float *b1;
  int64_t w0_cs, s0_cs, b0_cs, w1_cs, s1_cs, b1_cs;
  int K, N, E, bits, g;
  float *out;
  int64_t out_cs;
  DispatchBufs db;
};

__device__ __forceinline__ float swiglu(float glu, float lin) {
  // activations.ts:127-133: g = min(glu, 7), l = clamp(lin, ±7).
  float g = fminf(glu, 7.0f);
  float l = fminf(fmaxf(lin, -7.0f), 7.0f);
  return (g / (1.0f + expf(-1.702f * g))) * (l + 1.0f);
}

// Two quantW column words (rows r0..r3 of tile k4 and of tile k4+1) → 8 f16
// in k order. Byte b becomes f16(1024 + (b ^ 0x80)), minus 1152 gives b.
__device__ __forceinline__ half8 cvt_i8x8(uint32_t w0, uint32_t w1) {
  const half2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  uint32_t x0 = w0 ^ 0x80808080u, x1 = w1 ^ 0x80808080u;
  uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u);
  uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u);
  uint32_t p2 = __builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u);
  uint32_t p3 = __builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u);
  half2v h0 = __builtin_bit_cast(half2v, p0) - bias;
  half2v h1 = __builtin_bit_cast(half2v, p1) - bias;
  half2v h2 = __builtin_bit_cast(half2v, p2) - bias;
  half2v h3 = __builtin_bit_cast(half2v, p3) - bias;
  half8 r;
  r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
  r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
  return r;
}

// A fragment: 8 consecutive k of one row, as f16 hi (+ lo for f32 input).
template <typename AT>
struct AFrag;

template <>
struct AFrag<_Float16> {
  static constexpr bool SPLIT = false;
  __device__ __forceinline__ static void load(const void *base, int64_t row, int K, int k0,
                                              bool valid, half8 &hi, half8 &lo) {
    const _Float16 *p = (const _Float16 *)base + row * K + k0;
    if (valid && k0 + 8 <= K && (K & 7) == 0) {
      hi = *(const half8 *)p;
    } else {
#pragma unroll
      for (int j = 0; j < 8; j++) hi[j] = (valid && k0 + j < K) ? p[j] : (_Float16)0.0f;
    }
    (void)lo;
  }
};

template <>
struct AFrag<float> {
  static constexpr bool SPLIT = true;
  __device__ __forceinline__ static void load(const void *base, int64_t row, int K, int k0,
                                              bool valid, half8 &hi, half8 &lo) {
    const float *p = (const float *)base + row * K + k0;
    float v[8];
    if (valid && k0 + 8 <= K) {
      floatx4 a = *(const floatx4 *)p;
      floatx4 b = *(const floatx4 *)(p + 4);
      v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
      v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
    } else {
#pragma unroll
      for (int j = 0; j < 8; j++) v[j] = (valid && k0 + j < K) ? p[j] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
      _Float16 h = (_Float16)v[j];
      hi[j] = h;
      lo[j] = (_Float16)(v[j] - (float)h);
    }
  }
};

template <int NARR>
struct WTiles {
  uint4 t0[NARR], t1[NARR];
};

template <int MODE, typename AT>
__global__ __launch_bounds__(256) void k_expert_skinny(ExpertKArgs p) {
  constexpr int NARR = (MODE == MODE_UP) ? 2 : 1;
  __shared__ floatx4 red[4][NARR * 4][WAVE];

  const int call = blockIdx.z;
  const int32_t *meta = p.db.meta + call * p.db.meta_cs();
  const int slot = blockIdx.y;
  if (slot >= meta[META_ACTIVE]) return;
  const int e = p.db.active[call * p.db.act_cs() + slot];
  const int32_t *offsets = p.db.offsets + call * p.db.off_cs();
  const int32_t *perm = p.db.perm + call * p.db.perm_cs();
  const int p0 = offsets[e];
  const int cnt = offsets[e + 1] - p0;
  const void *abase = (const char *)p.a + call * p.a_cs * (int64_t)sizeof(AT);
  float *out = p.out + call * p.out_cs;
  const float *s0 = p.s0 + call * p.s0_cs;
  const float *s1 = (NARR == 2) ? p.s1 + call * p.s1_cs : nullptr;
  const float *b0 = p.b0 ? p.b0 + call * p.b0_cs : nullptr;
  const float *b1 = (NARR == 2 && p.b1) ? p.b1 + call * p.b1_cs : nullptr;

  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = threadIdx.x / WAVE;
  const int N4 = p.N / 4, K4 = p.K / 4;
  const int u = blockIdx.x * 16 + (lane & 15);
  const bool uok = u < N4;
  const int kq = lane >> 4;
  const int steps = (p.K + 31) / 32;
  const int per = (steps + 3) / 4;
  const int sb = wave * per;
  const int se = min(steps, sb + per);
  const int kg = p.K / p.g;

  const uint4 *wt[2];
  wt[0] = (const uint4 *)(p.w0 + call * p.w0_cs) + ((int64_t)e * N4 + (uok ? u : 0)) * K4;
  wt[1] = (NARR == 2) ? (const uint4 *)(p.w1 + call * p.w1_cs) + ((int64_t)e * N4 + (uok ? u : 0)) * K4
                      : nullptr;

  auto load_w = [&](int step, WTiles<NARR> &w) {
    const int k4 = step * 8 + kq * 2;
#pragma unroll
    for (int a = 0; a < NARR; a++) {
      w.t0[a] = (uok && k4 < K4) ? wt[a][k4] : uint4{0, 0, 0, 0};
      w.t1[a] = (uok && k4 + 1 < K4) ? wt[a][k4 + 1] : uint4{0, 0, 0, 0};
    }
  };

  for (int c0 = 0; c0 < cnt; c0 += 16) {
    const int m = lane & 15;
    const bool rvalid = c0 + m < cnt;
    int64_t src_row = 0;
    if (rvalid) src_row = perm[p0 + c0 + m] / p.a_row_div;

    floatx4 tot[NARR][4], tmp[NARR][4];
#pragma unroll
    for (int a = 0; a < NARR; a++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        tot[a][i] = floatx4{0.f, 0.f, 0.f, 0.f};
        tmp[a][i] = floatx4{0.f, 0.f, 0.f, 0.f};
      }

    // Double-buffered: the next step's weight tiles are in flight while the
    // current step's MFMAs run.
    WTiles<NARR> cur, nxt;
    if (sb < se) load_w(sb, nxt);
    for (int step = sb; step < se; step++) {
      cur = nxt;
      if (step + 1 < se) load_w(step + 1, nxt);
      const int k0 = step * 32 + kq * 8;
      half8 ahi, alo;
      AFrag<AT>::load(abase, src_row, p.K, k0, rvalid, ahi, alo);
#pragma unroll
      for (int a = 0; a < NARR; a++) {
        half8 b0v = cvt_i8x8(cur.t0[a].x, cur.t1[a].x);
        half8 b1v = cvt_i8x8(cur.t0[a].y, cur.t1[a].y);
        half8 b2v = cvt_i8x8(cur.t0[a].z, cur.t1[a].z);
        half8 b3v = cvt_i8x8(cur.t0[a].w, cur.t1[a].w);
        tmp[a][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, b0v, tmp[a][0], 0, 0, 0);
        tmp[a][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, b1v, tmp[a][1], 0, 0, 0);
        tmp[a][2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, b2v, tmp[a][2], 0, 0, 0);
        tmp[a][3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, b3v, tmp[a][3], 0, 0, 0);
        if (AFrag<AT>::SPLIT) {
          tmp[a][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, b0v, tmp[a][0], 0, 0, 0);
          tmp[a][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, b1v, tmp[a][1], 0, 0, 0);
          tmp[a][2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, b2v, tmp[a][2], 0, 0, 0);
          tmp[a][3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, b3v, tmp[a][3], 0, 0, 0);
        }
      }
      // Fold the group's partial sums with its scales at each group end and
      // at the end of this wavefront's K range.
      const int kend = min(p.K, (step + 1) * 32);
      if (kend % p.g == 0 || step == se - 1) {
        const int grp = (step * 32) / p.g;
#pragma unroll
        for (int a = 0; a < NARR; a++) {
          const float *sc = (a == 0) ? s0 : s1;
          floatx4 s4 = uok ? *(const floatx4 *)(sc + ((int64_t)e * kg + grp) * p.N + 4 * u)
                           : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int i = 0; i < 4; i++) {
            tot[a][i] += tmp[a][i] * s4[i];
            tmp[a][i] = floatx4{0.f, 0.f, 0.f, 0.f};
          }
        }
      }
    }

    __syncthreads();
#pragma unroll
    for (int a = 0; a < NARR; a++)
#pragma unroll
      for (int i = 0; i < 4; i++) red[wave][a * 4 + i][lane] = tot[a][i];
    __syncthreads();

    // Wavefront i finishes column i of every unit: C row 4·kq + q, unit u.
    {
      const int i = wave;
      floatx4 sum[NARR];
#pragma unroll
      for (int a = 0; a < NARR; a++) {
        sum[a] = red[0][a * 4 + i][lane];
        sum[a] += red[1][a * 4 + i][lane];
        sum[a] += red[2][a * 4 + i][lane];
        sum[a] += red[3][a * 4 + i][lane];
      }
      if (uok) {
        const int n = 4 * u + i;
        const float bias0 = b0 ? b0[(int64_t)e * p.N + n] : 0.f;
        const float bias1 = b1 ? b1[(int64_t)e * p.N + n] : 0.f;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int mm = kq * 4 + q;
          if (c0 + mm < cnt) {
            const int64_t asg = perm[p0 + c0 + mm];
            float v;
            if (MODE == MODE_UP)
              v = swiglu(sum[0][q] + bias0, sum[NARR - 1][q] + bias1);
            else
              v = sum[0][q] + bias0;
            out[asg * p.N + n] = v;
          }
        }
      }
    }
  }
}

__device__ __forceinline__ int route_expert(const float *route, int64_t a, int k, int E) {
  int64_t t = a / k;
  int s = (int)(a - t * k);
  float f = route[t * 2 * k + s];
  if (!(f >= 0.f) || f >= (float)E) return -1;
  int e = (int)f;
  return ((float)e == f) ? e : -1;
}

// Signed value of logical row kk, column n of expert e (quantCommon.ts:19-31).
__device__ __forceinline__ float qval(const uint32_t *w, int K, int N, int bits, int e, int kk,
                                      int n) {
  int u = n >> 2, c = n & 3, k4 = kk >> 2, r = kk & 3;
  int64_t tb = (((int64_t)e * (N / 4) + u) * (K / 4) + k4) * (bits / 2);
  uint32_t word = w[tb + (c * bits * 4) / 32];
  int off = (c * 4 * bits) % 32 + r * bits;
  int32_t raw = (int32_t)(word << (32 - off - bits)) >> (32 - bits);
  return (float)raw;
}

template <int MODE, typename AT>
__global__ __launch_bounds__(256) void k_expert_simple(ExpertKArgs p) {
  const int call = blockIdx.z;
  const int pos = blockIdx.x;
  if (pos >= p.db.meta[call * p.db.meta_cs() + META_VALID]) return;
  const int n = blockIdx.y * 256 + threadIdx.x;
  if (n >= p.N) return;
  const int64_t asg = p.db.perm[call * p.db.perm_cs() + pos];
  const int e = route_expert(p.route + call * p.route_cs, asg, p.k, p.E);
  const AT *x = (const AT *)p.a + call * p.a_cs + (asg / p.a_row_div) * p.K;
  const int kg = p.K / p.g;
  float acc[2] = {0.f, 0.f};
  constexpr int NARR = (MODE == MODE_UP) ? 2 : 1;
  for (int a = 0; a < NARR; a++) {
    const uint32_t *w = a == 0 ? p.w0 + call * p.w0_cs : p.w1 + call * p.w1_cs;
    const float *sc = a == 0 ? p.s0 + call * p.s0_cs : p.s1 + call * p.s1_cs;
    float tot = 0.f;
    for (int grp = 0; grp < kg; grp++) {
      float part = 0.f;
      for (int kk = grp * p.g; kk < (grp + 1) * p.g; kk++)
        part = fmaf((float)x[kk], qval(w, p.K, p.N, p.bits, e, kk, n), part);
      tot = fmaf(part, sc[((int64_t)e * kg + grp) * p.N + n], tot);
    }
    acc[a] = tot;
  }
  const float *b0 = p.b0 ? p.b0 + call * p.b0_cs : nullptr;
  const float *b1 = p.b1 ? p.b1 + call * p.b1_cs : nullptr;
  float v;
  if (MODE == MODE_UP) {
    float bb0 = b0 ? b0[(int64_t)e * p.N + n] : 0.f;
    float bb1 = b1 ? b1[(int64_t)e * p.N + n] : 0.f;
    v = swiglu(acc[0] + bb0, acc[1] + bb1);
  } else {
    v = acc[0] + (b0 ? b0[(int64_t)e * p.N + n] : 0.f);
  }
  p.out[call * p.out_cs + asg * p.N + n] = v;
}

// out[t] = residual[t] + Σ_s gate_s · y[t·k + s], slots in order; rows of
// ids that are not experts contribute nothing. Reads, never scatters.
__global__ __launch_bounds__(256) void k_combine(const float *__restrict__ y, int64_t y_cs,
                                                 const float *__restrict__ route, int64_t route_cs,
                                                 const float *__restrict__ residual, int64_t res_cs,
                                                 int T, int N, int E, int k,
                                                 float *__restrict__ out, int64_t out_cs) {
  const int call = blockIdx.z;
  const int t = blockIdx.x;
  const int n = blockIdx.y * 256 + threadIdx.x;
  if (n >= N) return;
  y += call * y_cs;
  route += call * route_cs;
  float acc = residual ? residual[call * res_cs + (int64_t)t * N + n] : 0.f;
  for (int s = 0; s < k; s++) {
    const int64_t asg = (int64_t)t * k + s;
    if (route_expert(route, asg, k, E) < 0) continue;
    const float gate = route[(int64_t)t * 2 * k + k + s];
    acc = fmaf(gate, y[asg * N + n], acc);
  }
  out[call * out_cs + (int64_t)t * N + n] = acc;
}

__global__ void k_zero(float *__restrict__ p, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = 0.f;
}

template <int MODE>
int launch_mode(const ExpertArgs &ea, const ExpertKArgs &p, hipStream_t s) {
  const bool mfma = ea.bits == 8 && (ea.g == ea.K || ea.g % 32 == 0);
  const int max_active = ea.E < ea.A ? ea.E : ea.A;
  if (mfma) {
    dim3 grid((ea.N / 4 + 15) / 16, max_active, ea.calls), block(256);
    if (ea.a_dtype == MOE_F16)
      hipLaunchKernelGGL((k_expert_skinny<MODE, _Float16>), grid, block, 0, s, p);
    else
      hipLaunchKernelGGL((k_expert_skinny<MODE, float>), grid, block, 0, s, p);
  } else {
    dim3 grid(ea.A, (ea.N + 255) / 256, ea.calls), block(256);
    if (ea.a_dtype == MOE_F16)
      hipLaunchKernelGGL((k_expert_simple<MODE, _Float16>), grid, block, 0, s, p);
    else
      hipLaunchKernelGGL((k_expert_simple<MODE, float>), grid, block, 0, s, p);
  }
  return 0;
}

}  // namespace

int launch_expert(const ExpertArgs &ea, const DispatchBufs &db, hipStream_t s) {
  MOE_NONNULL(ea.a);
  MOE_NONNULL(ea.route);
  MOE_NONNULL(ea.w0.w);
  MOE_NONNULL(ea.w0.scales);
  MOE_NONNULL(ea.out);
  if (ea.mode == MODE_UP) {
    MOE_NONNULL(ea.w1.w);
    MOE_NONNULL(ea.w1.scales);
  }
  MOE_NONNULL(db.perm);
  MOE_NONNULL(db.offsets);
  MOE_NONNULL(db.active);
  MOE_NONNULL(db.meta);
  if (db.E != ea.E || db.A != ea.A)
    return moe_fail(MOE_EXECUTION_FAILED, "expert: dispatch workspace sized for another shape");
  ExpertKArgs p;
  p.a = ea.a;
  p.a_cs = ea.a_cs;
  p.a_row_div = ea.a_row_div;
  p.route = ea.route;
  p.route_cs = ea.route_cs;
  p.k = ea.k;
  p.w0 = ea.w0.w;
  p.s0 = ea.w0.scales;
  p.b0 = ea.w0.bias;
  p.w1 = ea.w1.w;
  p.s1 = ea.w1.scales;
  p.b1 = ea.w1.bias;
  p.w0_cs = ea.w0_cs;
  p.s0_cs = ea.s0_cs;
  p.b0_cs = ea.b0_cs;
  p.w1_cs = ea.w1_cs;
  p.s1_cs = ea.s1_cs;
  p.b1_cs = ea.b1_cs;
  p.K = ea.K;
  p.N = ea.N;
  p.E = ea.E;
  p.bits = ea.bits;
  p.g = ea.g;
  p.out = ea.out;
  p.out_cs = ea.out_cs;
  p.db = db;
  if (ea.mode == MODE_UP) return launch_mode<MODE_UP>(ea, p, s);
  return launch_mode<MODE_DOWN>(ea, p, s);
}

int launch_combine(const float *y, int64_t y_cs, const float *route, int64_t route_cs,
                   const float *residual, int64_t res_cs, int T, int N, int E, int k, float *out,
                   int64_t out_cs, int calls, hipStream_t s) {
  MOE_NONNULL(y);
  MOE_NONNULL(route);
  MOE_NONNULL(out);
  dim3 grid(T, (N + 255) / 256, calls), block(256);
  hipLaunchKernelGGL(k_combine, grid, block, 0, s, y, y_cs, route, route_cs, residual, res_cs, T,
                     N, E, k, out, out_cs);
  return 0;
}

int launch_zero(float *p, size_t n, hipStream_t s) {
  MOE_NONNULL(p);
  size_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks == 0) return 0;
  hipLaunchKernelGGL(k_zero, dim3((unsigned)blocks), dim3(256), 0, s, p, n);
  return 0;
}
