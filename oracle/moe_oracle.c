/* CPU oracle for ruNNtime's int8 mixture-of-experts layer.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker that the HIP kernels in
 * runntime_amd/csrc are compared against. Only tests/, the smoke() check and
 * bench.py's cpu_baseline leg may load it. The product path never calls it.
 *
 * Every function restates one piece of the reference (software-mansion/
 * runntime, paths relative to packages/runntime/) and cites the lines it
 * follows. Two flavours of the expert products exist:
 *   - *_f64: the reference test's own f64 formulation
 *     (test/core/kernels/matmul/moeQuantW.gpu.test.ts:58-128). This is the
 *     parity oracle for the GPU outputs.
 *   - *_f32ref: the reference WGSL kernels' f32 arithmetic and lane structure
 *     (src/core/kernels/matmul/moeQuantW.ts:122-237): 32 K-lanes, a fixed
 *     16→1 tree merge. This is the "port" CPU baseline that bench.py times.
 * Both generalise the reference's compiled-in 4 slots (MOE_SLOTS,
 * moeQuantW.ts:28) to any k; at k = 4 they reduce to the reference exactly.
 *
 * Pinning (what checks each function, all in tests/test_oracle.py):
 *   orc_lcg_f32            test/gpu.ts:114-122 sequence, first values by hand
 *   orc_pack_quantw_nk     hand-worked words of test/core/weights/quantPack.test.ts
 *   orc_pack_quantw_ekn    same words + read-back identity + tile order
 *   orc_unpack_quantw      read-back identity (quantPack.test.ts:165-192)
 *   orc_topk               known answers of topkSelect.gpu.test.ts:54-72,
 *                          brute-force stable sort on random rows
 *   orc_router_logits      f64 matmul within a rounding bound; closed forms
 *   orc_moe_up_f64 / down  closed forms (identity weights, clamp saturation),
 *                          dense numpy dequant matmul, linearity
 *   orc_*_f32ref           agreement with the f64 forms at the reference
 *                          test's tolerance (atol 1e-5·K, rtol 1e-4)
 *   orc_dispatch           brute-force stable argsort
 *   orc_rmsnorm            the reference test's f64 formula at its tolerance
 *                          (test/core/kernels/reduce/rmsNorm.gpu.test.ts:33-61,
 *                          atol 1e-6, rtol 1e-5) on its shapes and options;
 *                          closed forms (constant rows, eps dominance, scale
 *                          and residual); the lane-order sum against a
 *                          different association, which it must not equal in
 *                          general
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/* ---------------------------------------------------------------- inputs */

/* test/gpu.ts:114-122 — randomF32: s = s·1664525 + 1013904223 (mod 2^32),
 * value s/2^31 − 1 computed in f64 and stored as f32. */
EXPORT void orc_lcg_f32(float *out, int64_t n, uint32_t seed) {
  uint32_t s = seed;
  for (int64_t i = 0; i < n; i++) {
    s = s * 1664525u + 1013904223u;
    out[i] = (float)((double)s / 2147483648.0 - 1.0);
  }
}

/* ---------------------------------------------------------------- quantW */

/* src/core/weights/quantPack.ts:12-28 — packQuantW: one expert's
 * output-first [n, k] ints into quantW words for the logical [k, n] weight.
 * 16-value tiles per (4-column unit, 4-row chunk), column-major in the tile,
 * `bits` per value, lowest bits first, tiles k4-major per unit. */
EXPORT void orc_pack_quantw_nk(const int8_t *ints, int k, int n, int bits, uint32_t *words) {
  memset(words, 0, (size_t)k * n * bits / 32 * sizeof(uint32_t));
  uint32_t mask = (1u << bits) - 1u;
  for (int unit = 0; unit < n / 4; unit++)
    for (int k4 = 0; k4 < k / 4; k4++) {
      int64_t tile_bit = ((int64_t)unit * (k / 4) + k4) * 16 * bits;
      for (int c = 0; c < 4; c++)
        for (int r = 0; r < 4; r++) {
          int8_t v = ints[(int64_t)(unit * 4 + c) * k + k4 * 4 + r];
          int64_t bit = tile_bit + (c * 4 + r) * bits;
          words[bit >> 5] |= ((uint32_t)(uint8_t)v & mask) << (bit & 31);
        }
    }
}

/* test/core/kernels/matmul/quantW.ts:24-43 — the test suite's independent
 * packer: logical q [E·K, N] (row e·K + k) into the same words, expert-major.
 * Word base of tile (e, unit, k4) is ((e·N/4 + unit)·K/4 + k4)·bits/2
 * (src/core/kernels/quantCommon.ts:8-15). */
EXPORT void orc_pack_quantw_ekn(const int8_t *q, int E, int K, int N, int bits, uint32_t *words) {
  memset(words, 0, (size_t)E * K * N * bits / 32 * sizeof(uint32_t));
  uint32_t mask = (1u << bits) - 1u;
  for (int e = 0; e < E; e++)
    for (int u = 0; u < N / 4; u++)
      for (int k4 = 0; k4 < K / 4; k4++) {
        int64_t tile_word = (((int64_t)e * (N / 4) + u) * (K / 4) + k4) * (bits / 2);
        for (int c = 0; c < 4; c++)
          for (int r = 0; r < 4; r++) {
            int8_t v = q[((int64_t)e * K + k4 * 4 + r) * N + u * 4 + c];
            int bit = (c * 4 + r) * bits;
            words[tile_word + bit / 32] |= ((uint32_t)(uint8_t)v & mask) << (bit % 32);
          }
      }
}

/* src/core/kernels/quantCommon.ts:19-31 (deqVec4, columnWord) and
 * moeQuantW.ts:73-89 (tileDots, colWord): column c of a tile sits in word
 * c·bits·4/32 at bit offset (c·4·bits) mod 32; row r is r·bits higher and is
 * sign-extended from `bits` (extractBits on i32). Output logical q [E·K, N]. */
EXPORT void orc_unpack_quantw(const uint32_t *words, int E, int K, int N, int bits, int8_t *q) {
  for (int e = 0; e < E; e++)
    for (int u = 0; u < N / 4; u++)
      for (int k4 = 0; k4 < K / 4; k4++) {
        int64_t tb = (((int64_t)e * (N / 4) + u) * (K / 4) + k4) * (bits / 2);
        for (int c = 0; c < 4; c++) {
          uint32_t w = words[tb + (c * bits * 4) / 32];
          int off = (c * 4 * bits) % 32;
          for (int r = 0; r < 4; r++) {
            int32_t raw = (int32_t)((w >> (off + r * bits)) & ((1u << bits) - 1u));
            if (raw >= (1 << (bits - 1))) raw -= (1 << bits);
            q[((int64_t)e * K + k4 * 4 + r) * N + u * 4 + c] = (int8_t)raw;
          }
        }
      }
}

/* ------------------------------------------------------------------ topk */

/* src/core/kernels/reduce/topkSelect.ts:21-92, generalised from 4 slots to k.
 * Slots start at (−3.4e38, id 0). Experts are visited in ascending id; a
 * value enters only if strictly greater than the last slot, then bubbles up
 * while strictly greater, so ties keep the lower id and NaN never enters.
 * Then w_i = exp(v_i − v_0) / Σ_j exp(v_j − v_0), the sum taken left to right.
 * Output row: k ids (as f32), then k weights. */
EXPORT void orc_topk(const float *logits, int T, int E, int k, float *route) {
  const float NEG = -3.4e38f;
  float v[64];
  int id[64];
  for (int t = 0; t < T; t++) {
    for (int i = 0; i < k; i++) { v[i] = NEG; id[i] = 0; }
    for (int e = 0; e < E; e++) {
      float x = logits[(int64_t)t * E + e];
      if (x > v[k - 1]) {
        v[k - 1] = x; id[k - 1] = e;
        for (int i = k - 1; i > 0; i--) {
          if (v[i] > v[i - 1]) {
            float tv = v[i - 1]; int ti = id[i - 1];
            v[i - 1] = v[i]; id[i - 1] = id[i];
            v[i] = tv; id[i] = ti;
          }
        }
      }
    }
    float m = v[0];
    float ex[64];
    float z = 0.0f;
    for (int i = 0; i < k; i++) { ex[i] = expf(v[i] - m); z = (i == 0) ? ex[0] : z + ex[i]; }
    for (int i = 0; i < k; i++) {
      route[(int64_t)t * 2 * k + i] = (float)id[i];
      route[(int64_t)t * 2 * k + k + i] = ex[i] / z;
    }
  }
}

/* ---------------------------------------------------------------- router */

/* The router is nn.Linear(h, e) → linear → matmul: logits = x·W + b with W
 * stored [d, E] (src/zoo/privacy-filter/moeMlp.ts:55,83;
 * src/core/nn/layers.ts:252-263; src/core/graph/compose.ts:45-53).
 *
 * The reference's f32 summation order depends on which matmul route its
 * dispatcher picks (src/core/gpu/dispatch/matmul.ts:76-101), so no order is
 * "the" reference's. This build fixes one canonical order, followed bit for
 * bit by the GPU router:
 *   c_j   = fma chain over k ascending in [64j, min(64j+64, d)), from 0
 *   S     = ((c_0 + c_1) + c_2) + … + c_{J−1}
 *   logit = S + b_e      (b_e = 0 when there is no bias)
 * with every operation a single IEEE f32 fma or add. */
#define ROUTER_CHUNK 64
EXPORT void orc_router_logits(const float *x, const float *w, const float *b, int T, int d, int E,
                              float *logits) {
  for (int t = 0; t < T; t++)
    for (int e = 0; e < E; e++) {
      float s = 0.0f;
      for (int k0 = 0; k0 < d; k0 += ROUTER_CHUNK) {
        float c = 0.0f;
        int k1 = k0 + ROUTER_CHUNK < d ? k0 + ROUTER_CHUNK : d;
        for (int kk = k0; kk < k1; kk++) c = fmaf(x[(int64_t)t * d + kk], w[(int64_t)kk * E + e], c);
        s = (k0 == 0) ? c : s + c;
      }
      logits[(int64_t)t * E + e] = b ? s + b[e] : s;
    }
}

/* --------------------------------------------------------------- helpers */

static inline int route_id(const float *route, int t, int k, int s, int E) {
  float f = route[(int64_t)t * 2 * k + s];
  if (!(f >= 0.0f) || f >= (float)E) return -1;
  int e = (int)f;
  return ((float)e == f) ? e : -1;
}

/* src/core/kernels/activations.ts:120-133 — gpt-oss clamped SwiGLU:
 * g = min(glu, 7), l = clamp(lin, −7, 7), g·σ(1.702·g)·(l + 1). */
EXPORT double orc_swiglu_f64(double glu, double lin) {
  double g = glu < 7.0 ? glu : 7.0;
  double l = lin < -7.0 ? -7.0 : (lin > 7.0 ? 7.0 : lin);
  return g / (1.0 + exp(-1.702 * g)) * (l + 1.0);
}
static inline float swiglu_f32(float glu, float lin) {
  float g = fminf(glu, 7.0f);
  float l = fminf(fmaxf(lin, -7.0f), 7.0f);
  return (g / (1.0f + expf(-1.702f * g))) * (l + 1.0f);
}

/* Dequantized weight value q·scale of logical row kk (within expert e) and
 * column n: scales are [E·K/g, N] row-major, row e·K/g + kk/g
 * (moeQuantW.ts:139-143). */
static inline int8_t qval(const uint32_t *words, int K, int N, int bits, int e, int kk, int n) {
  int u = n / 4, c = n % 4, k4 = kk / 4, r = kk % 4;
  int64_t tb = (((int64_t)e * (N / 4) + u) * (K / 4) + k4) * (bits / 2);
  uint32_t w = words[tb + (c * bits * 4) / 32];
  int off = (c * 4 * bits) % 32 + r * bits;
  int32_t raw = (int32_t)((w >> off) & ((1u << bits) - 1u));
  if (raw >= (1 << (bits - 1))) raw -= (1 << bits);
  return (int8_t)raw;
}

/* ------------------------------------------------------- expert products */

/* Projection of one input row through expert e in f64, bias first then the
 * K terms in order — test/core/kernels/matmul/moeQuantW.gpu.test.ts:59-71. */
static void project_f64(const float *xrow, const uint32_t *w, const float *sc, const float *bias,
                        int K, int N, int bits, int g, int e, double *out) {
  int kg = K / g;
  for (int n = 0; n < N; n++) out[n] = bias ? (double)bias[(int64_t)e * N + n] : 0.0;
  for (int kk = 0; kk < K; kk++) {
    double xv = xrow[kk];
    const float *srow = sc + ((int64_t)e * kg + kk / g) * N;
    for (int n = 0; n < N; n++) out[n] += xv * ((double)qval(w, K, N, bits, e, kk, n) * (double)srow[n]);
  }
}

/* moeUp (src/core/graph/ops/matmul.ts:220-244; kernel moeQuantW.ts:122-175):
 * act[t·k + s] = swiglu(x[t]·glu[e] + glu_b[e], x[t]·lin[e] + lin_b[e]) with
 * e = route[t, s]. f64 throughout, stored f32 as the reference stores act.
 * A route id that is not an expert index gives a zero row. */
EXPORT void orc_moe_up_f64(const float *x, const float *route, const uint32_t *glu_w,
                           const float *glu_s, const float *glu_b, const uint32_t *lin_w,
                           const float *lin_s, const float *lin_b, int T, int K, int N, int E,
                           int k, int bits, int g, float *act) {
  double *ga = malloc(sizeof(double) * N), *la = malloc(sizeof(double) * N);
  for (int t = 0; t < T; t++)
    for (int s = 0; s < k; s++) {
      float *arow = act + ((int64_t)t * k + s) * N;
      int e = route_id(route, t, k, s, E);
      if (e < 0) { memset(arow, 0, sizeof(float) * N); continue; }
      project_f64(x + (int64_t)t * K, glu_w, glu_s, glu_b, K, N, bits, g, e, ga);
      project_f64(x + (int64_t)t * K, lin_w, lin_s, lin_b, K, N, bits, g, e, la);
      for (int n = 0; n < N; n++) arow[n] = (float)orc_swiglu_f64(ga[n], la[n]);
    }
  free(ga); free(la);
}

/* moeDown (src/core/graph/ops/matmul.ts:246-272; kernel moeQuantW.ts:188-237):
 * out[t] = residual[t] + Σ_s gate_s·(act[t·k + s]·w[e_s] + bias[e_s]), f64,
 * slots in order (moeQuantW.gpu.test.ts:118-126). */
EXPORT void orc_moe_down_f64(const float *act, const float *route, const uint32_t *w,
                             const float *sc, const float *bias, const float *residual, int T,
                             int K, int N, int E, int k, int bits, int g, float *out) {
  double *acc = malloc(sizeof(double) * N), *y = malloc(sizeof(double) * N);
  for (int t = 0; t < T; t++) {
    for (int n = 0; n < N; n++) acc[n] = residual ? (double)residual[(int64_t)t * N + n] : 0.0;
    for (int s = 0; s < k; s++) {
      int e = route_id(route, t, k, s, E);
      if (e < 0) continue;
      double gate = route[(int64_t)t * 2 * k + k + s];
      project_f64(act + ((int64_t)t * k + s) * K, w, sc, bias, K, N, bits, g, e, y);
      for (int n = 0; n < N; n++) acc[n] += gate * y[n];
    }
    for (int n = 0; n < N; n++) out[(int64_t)t * N + n] = (float)acc[n];
  }
  free(acc); free(y);
}

/* ---------------------------------------- f32 restatement of the kernels */

#define K_LANES 32

/* tileDots (moeQuantW.ts:73-83) for one column: dot(x, deqVec4(word)) in f32,
 * the four products added left to right. */
static inline float col_dot(const float *x4, uint32_t word, int off, int bits) {
  float d[4];
  for (int r = 0; r < 4; r++) {
    int32_t raw = (int32_t)((word >> (off + r * bits)) & ((1u << bits) - 1u));
    if (raw >= (1 << (bits - 1))) raw -= (1 << bits);
    d[r] = (float)raw;
  }
  return ((x4[0] * d[0] + x4[1] * d[1]) + x4[2] * d[2]) + x4[3] * d[3];
}

/* One lane's share of a K-split dot for unit `unit` (4 columns): k4 = lane,
 * lane + 32, … (moeQuantW.ts:141-161, :209-220). */
static void lane_dots(const float *xrow, const uint32_t *w, const float *sc, int K, int N, int bits,
                      int g, int e, int unit, int lane, float out[4]) {
  int n4 = N / 4, k4count = K / 4, tile_words = bits / 2, g4 = g / 4, kg = K / g;
  int64_t wbase = ((int64_t)e * n4 + unit) * k4count * tile_words;
  int64_t srow = (int64_t)e * kg;
  for (int c = 0; c < 4; c++) out[c] = 0.0f;
  for (int k4 = lane; k4 < k4count; k4 += K_LANES) {
    const float *x4 = xrow + 4 * k4;
    int64_t s = (srow + k4 / g4) * n4 + unit;
    int64_t tb = wbase + (int64_t)k4 * tile_words;
    for (int c = 0; c < 4; c++) {
      float dv = col_dot(x4, w[tb + (c * bits * 4) / 32], (c * bits * 4) % 32, bits);
      out[c] += dv * sc[s * 4 + c];
    }
  }
}

/* mergeLanes (moeQuantW.ts:93-105): strides 16, 8, 4, 2, 1; lane l adds
 * lane l + stride. */
static void merge_lanes(float p[K_LANES][4]) {
  for (int stride = K_LANES / 2; stride >= 1; stride >>= 1)
    for (int l = 0; l < stride; l++)
      for (int c = 0; c < 4; c++) p[l][c] = p[l][c] + p[l + stride][c];
}

/* moeUpKernel (moeQuantW.ts:122-175) in f32. Like the reference's grid, every
 * (row, 4-column unit) is independent: they run in parallel. */
EXPORT void orc_moe_up_f32ref(const float *x, const float *route, const uint32_t *glu_w,
                              const float *glu_s, const float *glu_b, const uint32_t *lin_w,
                              const float *lin_s, const float *lin_b, int T, int K, int N, int E,
                              int k, int bits, int g, float *act) {
  int64_t rows = (int64_t)T * k;
  int n4 = N / 4;
#pragma omp parallel for schedule(dynamic, 8)
  for (int64_t ru = 0; ru < rows * n4; ru++) {
    int64_t row = ru / n4;
    int unit = (int)(ru % n4);
    int t = (int)(row / k), s = (int)(row % k);
    float *arow = act + row * N;
    int e = route_id(route, t, k, s, E);
    if (e < 0) { for (int c = 0; c < 4; c++) arow[unit * 4 + c] = 0.0f; continue; }
    float pa[K_LANES][4], pb[K_LANES][4];
    for (int lane = 0; lane < K_LANES; lane++) {
      lane_dots(x + (int64_t)t * K, glu_w, glu_s, K, N, bits, g, e, unit, lane, pa[lane]);
      lane_dots(x + (int64_t)t * K, lin_w, lin_s, K, N, bits, g, e, unit, lane, pb[lane]);
    }
    merge_lanes(pa);
    merge_lanes(pb);
    for (int c = 0; c < 4; c++) {
      int n = unit * 4 + c;
      float gb = glu_b ? glu_b[(int64_t)e * N + n] : 0.0f;
      float lb = lin_b ? lin_b[(int64_t)e * N + n] : 0.0f;
      arow[n] = swiglu_f32(pa[0][c] + gb, pb[0][c] + lb);
    }
  }
}

/* moeDownKernel (moeQuantW.ts:188-237) in f32: per slot a K-split dot scaled
 * by its gate, lanes merged, then residual and the gate-weighted biases.
 * Every (token, unit) is independent: they run in parallel. */
EXPORT void orc_moe_down_f32ref(const float *act, const float *route, const uint32_t *w,
                                const float *sc, const float *bias, const float *residual, int T,
                                int K, int N, int E, int k, int bits, int g, float *out) {
  int n4 = N / 4;
#pragma omp parallel for schedule(dynamic, 8)
  for (int64_t tu = 0; tu < (int64_t)T * n4; tu++) {
    int t = (int)(tu / n4);
    int unit = (int)(tu % n4);
    float p[K_LANES][4];
    for (int lane = 0; lane < K_LANES; lane++) {
      float acc[4] = {0, 0, 0, 0};
      for (int s = 0; s < k; s++) {
        int e = route_id(route, t, k, s, E);
        if (e < 0) continue;
        float gate = route[(int64_t)t * 2 * k + k + s];
        float dot[4];
        lane_dots(act + ((int64_t)t * k + s) * K, w, sc, K, N, bits, g, e, unit, lane, dot);
        for (int c = 0; c < 4; c++) acc[c] += dot[c] * gate;
      }
      for (int c = 0; c < 4; c++) p[lane][c] = acc[c];
    }
    merge_lanes(p);
    for (int c = 0; c < 4; c++) {
      int n = unit * 4 + c;
      float sum = p[0][c] + (residual ? residual[(int64_t)t * N + n] : 0.0f);
      for (int s = 0; s < k; s++) {
        int e = route_id(route, t, k, s, E);
        if (e < 0 || !bias) continue;
        sum += bias[(int64_t)e * N + n] * route[(int64_t)t * 2 * k + k + s];
      }
      out[(int64_t)t * N + n] = sum;
    }
  }
}

/* ------------------------------------------------------------- dispatch */

/* The dispatch permutation has no reference function: the reference reads
 * each (token, slot) row's expert weights directly (moeQuantW.ts:131-134).
 * This build defines it as the stable counting sort of assignment index
 * a = t·k + s by expert id: offsets[e] = Σ_{e' < e} count(e'), and within an
 * expert, assignments keep ascending a. perm[pos] = a, inv[a] = pos; an
 * assignment whose id is not an expert index is left out (inv = −1). */
EXPORT void orc_dispatch(const float *route, int T, int k, int E, int32_t *perm, int32_t *inv,
                         int32_t *offsets) {
  int64_t A = (int64_t)T * k;
  int32_t *cursor = calloc((size_t)E + 1, sizeof(int32_t));
  for (int e = 0; e <= E; e++) offsets[e] = 0;
  for (int64_t a = 0; a < A; a++) {
    int e = route_id(route, (int)(a / k), k, (int)(a % k), E);
    if (e >= 0) offsets[e + 1]++;
  }
  for (int e = 0; e < E; e++) offsets[e + 1] += offsets[e];
  for (int e = 0; e < E; e++) cursor[e] = offsets[e];
  for (int64_t a = 0; a < A; a++) {
    int e = route_id(route, (int)(a / k), k, (int)(a % k), E);
    if (e < 0) { inv[a] = -1; continue; }
    int32_t pos = cursor[e]++;
    perm[pos] = (int32_t)a;
    inv[a] = pos;
  }
  for (int64_t p = offsets[E]; p < A; p++) perm[p] = -1;
  free(cursor);
}

/* -------------------------------------------------------------- the layer */

/* EagerMoeMlp.forward's routed part (src/zoo/privacy-filter/moeMlp.ts:82-121)
 * on an already-normalised input: router → topk → moeUp → moeDown, with the
 * residual added by moeDown. act is kept in f32 between the two products, as
 * the reference keeps it. x_res may equal NULL (zero residual). */
EXPORT void orc_moe_layer_f64(const float *x, const float *router_w, const float *router_b,
                              const uint32_t *glu_w, const float *glu_s, const float *glu_b,
                              const uint32_t *lin_w, const float *lin_s, const float *lin_b,
                              const uint32_t *down_w, const float *down_s, const float *down_b,
                              const float *residual, int T, int d, int I, int E, int k, int bits,
                              int g_up, int g_down, float *route, float *act, float *out) {
  float *logits = malloc(sizeof(float) * (size_t)T * E);
  orc_router_logits(x, router_w, router_b, T, d, E, logits);
  orc_topk(logits, T, E, k, route);
  free(logits);
  orc_moe_up_f64(x, route, glu_w, glu_s, glu_b, lin_w, lin_s, lin_b, T, d, I, E, k, bits, g_up, act);
  orc_moe_down_f64(act, route, down_w, down_s, down_b, residual, T, I, d, E, k, bits, g_down, out);
}

/* ------------------------------------------------------------------ norm */

/* src/core/graph/ops/reduce.ts:61-92 and src/core/kernels/reduce/rmsNorm.ts
 * :84-140 — rmsNorm(x, weight, eps, {group, residual, scale}): over each
 * run of `group` columns, inv = 1/sqrt(Σx²/group + eps), then
 * v = x·inv·w (left to right), v = v + residual, out = v·scale.
 * The sum follows this library's canonical f32 order (the reference sums in
 * a device-dependent subgroup or tree order): 64 lane sums, lane l adding
 * x·x for the quads q ≡ l (mod 64) of the run in ascending order (within a
 * quad ascending), no fused multiply-add; then an xor butterfly over the
 * lane sums, strides 32, 16, …, 1, read at lane 0; every operation one IEEE
 * f32 rounding. w is `group` long (shared by every run) or `cols` long (a
 * slice per run). Inputs and outputs are f32; an f16 caller rounds them. */
EXPORT void orc_rmsnorm(const float *x, int64_t rows, int cols, int group, const float *w,
                        int wlen, float eps, const float *res, float scale, float *out) {
  float lanes[64];
  for (int64_t r = 0; r < rows; r++)
    for (int g0 = 0; g0 < cols; g0 += group) {
      const float *xr = x + r * cols + g0;
      for (int l = 0; l < 64; l++) {
        float s = 0.0f;
        for (int q = l; 4 * q < group; q += 64)
          for (int j = 0; j < 4; j++) {
            int i = 4 * q + j;
            if (i < group) {
              float sq = xr[i] * xr[i];
              s = s + sq;
            }
          }
        lanes[l] = s;
      }
      for (int m = 32; m >= 1; m >>= 1) {
        float nxt[64];
        for (int l = 0; l < 64; l++) nxt[l] = lanes[l] + lanes[l ^ m];
        memcpy(lanes, nxt, sizeof(lanes));
      }
      float mean = lanes[0] / (float)group;
      float inv = 1.0f / sqrtf(mean + eps);
      const float *wr = wlen == group ? w : w + g0;
      for (int i = 0; i < group; i++) {
        float v = xr[i] * inv;
        v = v * wr[i];
        if (res) v = v + res[r * cols + g0 + i];
        v = v * scale;
        out[r * cols + g0 + i] = v;
      }
    }
}
