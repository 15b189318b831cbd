// Attention ops of the privacy-filter block for gfx950: the rotary
// embedding and banded GQA attention with sinks.
//
// Reference: src/core/graph/ops/attention.ts:28-145 (sdpa: band mask
// qPos − windowLeft ≤ j ≤ qPos + windowRight, qPos = qPosOffset + i, GQA,
// sinks, segments, key bias), :146-214 (sdpaPacked: q, k, v as column
// blocks of one tensor), :220-262 (rope); kernels src/core/kernels/
// attention/rope.ts:14-68 and attn.ts; the semantics pinned by the
// reference's f64 check test/core/kernels/attention/checkSdpa.ts:55-103:
// q and k arrive pre-scaled, a sink adds exp(sink · ln 2) to the softmax
// denominator alone, a row that sees no key (and has no sink) is 0.
//
// sdpa: one block of 8 wavefronts per (group of query rows, kv head). The
// block's items are (row, query head of this kv head), at most 8 per
// wavefront; the keys its rows can see are staged 64 at a time into LDS as
// f32 (K and V rows padded to a 16-byte bank shift). Per chunk a wavefront
// holds 64 keys' K rows in registers (lane = key) to score each of its
// items, updates the item's online softmax (running max m, sum l), and
// accumulates P·V with lane = output column, the weights read from the
// scoring lanes with readlane. Sums are f32; exp is expf.
#include "moe_internal.h"

#include <math.h>

#include <type_traits>

namespace {

constexpr int WAVE = 64;
constexpr int AW = 8;        // wavefronts per block
constexpr int AI = 8;        // items per wavefront
constexpr int AKC = 64;      // keys per chunk
constexpr float LN2 = 0.69314718055994530942f;

__device__ __forceinline__ float ld(const float *p, int64_t i) { return p[i]; }
__device__ __forceinline__ float ld(const _Float16 *p, int64_t i) { return (float)p[i]; }
__device__ __forceinline__ void st(float *p, int64_t i, float v) { p[i] = v; }
__device__ __forceinline__ void st(_Float16 *p, int64_t i, float v) { p[i] = (_Float16)v; }

// Element x of a head row after rope (rope.ts:55-66): pair (x0, x1) =
// (x & ~1, x | 1), out[2p] = x0·c − x1·s, out[2p+1] = x1·c + x0·s; c and s
// are the pair-duplicated table entries of the element's row.
template <typename T>
__device__ __forceinline__ float roped(const T *p, int64_t i, int x, float c, float s) {
  const int64_t pair = i - (x & 1);
  const float x0 = ld(p, pair), x1 = ld(p, pair + 1);
  return (x & 1) ? x1 * c + x0 * s : x0 * c - x1 * s;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 1; m < WAVE; m <<= 1) v = fmaxf(v, __shfl_xor(v, m));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 1; m < WAVE; m <<= 1) v += __shfl_xor(v, m);
  return v;
}
__device__ __forceinline__ float lane_f(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// rope.ts:14-68: one thread per (row, pair) of the output window.
template <typename T>
__global__ void k_rope(const T *__restrict__ x, const float *__restrict__ cs,
                       const float *__restrict__ sn, T *__restrict__ out, int rows, int cols,
                       int hd, int src_start, int width) {
  const int64_t pairs = width / 2;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)rows * pairs) return;
  const int64_t row = idx / pairs;
  const int col0 = (int)(idx - row * pairs) * 2;
  const int dcol = col0 % hd;
  const float c = cs[row * hd + dcol], s = sn[row * hd + dcol];
  const int64_t src = row * cols + src_start + col0;
  const float x0 = ld(x, src), x1 = ld(x, src + 1);
  st(out, row * width + col0, x0 * c - x1 * s);
  st(out, row * width + col0 + 1, x1 * c + x0 * s);
}

// NS 64-column slabs of the head (head_dim ≤ 64·NS).
template <typename T, int NS>
__global__ __launch_bounds__(AW *WAVE) void k_sdpa(AttnArgs a) {
  constexpr int HP = 64 * NS;   // padded head width
  constexpr int KST = HP + 4;   // LDS row stride of K and V (floats)
  extern __shared__ __align__(16) float smem[];
  float *qs = smem;                    // [AW·AI][HP]
  float *ks = qs + AW * AI * HP;       // [AKC][KST]
  float *vs = ks + AKC * KST;          // [AKC][KST]

  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = threadIdx.x / WAVE;
  const int G = a.q_heads / a.kv_heads;
  const int R = a.rows_per_block;
  const int row0 = blockIdx.x * R;
  const int kvh = blockIdx.y;
  const int hd = a.head_dim;
  const T *q = (const T *)a.q;
  const T *k = (const T *)a.k;
  const T *v = (const T *)a.v;
  T *out = (T *)a.out;

  // Items: it = wave + AW·i → row it / G, head kvh·G + it % G.
  const int nitems = min(R, a.q_len - row0) * G;
  // Staging (q here, K and V per chunk below): 8 elements per thread at a
  // time, their loads issued before the LDS stores, from indices clamped
  // into the tensors (values past them zeroed), so no load sits under a
  // branch; rope or not is one uniform choice around the whole loop. (A
  // load and store per strided iteration waited out each load in turn.)
  constexpr int NT = AW * WAVE;    // threads per block
  constexpr int PER = AKC * HP / NT;  // = AW·AI·HP / NT: elements per thread
  static_assert(AKC == AW * AI && PER % 8 == 0, "staging shape");
  auto stage_q = [&](auto rope) {
#pragma unroll
    for (int b0 = 0; b0 < PER; b0 += 8) {
      float qv[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int e = threadIdx.x + NT * (b0 + u), it = e / HP, x = e % HP;
        const int itc = min(it, nitems - 1), xc = min(x, hd - 1);
        const int r = row0 + itc / G, h = kvh * G + itc % G;
        const int64_t qi = (int64_t)r * a.q_rs + (int64_t)h * hd + xc;
        float val;
        if constexpr (decltype(rope)::value)
          val = roped(q, qi, xc, a.rope_cos[(int64_t)r * hd + xc], a.rope_sin[(int64_t)r * hd + xc]);
        else
          val = ld(q, qi);
        qv[u] = (it < nitems && x < hd) ? val : 0.f;
      }
#pragma unroll
      for (int u = 0; u < 8; u++) qs[threadIdx.x + NT * (b0 + u)] = qv[u];
    }
  };
  if (a.rope_cos) stage_q(std::true_type{});
  else stage_q(std::false_type{});

  // The rows' key ranges.
  auto range = [&](int r, int &lo, int &hi) {
    const long long qpos = (long long)a.q_pos_offset + r;
    long long l = a.window_left < 0 ? 0 : qpos - a.window_left;
    long long hgh = a.window_right < 0 ? (long long)a.kv_len - 1 : qpos + a.window_right;
    if (l < 0) l = 0;
    if (hgh > a.kv_len - 1) hgh = a.kv_len - 1;
    if (a.segs) {
      const long long s0 = (long long)a.segs[2 * r], s1 = (long long)a.segs[2 * r + 1] - 1;
      if (s0 > l) l = s0;
      if (s1 < hgh) hgh = s1;
    }
    lo = (int)l;
    hi = (int)(hgh < l - 1 ? l - 1 : hgh);  // empty: hi < lo
  };
  int lo_i[AI], hi_i[AI];
  bool ok_i[AI];
  float m_i[AI], l_i[AI], acc[AI][NS];
#pragma unroll
  for (int i = 0; i < AI; i++) {
    const int it = wave + AW * i;
    ok_i[i] = it < nitems;
    lo_i[i] = 0;
    hi_i[i] = -1;
    if (ok_i[i]) range(row0 + it / G, lo_i[i], hi_i[i]);
    m_i[i] = -INFINITY;
    l_i[i] = 0.f;
#pragma unroll
    for (int sl = 0; sl < NS; sl++) acc[i][sl] = 0.f;
  }
  // The block's key span: the union of its rows' ranges.
  int blo = 0x7fffffff, bhi = -1;
  for (int r = row0; r < min(a.q_len, row0 + R); r++) {
    int l, h;
    range(r, l, h);
    if (h >= l) {
      blo = min(blo, l);
      bhi = max(bhi, h);
    }
  }

  for (int c0 = blo; c0 <= bhi; c0 += AKC) {
    __syncthreads();  // the previous chunk's reads are done (and qs is written)
    auto stage_kv = [&](auto rope) {
#pragma unroll
      for (int b0 = 0; b0 < PER; b0 += 8) {
        float kv[8], vv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
          const int e = threadIdx.x + NT * (b0 + u), j = e / HP, x = e % HP;
          const int key = c0 + j;
          const int kc = min(key, bhi), xc = min(x, hd - 1);  // c0 ≤ kc ≤ bhi < kv_len
          const int64_t ki = (int64_t)kc * a.k_rs + (int64_t)kvh * hd + xc;
          float kval;
          if constexpr (decltype(rope)::value)
            kval = roped(k, ki, xc, a.rope_cos[(int64_t)kc * hd + xc],
                         a.rope_sin[(int64_t)kc * hd + xc]);
          else
            kval = ld(k, ki);
          const float vval = ld(v, (int64_t)kc * a.v_rs + (int64_t)kvh * hd + xc);
          const bool in = key <= bhi && x < hd;
          kv[u] = in ? kval : 0.f;
          vv[u] = in ? vval : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
          const int e = threadIdx.x + NT * (b0 + u), j = e / HP, x = e % HP;
          ks[j * KST + x] = kv[u];
          vs[j * KST + x] = vv[u];
        }
      }
    };
    if (a.rope_cos) stage_kv(std::true_type{});
    else stage_kv(std::false_type{});
    __syncthreads();
    const int key = c0 + lane;
    float s[AI];
#pragma unroll
    for (int i = 0; i < AI; i++) s[i] = 0.f;
    bool live[AI];
#pragma unroll
    for (int i = 0; i < AI; i++) live[i] = ok_i[i] && lo_i[i] <= c0 + AKC - 1 && hi_i[i] >= c0;
    // Scores: lane = key, the key's K row in registers, q broadcast from LDS.
#pragma unroll
    for (int sl = 0; sl < NS; sl++) {
      float kr[64];
#pragma unroll
      for (int x = 0; x < 64; x += 4) {
        const float4 t = *(const float4 *)&ks[lane * KST + sl * 64 + x];
        kr[x] = t.x;
        kr[x + 1] = t.y;
        kr[x + 2] = t.z;
        kr[x + 3] = t.w;
      }
#pragma unroll
      for (int i = 0; i < AI; i++) {
        if (!live[i]) continue;
        const float *qr = qs + (wave + AW * i) * HP + sl * 64;
        // Two chains (even and odd columns) halve the dependent FMA latency.
        float d0 = 0.f, d1 = 0.f;
#pragma unroll
        for (int x = 0; x < 64; x += 4) {
          const float4 t = *(const float4 *)&qr[x];
          d0 = fmaf(t.x, kr[x], d0);
          d1 = fmaf(t.y, kr[x + 1], d1);
          d0 = fmaf(t.z, kr[x + 2], d0);
          d1 = fmaf(t.w, kr[x + 3], d1);
        }
        s[i] += d0 + d1;
      }
    }
    // Online softmax per item.
    float p[AI];
#pragma unroll
    for (int i = 0; i < AI; i++) {
      p[i] = 0.f;
      if (!live[i]) continue;
      const bool vis = key >= lo_i[i] && key <= hi_i[i];
      float sc = s[i];
      if (a.has_kb && key >= a.kb_start && key < a.kb_end) sc += a.kb_value;
      sc = vis ? sc : -INFINITY;
      const float mc = wave_max(sc);
      const float mn = fmaxf(m_i[i], mc);
      if (mn == -INFINITY) continue;
      const float scale = m_i[i] == -INFINITY ? 0.f : expf(m_i[i] - mn);
      p[i] = vis ? expf(sc - mn) : 0.f;
      l_i[i] = l_i[i] * scale + wave_sum(p[i]);
#pragma unroll
      for (int sl = 0; sl < NS; sl++) acc[i][sl] *= scale;
      m_i[i] = mn;
    }
    // P·V: lane = output column, V column in registers.
#pragma unroll
    for (int sl = 0; sl < NS; sl++) {
      float vr[AKC];
#pragma unroll
      for (int j = 0; j < AKC; j++) vr[j] = vs[j * KST + sl * 64 + lane];
#pragma unroll
      for (int i = 0; i < AI; i++) {
        if (!live[i]) continue;
        float o0 = 0.f, o1 = 0.f;
#pragma unroll
        for (int j = 0; j < AKC; j += 2) {
          o0 = fmaf(lane_f(p[i], j), vr[j], o0);
          o1 = fmaf(lane_f(p[i], j + 1), vr[j + 1], o1);
        }
        acc[i][sl] += o0 + o1;
      }
    }
  }

  // Sinks join the denominator; store.
#pragma unroll
  for (int i = 0; i < AI; i++) {
    if (!ok_i[i]) continue;
    const int it = wave + AW * i;
    const int r = row0 + it / G, h = kvh * G + it % G;
    const float sg = a.sinks ? a.sinks[h] * LN2 : -INFINITY;
    const float mf = fmaxf(m_i[i], sg);
    float scale = 0.f, inv = 0.f;
    if (mf != -INFINITY) {
      scale = m_i[i] == -INFINITY ? 0.f : expf(m_i[i] - mf);
      const float l = l_i[i] * scale + (a.sinks ? expf(sg - mf) : 0.f);
      inv = 1.0f / l;
    }
#pragma unroll
    for (int sl = 0; sl < NS; sl++) {
      const int x = sl * 64 + lane;
      if (x < hd) st(out, (int64_t)r * a.o_rs + (int64_t)h * hd + x, acc[i][sl] * scale * inv);
    }
  }
}

}  // namespace

int launch_rope(const void *x, moe_dtype dt, int rows, int cols, int hd, int src_start, int width,
                const float *cs, const float *sn, void *out, hipStream_t s) {
  MOE_NONNULL(x);
  MOE_NONNULL(cs);
  MOE_NONNULL(sn);
  MOE_NONNULL(out);
  const int64_t n = (int64_t)rows * (width / 2);
  const int64_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffff) return moe_fail(MOE_INVALID_ARGUMENT, "rope: input too large");
  if (dt == MOE_F16)
    hipLaunchKernelGGL(k_rope<_Float16>, dim3((unsigned)blocks), dim3(256), 0, s,
                       (const _Float16 *)x, cs, sn, (_Float16 *)out, rows, cols, hd, src_start,
                       width);
  else
    hipLaunchKernelGGL(k_rope<float>, dim3((unsigned)blocks), dim3(256), 0, s, (const float *)x, cs,
                       sn, (float *)out, rows, cols, hd, src_start, width);
  return 0;
}

int launch_sdpa(AttnArgs a, hipStream_t s) {
  MOE_NONNULL(a.q);
  MOE_NONNULL(a.k);
  MOE_NONNULL(a.v);
  MOE_NONNULL(a.out);
  const int G = a.q_heads / a.kv_heads;
  if (G > AW * AI)
    return moe_fail(MOE_INVALID_ARGUMENT, "sdpa: more than " + std::to_string(AW * AI) +
                                              " query heads per kv head");
  // Rows per block: up to the 64 items a block holds, fewer for short
  // sequences so that the grid still has ~512 blocks (each block stages its
  // keys once; more rows per block share more of them).
  const int max_rows = (AW * AI) / G;
  const long want = ((long)a.q_len * a.kv_heads + 511) / 512;
  a.rows_per_block = (int)std::max(1L, std::min((long)max_rows, want));
  const int ns = a.head_dim <= 64 ? 1 : 2;
  const size_t lds = (size_t)(AW * AI * 64 * ns + 2 * AKC * (64 * ns + 4)) * 4;
  dim3 grid((a.q_len + a.rows_per_block - 1) / a.rows_per_block, a.kv_heads), block(AW * WAVE);
  // Dynamic LDS past 64 KB (the two-slab kernels) needs the kernel's limit raised.
  static bool raised = false;
  if (!raised) {
    const int big = (AW * AI * 128 + 2 * AKC * 132) * 4;
    if (hipFuncSetAttribute((const void *)k_sdpa<_Float16, 2>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, big) != hipSuccess ||
        hipFuncSetAttribute((const void *)k_sdpa<float, 2>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, big) != hipSuccess)
      return moe_fail(MOE_EXECUTION_FAILED, "sdpa: cannot raise the LDS limit of the kernel");
    raised = true;
  }
  if (a.dtype == MOE_F16) {
    if (ns == 1) hipLaunchKernelGGL((k_sdpa<_Float16, 1>), grid, block, lds, s, a);
    else hipLaunchKernelGGL((k_sdpa<_Float16, 2>), grid, block, lds, s, a);
  } else {
    if (ns == 1) hipLaunchKernelGGL((k_sdpa<float, 1>), grid, block, lds, s, a);
    else hipLaunchKernelGGL((k_sdpa<float, 2>), grid, block, lds, s, a);
  }
  return 0;
}
