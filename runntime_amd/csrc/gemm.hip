// Grouped expert GEMM for prefill shapes (many rows per expert) on gfx950.
//
// Reference: src/core/kernels/matmul/moeQuantW.ts:122-175 (moeUp) and
// :188-237 (moeDown); quantW layout src/core/kernels/quantCommon.ts:8-31.
// Same results as the expert kernels of expert.hip; this one is shaped for
// rows per expert in the hundreds.
//
// Work: for every active expert e (rows grouped by the dispatch), C_e =
// A_e · W_e with A_e the expert's gathered input rows (x for up, act for
// down) and W_e its int8 weights. Up computes glu and lin for the same
// outputs in one tile (64 glu + 64 lin columns) and applies the SwiGLU in the
// epilogue; down adds the bias.
//
// Tiles: 128 rows × 128 columns × 64-wide K steps, 4 wavefronts in a 2×2
// grid, each with 2×2 v_mfma_f32_32x32x16_f16 tiles (64 × 64). Per K step the
// block loads the int8 weight tiles (8 KB) and the gathered A rows into
// registers one step ahead, then converts and stores them to LDS: weights
// dequantized to f16 (exact: |q| ≤ 127), A as f16, or for f32 input as f16
// hi + lo planes (two MFMAs; ~2^-22 relative). Scales (one per column and K
// group) and biases run in the epilogue.
//
// Order of tiles: expert, then N-tile, then M-tile, so the M-tiles of one
// (expert, N-tile) — which share its weights — run back to back; blocks are
// then dealt to the 8 XCDs in contiguous ranges (block b runs on XCD b mod 8),
// so those neighbours share one L2.
#include "moe_internal.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int WAVE = 64;
constexpr int BM = GEMM_TILE_M;  // 128
constexpr int BN = 128;
constexpr int BK = 64;
constexpr int LDK = BK + 8;  // LDS row stride (halves): +16 B shifts rows 4 banks

struct GemmArgs {
  const void *a;
  int a_row_div;
  const uint32_t *w0;  // glu (up) or down
  const float *s0;
  const float *b0;
  const uint32_t *w1;  // lin (up)
  const float *s1;
  const float *b1;
  int K, N, E, g;      // N: output columns (up: I, per projection)
  float *out;
  const int32_t *perm;
  const int32_t *active;  // [E][4] {e, first row, rows, first M-tile}
  const int32_t *meta;
  int nt;                 // N-tiles
};

__device__ __forceinline__ float swiglu(float glu, float lin) {
  // activations.ts:127-133: g = min(glu, 7), l = clamp(lin, ±7).
  float g = fminf(glu, 7.0f);
  float l = fminf(fmaxf(lin, -7.0f), 7.0f);
  return (g / (1.0f + expf(-1.702f * g))) * (l + 1.0f);
}

// Two quantW column words (4 rows each, consecutive in K) → 8 f16 in K
// order. Byte b becomes f16(1024 + (b ^ 0x80)), minus 1152 gives b.
__device__ __forceinline__ half8 cvt_i8x8(uint32_t w0, uint32_t w1) {
  const half2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  uint32_t x0 = w0 ^ 0x80808080u, x1 = w1 ^ 0x80808080u;
  half2v h0 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u)) - bias;
  half2v h1 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u)) - bias;
  half2v h2 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u)) - bias;
  half2v h3 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u)) - bias;
  half8 r;
  r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
  r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
  return r;
}

// Global loads of one K step: this thread's weight bytes and A elements.
template <typename AT>
struct Prefetch {
  uint4 w[2];                                   // 32 B: two quantW tiles of one unit
  uint4 a[sizeof(AT) == 4 ? 8 : 4];             // 32 consecutive k of one A row
};

template <int MODE, typename AT>
__global__ __launch_bounds__(256) void k_expert_gemm(GemmArgs p) {
  constexpr bool SPLIT = sizeof(AT) == 4;
  constexpr int PLANES = SPLIT ? 2 : 1;
  __shared__ __align__(16) _Float16 As[PLANES][BM * LDK];
  __shared__ __align__(16) _Float16 Bs[BN * LDK];

  // ---- which tile: XCD-contiguous block order (gridDim.x is a multiple of
  // 8), then expert / N / M.
  const int nblk = gridDim.x;
  const int b = blockIdx.x;
  const int per_xcd = (nblk + 7) / 8;
  const int L = (b % 8) * per_xcd + b / 8;
  const int total_tiles = p.meta[META_TILES];
  if (L >= total_tiles * p.nt) return;
  const int n_active = p.meta[META_ACTIVE];
  const int t = L / p.nt;  // global M-tile index of this tile's expert range
  int lo = 0, hi = n_active - 1;
  while (lo < hi) {  // last active expert whose first M-tile ≤ t
    const int mid = (lo + hi + 1) >> 1;
    if (p.active[4 * mid + 3] <= t) lo = mid; else hi = mid - 1;
  }
  const int4 desc = ((const int4 *)p.active)[lo];
  const int e = desc.x, row0 = desc.y, cnt = desc.z, tile0 = desc.w;
  const int mt = (cnt + BM - 1) / BM;
  const int local = L - tile0 * p.nt;
  const int ntile = local / mt;
  const int mtile = local % mt;
  const int m0 = mtile * BM;
  const int rows = min(BM, cnt - m0);

  const int tid = threadIdx.x;
  const int lane = tid & (WAVE - 1);
  const int wave = tid / WAVE;
  const int wm = wave >> 1, wn = wave & 1;
  const int N4 = p.N / 4, K4 = p.K / 4;
  const int ksteps = p.K / BK;

  // ---- this thread's share of the staging
  // Weights: unit ut (of the tile's 32), tiles 2·tp, 2·tp + 1 of the K step.
  const int ut = tid >> 3, tp = tid & 7;
  const uint32_t *wsrc;
  int ucol;  // first of the unit's 4 columns in the tile's B (0..127)
  if (MODE == MODE_UP) {
    const bool second = ut >= 16;  // lin units follow the glu units
    const int u = ntile * 16 + (ut & 15);
    wsrc = (second ? p.w1 : p.w0) + ((int64_t)e * N4 + u) * K4 * 4;
    ucol = (second ? 64 : 0) + (ut & 15) * 4;
  } else {
    const int u = ntile * 32 + ut;
    wsrc = p.w0 + ((int64_t)e * N4 + u) * K4 * 4;
    ucol = ut * 4;
  }
  // A: row ar of the tile, 32 consecutive k from ak.
  const int ar = tid >> 1, ak = (tid & 1) * 32;
  const bool arow_ok = ar < rows;
  const int64_t asrc_row = arow_ok ? p.perm[row0 + m0 + ar] / p.a_row_div : 0;
  const AT *asrc = (const AT *)p.a + asrc_row * p.K + ak;

  auto load = [&](int ks, Prefetch<AT> &f) {
    const uint4 *wp = (const uint4 *)wsrc + ks * (BK / 4) + 2 * tp;
    f.w[0] = wp[0];
    f.w[1] = wp[1];
    const uint4 *ap = (const uint4 *)(asrc + ks * BK);
#pragma unroll
    for (int i = 0; i < (SPLIT ? 8 : 4); i++) f.a[i] = arow_ok ? ap[i] : uint4{0, 0, 0, 0};
  };
  auto store = [&](const Prefetch<AT> &f) {
    // weights: 4 columns × 8 k each, k contiguous per column
    const uint32_t w0[4] = {f.w[0].x, f.w[0].y, f.w[0].z, f.w[0].w};
    const uint32_t w1[4] = {f.w[1].x, f.w[1].y, f.w[1].z, f.w[1].w};
#pragma unroll
    for (int c = 0; c < 4; c++)
      *(half8 *)&Bs[(ucol + c) * LDK + tp * 8] = cvt_i8x8(w0[c], w1[c]);
    // A
    if (SPLIT) {
      const float *v = (const float *)f.a;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        half8 h, l;
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const float x = v[8 * j + i];
          const _Float16 xh = (_Float16)x;
          h[i] = xh;
          l[i] = (_Float16)(x - (float)xh);
        }
        *(half8 *)&As[0][ar * LDK + ak + 8 * j] = h;
        *(half8 *)&As[PLANES - 1][ar * LDK + ak + 8 * j] = l;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; j++) *(uint4 *)&As[0][ar * LDK + ak + 8 * j] = f.a[j];
    }
  };

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  // MFMA operands: lane L reads row (or column) L%32, k 8·(L/32) .. +7 of a
  // 16-wide K slice.
  const int fr = lane & 31, fk = (lane >> 5) * 8;
  // B column tiles of this wavefront: up → glu cols 32·wn.. and the lin cols
  // at +64 (so each wavefront holds matching glu/lin sums); down → 64·wn, +32.
  const int bc0 = MODE == MODE_UP ? 32 * wn : 64 * wn;
  const int bc1 = MODE == MODE_UP ? 64 + 32 * wn : 64 * wn + 32;

  Prefetch<AT> f;
  load(0, f);
  for (int ks = 0; ks < ksteps; ks++) {
    __syncthreads();  // the previous step's LDS reads are done
    store(f);
    __syncthreads();
    if (ks + 1 < ksteps) load(ks + 1, f);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      half8 bf[2];
      bf[0] = *(const half8 *)&Bs[(bc0 + fr) * LDK + kk + fk];
      bf[1] = *(const half8 *)&Bs[(bc1 + fr) * LDK + kk + fk];
#pragma unroll
      for (int pl = 0; pl < PLANES; pl++) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
          const half8 af = *(const half8 *)&As[pl][(wm * 64 + i * 32 + fr) * LDK + kk + fk];
#pragma unroll
          for (int j = 0; j < 2; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf[j], acc[i][j], 0, 0, 0);
        }
      }
    }
  }

  // ---- epilogue. acc[i][j][r]: row wm·64 + 32i + 8(r/4) + 4(L/32) + r%4,
  // column (of tile j) L%32.
  const int kg = p.K / p.g;  // the GEMM path runs with one scale group
  (void)kg;
  if (MODE == MODE_UP) {
    const int col = ntile * 64 + 32 * wn + fr;  // output column (glu index = lin index)
    const float sg = p.s0[(int64_t)e * p.N + col], sl = p.s1[(int64_t)e * p.N + col];
    const float bg = p.b0 ? p.b0[(int64_t)e * p.N + col] : 0.f;
    const float bl = p.b1 ? p.b1[(int64_t)e * p.N + col] : 0.f;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = wm * 64 + i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
        if (row < rows) {
          const int64_t asg = p.perm[row0 + m0 + row];
          p.out[asg * p.N + col] = swiglu(acc[i][0][r] * sg + bg, acc[i][1][r] * sl + bl);
        }
      }
  } else {
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int col = ntile * BN + (j == 0 ? bc0 : bc1) + fr;
      const float sc = p.s0[(int64_t)e * p.N + col];
      const float bb = p.b0 ? p.b0[(int64_t)e * p.N + col] : 0.f;
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int row = wm * 64 + i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
          if (row < rows) {
            const int64_t asg = p.perm[row0 + m0 + row];
            p.out[asg * p.N + col] = acc[i][j][r] * sc + bb;
          }
        }
    }
  }
}

}  // namespace

bool gemm_eligible(const ExpertArgs &ea) {
  // One scale group per column, K in whole steps, N in whole tiles.
  const int tile_cols = ea.mode == MODE_UP ? 64 : BN;
  return ea.bits == 8 && ea.g == ea.K && ea.K % BK == 0 && ea.N % tile_cols == 0;
}

int launch_expert_gemm(const ExpertArgs &ea, const DispatchBufs &db, hipStream_t s) {
  if (ea.calls != 1)
    return moe_fail(MOE_EXECUTION_FAILED, "expert gemm: one call per launch");
  GemmArgs p;
  p.a = ea.a;
  p.a_row_div = ea.a_row_div;
  p.w0 = ea.w0.w;
  p.s0 = ea.w0.scales;
  p.b0 = ea.w0.bias;
  p.w1 = ea.w1.w;
  p.s1 = ea.w1.scales;
  p.b1 = ea.w1.bias;
  p.K = ea.K;
  p.N = ea.N;
  p.E = ea.E;
  p.g = ea.g;
  p.out = ea.out;
  p.perm = db.perm;
  p.active = db.active;
  p.meta = db.meta;
  p.nt = ea.mode == MODE_UP ? ea.N / 64 : ea.N / BN;
  // Upper bound of M-tiles over all experts: each active expert adds at most
  // one partial tile.
  const int a_tiles = (ea.A + BM - 1) / BM + (ea.E < ea.A ? ea.E : ea.A);
  // A multiple of 8 blocks, so the XCD-contiguous renumbering in the kernel
  // is a bijection; the extra blocks find no tile and exit.
  const long blocks = ((long)a_tiles * p.nt + 7) / 8 * 8;
  if (blocks > 0x7fffffffL) return moe_fail(MOE_INVALID_ARGUMENT, "expert gemm: grid too large");
  dim3 grid((unsigned)blocks), block(256);
  if (ea.mode == MODE_UP) {
    if (ea.a_dtype == MOE_F16)
      hipLaunchKernelGGL((k_expert_gemm<MODE_UP, _Float16>), grid, block, 0, s, p);
    else
      hipLaunchKernelGGL((k_expert_gemm<MODE_UP, float>), grid, block, 0, s, p);
  } else {
    if (ea.a_dtype == MOE_F16)
      hipLaunchKernelGGL((k_expert_gemm<MODE_DOWN, _Float16>), grid, block, 0, s, p);
    else
      hipLaunchKernelGGL((k_expert_gemm<MODE_DOWN, float>), grid, block, 0, s, p);
  }
  return 0;
}
