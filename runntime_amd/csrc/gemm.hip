// Grouped expert GEMM for prefill shapes (many rows per expert) on gfx950.
//
// Reference: src/core/kernels/matmul/moeQuantW.ts:122-175 (moeUp) and
// :188-237 (moeDown); quantW layout src/core/kernels/quantCommon.ts:8-31.
// Same results as the expert kernels of expert.hip; this one is shaped for
// rows per expert in the hundreds.
//
// Work: for every active expert e (rows grouped by the dispatch), C_e =
// A_e · W_e with A_e the expert's gathered input rows (x for up, act for
// down) and W_e its int8 weights. Up computes glu and lin for the same 128
// outputs in one tile (128 glu + 128 lin columns) and applies the SwiGLU in
// the epilogue; down adds the bias.
//
// Tiles: 128 rows × 256 weight columns per block, 4 wavefronts side by side,
// each owning all 128 rows × 64 columns (4 × 2 v_mfma_f32_32x32x16_f16
// tiles, 128 accumulators, two wavefronts per SIMD): a weight fragment is
// read and converted by exactly one wavefront. Reading the LDS fragments is
// what bounds this kernel (measured: without those reads the same kernel
// runs 30% faster; without the int8 conversion, 1%). Per K step the block's
// global loads for the next step are issued first, the MFMAs run from one
// LDS buffer, then the loaded data goes to the other buffer: one barrier
// per step.
//  - Weights stay int8 in LDS ([column][k] bytes, row pitch BK + 8: the
//    8-byte fragment reads of 32 columns hit 64 distinct banks), stored
//    with the sign bit flipped (q + 128 as a byte), and become f16 after the
//    read (exact: |q| ≤ 127).
//  - A is f16 in LDS ([row][k], pitch BK + 8 halves); f32 input is split
//    into f16 hi + lo planes (two MFMAs per tile; ~2^-22 relative), with
//    BK 32 instead of 64 so that a step holds the same MFMA work and two
//    blocks still fit a CU's LDS.
// Scales (one per column: the GEMM path runs with groupSize = K) and biases
// apply in the epilogue.
//
// Order of tiles: expert, then N-tile, then M-tile, so the M-tiles of one
// (expert, N-tile) — which share its weights — run back to back; blocks are
// then dealt to the 8 XCDs in contiguous ranges (block b runs on XCD b mod 8),
// so those neighbours share one L2.
#include "moe_internal.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
// Native vectors for the staging registers: HIP's uint4 struct is copied
// through private memory when moved whole.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// 16 bytes at an 8-byte aligned LDS address (weight rows have pitch BK + 8).
typedef uint32_t u32x4_a8 __attribute__((ext_vector_type(4), aligned(8)));

constexpr int WAVE = 64;
constexpr int BM = GEMM_TILE_M;  // 128 rows
constexpr int BNW = 256;         // weight columns per block (up: 128 glu + 128 lin)

struct GemmArgs {
  const void *a;
  int a_row_div;
  const uint32_t *w0;  // glu (up) or down
  const float *s0;
  const float *b0;
  const uint32_t *w1;  // lin (up)
  const float *s1;
  const float *b1;
  int K, N, E;         // N: output columns (up: I, per projection)
  float *out;
  const int32_t *perm;
  const int32_t *active;  // [E][4] {e, first row, rows, first M-tile}
  const int32_t *meta;
  int nt;                 // N-tiles
};

__device__ __forceinline__ float swiglu(float glu, float lin) {
  // activations.ts:127-133: g = min(glu, 7), l = clamp(lin, ±7),
  // g / (1 + exp(−1.702·g)) · (l + 1). exp via the hardware 2^x and the
  // quotient via the hardware reciprocal (each within 1 ulp): the precise
  // library forms cost more VALU than the GEMM epilogue can hide.
  const float g = fminf(glu, 7.0f);
  const float l = fminf(fmaxf(lin, -7.0f), 7.0f);
  const float e = __builtin_amdgcn_exp2f(g * (-1.702f * 1.4426950408889634f));
  return g * __builtin_amdgcn_rcpf(1.0f + e) * (l + 1.0f);
}

// 8 offset bytes u = q + 128 (k order, little-endian in two words) → 8 f16
// q. Placing u under the exponent byte 0x64 gives the f16 1024 + u; minus
// 1152 leaves q exactly.
__device__ __forceinline__ uint32_t u8x2_to_h2(uint32_t x, uint32_t sel) {
  const half2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  return __builtin_bit_cast(
      uint32_t, __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, x, sel)) - bias);
}
__device__ __forceinline__ half8 cvt_u8x8(uint32_t x0, uint32_t x1) {
  const u32x4 r = {u8x2_to_h2(x0, 0x04010400u), u8x2_to_h2(x0, 0x04030402u),
                   u8x2_to_h2(x1, 0x04010400u), u8x2_to_h2(x1, 0x04030402u)};
  return __builtin_bit_cast(half8, r);
}

template <int MODE, typename AT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void k_expert_gemm(GemmArgs p) {
  constexpr bool SPLIT = sizeof(AT) == 4;
  constexpr int PLANES = SPLIT ? 2 : 1;
  constexpr int BK = SPLIT ? 32 : 64;
  constexpr int LDA = BK + 8;   // halves
  constexpr int LDW = BK + 8;   // bytes
  constexpr int KT = BK / 16;   // quantW tiles (4 k each) per thread per step
  __shared__ __align__(16) _Float16 As[2][PLANES][BM * LDA];
  __shared__ __align__(16) uint8_t Ws[2][BNW * LDW];
  __shared__ int32_t rowmap[BM];  // assignment of each tile row (for the epilogue)

  // ---- which tile: XCD-contiguous block order (gridDim.x is a multiple of
  // 8), then expert / N / M.
  const int nblk = gridDim.x;
  const int b = blockIdx.x;
  const int per_xcd = nblk / 8;
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
  const int N4 = p.N / 4, K4 = p.K / 4;
  const int ksteps = p.K / BK;

  // ---- this thread's share of the staging
  // Weights: block unit bu (of 64, 4 columns each), tiles KT·q .. KT·q + KT − 1
  // of the step. Up: units 0..31 are glu, 32..63 lin, of the same outputs.
  const int bu = tid >> 2, q = tid & 3;
  int u;
  const uint32_t *wbase;
  if (MODE == MODE_UP) {
    u = ntile * 32 + (bu & 31);
    wbase = bu < 32 ? p.w0 : p.w1;
  } else {
    u = ntile * 64 + bu;
    wbase = p.w0;
  }
  // Columns past N read unit 0 and rows past the tile's read its last row:
  // MFMA rows and columns are independent, and the epilogue writes neither.
  const u32x4 *wsrc = (const u32x4 *)(wbase + ((int64_t)e * N4 + (u < N4 ? u : 0)) * K4 * 4) + KT * q;
  // A: row ar of the tile, BK/2 consecutive k from ak (64 bytes either way).
  const int ar = tid >> 1, ak = (tid & 1) * (BK / 2);
  const int32_t asg_ar = p.perm[row0 + m0 + min(ar, rows - 1)];
  if ((tid & 1) == 0) rowmap[ar] = asg_ar;  // read after the loop's barriers
  const int64_t asrc_row = asg_ar / p.a_row_div;
  const u32x4 *asrc = (const u32x4 *)((const AT *)p.a + asrc_row * p.K + ak);

  // Staging registers of one K step.
  u32x4 wreg[KT], areg[4];
  auto load = [&](int ks) {
#pragma unroll
    for (int i = 0; i < KT; i++) wreg[i] = wsrc[ks * (BK / 4) + i];
#pragma unroll
    for (int i = 0; i < 4; i++) areg[i] = asrc[ks * (BK * (int)sizeof(AT) / 16) + i];
  };
  auto store = [&](int buf) {
    // Tile i, word c = column c, rows 4(KT·q + i) .. +3 (one byte each).
    constexpr uint32_t FLIP = 0x80808080u;
    auto put = [&](int c, uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
      uint8_t *dst = &Ws[buf][(bu * 4 + c) * LDW + q * KT * 4];
      if constexpr (KT == 4)
        *(u32x4_a8 *)dst = u32x4_a8{w0, w1, w2, w3} ^ FLIP;
      else
        *(u32x2 *)dst = u32x2{w0, w1} ^ FLIP;
    };
    const u32x4 t0 = wreg[0], t1 = wreg[1], t2 = wreg[KT == 4 ? 2 : 0], t3 = wreg[KT == 4 ? 3 : 1];
    put(0, t0.x, t1.x, t2.x, t3.x);
    put(1, t0.y, t1.y, t2.y, t3.y);
    put(2, t0.z, t1.z, t2.z, t3.z);
    put(3, t0.w, t1.w, t2.w, t3.w);
    if constexpr (SPLIT) {
      const float *v = (const float *)areg;  // 16 k
#pragma unroll
      for (int j = 0; j < 2; j++) {
        half8 h, l;
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const float x = v[8 * j + i];
          const _Float16 xh = (_Float16)x;
          h[i] = xh;
          l[i] = (_Float16)(x - (float)xh);
        }
        *(half8 *)&As[buf][0][ar * LDA + ak + 8 * j] = h;
        *(half8 *)&As[buf][PLANES - 1][ar * LDA + ak + 8 * j] = l;
      }
    } else {
      u32x4 *dst = (u32x4 *)&As[buf][0][ar * LDA + ak];
      dst[0] = areg[0];
      dst[1] = areg[1];
      dst[2] = areg[2];
      dst[3] = areg[3];
    }
  };

  floatx16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  // MFMA operands: lane L reads row (or column) L%32, k 8·(L/32) .. +7 of a
  // 16-wide K slice.
  const int fr = lane & 31, fk = (lane >> 5) * 8;
  // Weight columns of this wavefront's tiles: up → glu 32·wave (j = 0) and
  // the matching lin columns at +128 (j = 1); down → 64·wave + 32j.
  const int wcol[2] = {MODE == MODE_UP ? 32 * wave : 64 * wave,
                       MODE == MODE_UP ? 128 + 32 * wave : 64 * wave + 32};

  auto compute = [&](int cur) {
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      half8 bf[2];
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const u32x2 raw = *(const u32x2 *)&Ws[cur][(wcol[j] + fr) * LDW + kk + fk];
        bf[j] = cvt_u8x8(raw.x, raw.y);
      }
#pragma unroll
      for (int pl = 0; pl < PLANES; pl++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const half8 af = *(const half8 *)&As[cur][pl][(i * 32 + fr) * LDA + kk + fk];
#pragma unroll
          for (int j = 0; j < 2; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf[j], acc[i][j], 0, 0, 0);
        }
      }
    }
  };

  // Step s computes LDS buffer s & 1 while step s + 1 loads into registers;
  // then step s + 1 goes to the other buffer. The last step re-reads itself (unconditional: a branch would keep the
  // staging registers in memory).
  load(0);
  store(0);
  __syncthreads();
  for (int ks = 0; ks < ksteps; ks++) {
    const int cur = ks & 1;
    load(min(ks + 1, ksteps - 1));
    compute(cur);
    // Keep the staging work (which waits for the loads above) after the
    // MFMAs: hoisted into them it would stall each step on the loads.
    __builtin_amdgcn_sched_barrier(0);
    store(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue. acc[i][j][r]: row 32i + 8(r/4) + 4(L/32) + r%4, column
  // L%32 of tile j.
  if (MODE == MODE_UP) {
    const int col = ntile * 128 + 32 * wave + fr;  // glu index = lin index
    if (col < p.N) {
      const float sg = p.s0[(int64_t)e * p.N + col], sl = p.s1[(int64_t)e * p.N + col];
      const float bg = p.b0 ? p.b0[(int64_t)e * p.N + col] : 0.f;
      const float bl = p.b1 ? p.b1[(int64_t)e * p.N + col] : 0.f;
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int row = i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
          if (row < rows) {
            const int64_t asg = rowmap[row];
            p.out[asg * p.N + col] = swiglu(acc[i][0][r] * sg + bg, acc[i][1][r] * sl + bl);
          }
        }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int col = ntile * BNW + wcol[j] + fr;
      if (col >= p.N) continue;
      const float sc = p.s0[(int64_t)e * p.N + col];
      const float bb = p.b0 ? p.b0[(int64_t)e * p.N + col] : 0.f;
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int row = i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
          if (row < rows) {
            const int64_t asg = rowmap[row];
            p.out[asg * p.N + col] = acc[i][j][r] * sc + bb;
          }
        }
    }
  }
}

}  // namespace

bool gemm_eligible(const ExpertArgs &ea) {
  // One scale group per column, K in whole steps.
  const int bk = ea.a_dtype == MOE_F16 ? 64 : 32;
  return ea.bits == 8 && ea.g == ea.K && ea.K % bk == 0 && ea.N % 4 == 0;
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
  p.out = ea.out;
  p.perm = db.perm;
  p.active = db.active;
  p.meta = db.meta;
  const int cols = ea.mode == MODE_UP ? BNW / 2 : BNW;  // output columns per tile
  p.nt = (ea.N + cols - 1) / cols;
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
