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
// outputs in one tile and applies the SwiGLU in the epilogue; down adds the
// bias.
//
// Tiles: 128 rows × 128 weight units (512 columns) per block, eight
// wavefronts, two per SIMD, 128 accumulators each. The block's units come
// from two sources of 64 units each: up takes the same 64 units (256
// outputs) of glu and of lin, down takes 128 consecutive units of its one
// weight (512 outputs). Two wavefront shapes:
//  - f16 A (up with f16 x when gemm_wide.hip does not take the shape): each
//    wavefront takes all 128 rows and 16 slots
//    (8 glu units and the same 8 lin units) with two of each unit's four
//    columns per lane: 4 × 2 v_mfma_f32_32x32x16_f16 tiles, so one
//    converted weight fragment feeds four MFMAs. The SwiGLU pairs lanes 16
//    apart.
//  - f32 or f16-pair A (down, up with f32 x): 2 (row halves) × 4 (unit
//    groups), 64 rows × 32 units with all four columns each: 2 × 4 tiles.
// A tile's operands (16 KB of int8 weights and 8 or 16 KB of A per 32 k)
// come through L2.
//
// Weights go to LDS as the quantW words are: 16-byte tiles of 4 columns × 4
// k, [column][k] bytes, so dword c of a tile is column c's four k values.
// A lane of the MFMA B operand owns one unit (L % 32) and, per 16-k slice,
// two tiles (32 bytes): that is columns c = 0..3 of its unit with 8 k each,
// the B operands of four MFMAs whose 32 columns are "column c of units
// 0..31". The k order inside a 32-k step is a fixed permutation (lane half
// h, slice kk holds k = 16h + 8kk .. +7) that A follows too, so the sum is
// unchanged. int8 → f16 is exact (|q| ≤ 127).
//
// Loads go straight from global memory to LDS (buffer_load … lds): a ring of
// STAGES 32-k steps; no staging registers and no LDS stores. A workgroup
// barrier comes every step, or every second step when a tile's step count
// is even (PAIR): at the barrier every wavefront has read the slots of the
// steps it just used, so their loads for STAGES steps ahead may go out. A
// wavefront issues those loads spread between its MFMA groups rather than
// all at once after the barrier: when every wavefront issues its DMA burst
// at the same moment their issue stalls together and the matrix cores idle
// (measured: the memory-only and compute-only variants of the loop took
// 0.53 ms each at config 4's up shape, together 0.94 ms with the burst).
// The waits are explicit vmcnt counts: the compiler does not track loads
// that write LDS.
//
// LDS positions are chosen so that the fragment reads hit distinct banks
// (SQ_LDS_BANK_CONFLICT reads 0). Rows of 128 bytes (a weight slot's 8
// tiles, an f32 A row) are XOR-swizzled: chunk c of row r at
// r·128 + ((c ^ sw8(r))·16), sw8(r) = (r ^ (r >> 3)) & 7. f16 A rows (64
// bytes) go chunk-major per 16 rows: chunk c of row r at
// (r / 16)·1024 + c·256 + (r % 16)·16, so the 16 lanes reading one chunk of
// 16 rows read 256 contiguous bytes (a row-major layout of 64-byte rows
// costs two passes per read whatever the swizzle).
// f32 A is split into f16 hi + lo after the read (two MFMAs per product;
// ~2^-22 relative).
//
// Order of tiles: expert, then N-tile, then M-tile, so the M-tiles of one
// (expert, N-tile) — which share its weights — run back to back; blocks are
// dealt to the 8 XCDs in contiguous ranges (block b runs on XCD b mod 8),
// so those neighbours share one L2.
#include "gemm_dev.h"

#include <type_traits>

namespace {

// OPAIR (up): write act as f16 pairs. AT = f16pair (down): read them.
template <int MODE, typename AT, bool OPAIR, bool PAIR>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))
void k_expert_gemm(GemmArgs p) {
  constexpr bool SPLIT = sizeof(AT) == 4;
  constexpr bool PAIRS = std::is_same_v<AT, f16pair>;
  // f16 A: each wavefront covers all 128 rows and two of each unit's four
  // columns (4 × 2 MFMA tiles), so one converted weight fragment feeds four
  // MFMAs. f32 A (split into hi + lo, whose conversion scales with the row
  // tiles) keeps 64 rows × four columns (2 × 4 tiles).
  constexpr bool TALL = !SPLIT;
  constexpr int RT = TALL ? 4 : 2;  // 32-row MFMA tiles per wavefront
  constexpr int CT = TALL ? 2 : 4;  // columns of each unit per wavefront
  constexpr int A_BYTES = BM * BK * (int)sizeof(AT);  // 8 or 16 KB
  constexpr int STAGE = W_BYTES + A_BYTES;
  constexpr int STAGES = SPLIT ? 4 : 6;               // 128 or 144 KB
  constexpr int LOADS = SPLIT ? 4 : 3;                // ring loads per lane per step
  constexpr int TILE_LOADS = 2;                       // row map + constants, per lane per tile
  // epilogue stores per lane
  constexpr int STORES = MODE == MODE_UP ? 8 * RT : 16 * RT;
  constexpr int BASE_WAIT = (STAGES - 2) * LOADS;
  // vmcnt counts to 63; a smaller count only waits longer (for some stores).
  constexpr int STORE_WAIT = BASE_WAIT + STORES < 63 ? BASE_WAIT + STORES : 63;
  __shared__ __align__(16) uint8_t lds[STAGES * STAGE];
  __shared__ __align__(16) int32_t rowmap[2][BM];     // assignment of each tile row
  // Per-tile epilogue constants: up → glu scales, lin scales, glu biases,
  // lin biases (256 each); down → scales, biases (512 each).
  __shared__ __align__(16) float consts[2][1024];
  __shared__ int4 descs[GEMM_MAX_E];                  // active-expert descriptors

  // ---- this block's tiles. The tile list (expert, then N-tile, then
  // M-tile) is cut into 8 contiguous ranges, one per XCD (block b runs on
  // XCD b mod 8); the XCD's blocks take its tiles round robin, so the tiles
  // in flight on one XCD at a time are neighbours that share weights.
  const int total = p.meta[META_TILES] * p.nt * p.parts;
  const int n_active = p.meta[META_ACTIVE];
  const int bx = gridDim.x >> 3;  // blocks per XCD
  const int xcd = blockIdx.x & 7, xb = blockIdx.x >> 3;
  const int per_x = (total + 7) >> 3;
  const int start = xcd * per_x + xb, end = min(total, (xcd + 1) * per_x);
  if (start >= end) return;
  const int ntiles = (end - start + bx - 1) / bx;

  const int tid = threadIdx.x;
  const int lane = tid & (WAVE - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);  // uniform
  // Slots (weight units of the tile; up: 0-63 glu, 64-127 the same lin
  // units). Two wavefront shapes:
  //  - TALL: wavefront w takes all 128 rows and 16 slots, up: glu units
  //    8w .. 8w + 7 and the same lin units, down: slots 16w .. 16w + 15.
  //    Lane lm = 2σ + b holds slot σ (up: glu for σ < 8, lin for σ ≥ 8),
  //    columns 2b and 2b + 1. Neighbouring lanes read the two 8-byte
  //    halves of one 16-byte tile, and the 8 slots of 16 lanes sit in
  //    distinct bank groups, so each 16 lanes read 128 bytes without a
  //    bank conflict.
  //  - otherwise 2 (row halves) × 4 (unit groups), 64 rows and 32 slots
  //    each, up: glu units 16·wn .. + 15 and the same lin units; lane lm
  //    holds slot lm (up: glu for lm < 16), all four columns.
  // Wavefront w runs on SIMD w % 4. A tile with at most 32 units per source
  // (the last N-tile of I = 1408) idles the upper unit groups; each SIMD
  // still keeps one busy wavefront: TALL wavefronts w and w + 4 hold unit
  // groups w and w + 4; otherwise SIMD s holds unit groups s and s ^ 2 (the
  // second row half mirrored), which also balances a tile of at most 64 rows.
  const int wm = TALL ? 0 : wave >> 2;
  const int wn = (wave >> 2) ? (wave & 3) ^ 2 : wave & 3;
  const int lm = lane & 31, h = lane >> 5;
  constexpr int UPW = TALL ? 8 : 16;  // up: units per source per wavefront
  // The lane's unit within its group (up: within each source) and the first
  // of its columns.
  const int usub = TALL ? (MODE == MODE_UP ? (lm >> 1) & 7 : lm >> 1) : (MODE == MODE_UP ? lm & 15 : lm);
  const int cb = TALL ? 2 * (lm & 1) : 0;
  const int N4 = p.N / 4;
  const int ksteps = p.kpart;  // steps per tile

  for (int i = tid; i < n_active; i += blockDim.x) descs[i] = ((const int4 *)p.active)[i];
  __syncthreads();

  // Tile L: expert (by its M-tile range), then N-tile, then K part, then
  // M-tile.
  const int ntp = p.nt * p.parts;
  auto tile_at = [&](int L) {
    const int t = L / ntp;  // global M-tile index within the tile's expert range
    int lo = 0, hi = n_active - 1;
    while (lo < hi) {  // last active expert whose first M-tile ≤ t
      const int mid = (lo + hi + 1) >> 1;
      if (descs[mid].w <= t) lo = mid; else hi = mid - 1;
    }
    const int4 d = descs[lo];
    const int mt = (d.z + BM - 1) / BM;
    const int local = L - d.w * ntp;
    const int ntile = local / (mt * p.parts), rem = local % (mt * p.parts);
    const int part = rem / mt, mtile = rem % mt;
    Tile T;
    T.e = __builtin_amdgcn_readfirstlane(d.x);
    T.r0 = __builtin_amdgcn_readfirstlane(d.y + mtile * BM);
    T.rows = __builtin_amdgcn_readfirstlane(min(BM, d.z - mtile * BM));
    T.U0 = __builtin_amdgcn_readfirstlane(MODE == MODE_UP ? ntile * 64 : ntile * 128);
    T.U1 = __builtin_amdgcn_readfirstlane(MODE == MODE_UP ? ntile * 64 : ntile * 128 + 64);
    T.part = __builtin_amdgcn_readfirstlane(part);
    T.kb = __builtin_amdgcn_readfirstlane(part * p.kpart);
    return T;
  };

  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)lds;
  const uint32_t rowmap0 =
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int32_t *)&rowmap[0][0];
  const uint32_t consts0 =
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float *)&consts[0][0];
  const uint32_t slab = (uint32_t)p.K * (uint32_t)p.N;  // weight bytes of one expert
  const i32x4 ar = buffer_rsrc(p.a, (uint32_t)p.a_bytes);
  const i32x4 pr = buffer_rsrc(p.perm, (uint32_t)p.perm_bytes);
  // Constants this wavefront loads per tile: up → array wave/2 (glu scales,
  // lin scales, glu biases, lin biases), half wave & 1; down → array wave/4
  // (scales, biases), quarter wave & 3. A missing bias reads zeros (an empty
  // buffer).
  const float *cbase = MODE == MODE_UP
                           ? (wave < 2 ? p.s0 : wave < 4 ? p.s1 : wave < 6 ? p.b0 : p.b1)
                           : (wave < 4 ? p.s0 : p.b0);
  const i32x4 cr = buffer_rsrc(cbase, cbase ? (uint32_t)p.E * (uint32_t)p.N * 4u : 0u);

  // ---- per-tile loads into LDS buffer `sel`: the row map (perm entries of
  // rows 16·wave + l, l < 16; rows past the tile repeat its last) and the
  // epilogue constants (512 bytes per wavefront, lanes 0-31). One load
  // instruction each per wavefront.
  auto issue_tile = [&](const Tile &T, int sel) {
    if (lane < 16) {
      const int r = 16 * wave + lane;
      dma4(pr, (uint32_t)(T.r0 + min(r, T.rows - 1)) * 4u, 0, rowmap0 + sel * (BM * 4) + 64 * wave);
    }
    if (lane < 32) {
      const int col = 4 * T.U0 + (MODE == MODE_UP ? (wave & 1) : (wave & 3)) * 128 + 4 * lane;
      dma16(cr, ((uint32_t)T.e * (uint32_t)p.N + (uint32_t)col) * 4u, 0,
            consts0 + sel * 4096 + 512 * wave);
    }
  };

  // ---- ring loads of a step. Each load instruction fills 1 KB of LDS
  // (lane l at +16·l), so lane l picks the global chunk that belongs at that
  // position.
  // Weights: instructions i = 0, 1 fill slots 16·wave + 8i .. +7 (wavefronts
  // 0-3: source 0, 4-7: source 1); lane l: slot + (l >> 3), position l & 7
  // holds tile (l & 7) ^ sw8(slot). A unit past N gets an offset past the
  // expert's slab, which the buffer's range check turns into zeros.
  // A: f16 → one instruction, lane l: row 16·wave + (l & 15), 8-half chunk
  //    l >> 4 (chunk-major); f32 → instructions i = 0, 1, rows
  //    16·wave + 8i + (l >> 3), position l & 7 holds 4-float chunk
  //    (l & 7) ^ sw8(row). Rows past the tile's read its last row: MFMA rows
  //    are independent and the epilogue writes none of them.
  constexpr int AI = SPLIT ? 2 : 1;
  struct Params {
    i32x4 wr;
    uint32_t woff[2], aoff[AI];
  };
  auto make_params = [&](const Tile &T, int sel) {
    Params P;
    P.wr = buffer_rsrc((wave < 4 ? p.w0 : p.w1) + (int64_t)T.e * (slab / 4), slab);
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int slot = 16 * wave + 8 * i + (lane >> 3);
      const int u = (wave < 4 ? T.U0 : T.U1) + (slot & 63);
      const int tile = (lane & 7) ^ sw8w<TALL>(slot);
      P.woff[i] = u < N4 ? (uint32_t)u * (uint32_t)p.K * 4u + tile * 16u : 0x80000000u;
    }
#pragma unroll
    for (int i = 0; i < AI; i++) {
      if (SPLIT) {
        const int r = 16 * wave + 8 * i + (lane >> 3);
        const uint32_t srow = MODE == MODE_DOWN && p.sorted ? (uint32_t)(T.r0 + min(r, T.rows - 1))
                                       : (uint32_t)(rowmap[sel][r] / p.a_row_div);
        P.aoff[i] = srow * (uint32_t)p.K * 4u + ((lane & 7) ^ sw8(r)) * 16u;
      } else {
        const int r = 16 * wave + (lane & 15);
        const uint32_t srow = MODE == MODE_DOWN && p.sorted ? (uint32_t)(T.r0 + min(r, T.rows - 1))
                                       : (uint32_t)(rowmap[sel][r] / p.a_row_div);
        P.aoff[i] = srow * (uint32_t)p.K * 2u + (lane >> 4) * 16u;
      }
    }
    return P;
  };
  // Load instruction q of step ks into slot `stage`: q < 2 weights, else A.
  auto issue_q = [&](const Params &P, int ks, int stage, int q) {
    const uint32_t st = lds0 + stage * STAGE;
    if (q < 2) dma16(P.wr, P.woff[q], ks * (TPS * 16), st + (2 * wave + q) * 1024);
    else dma16(ar, P.aoff[q - 2], ks * BK * (int)sizeof(AT), st + W_BYTES + (AI * wave + q - 2) * 1024);
  };
  auto issue = [&](const Params &P, int ks, int stage) {
#pragma unroll
    for (int q = 0; q < LOADS; q++) issue_q(P, ks, stage, q);
  };

  floatx16 acc[RT][CT];

  // Fragment positions. B: this lane's slot, tiles 4h + 2kk (+1), of each
  // dwords cb .. (TALL: two, else four). A: rows 64·wm + 32i + lm, k
  // 16h + 8kk .. +7.
  const int ug = TALL ? wave : wn;  // unit group
  const int slot = MODE == MODE_UP ? (lm < 16 ? 0 : 64) + UPW * ug + usub
                                   : (TALL ? 16 * wave : 32 * wn) + usub;
  const int boff = slot * 128, bsw = sw8w<TALL>(slot);
  int aoff[RT], asw[RT];
#pragma unroll
  for (int i = 0; i < RT; i++) {
    const int arow = 64 * wm + 32 * i + lm;
    aoff[i] = W_BYTES + (SPLIT ? arow * BK * 4 : (arow >> 4) * 1024 + (arow & 15) * 16);
    asw[i] = SPLIT ? sw8(arow) : 0;
  }

  // One step's fragments as read from LDS: raw weight tiles and A, per
  // 16-k slice kk.
  using WV = std::conditional_t<TALL, u32x2, u32x4>;  // this lane's CT dwords of a tile
  struct Frags {
    WV w[2][2];                     // [kk][tile]
    u32x4 a[2][RT][SPLIT ? 2 : 1];  // [kk][i][16-byte chunk]
  };
  const int wdw = 4 * cb;  // byte of the first dword within a tile
  auto read_frags = [&](Frags &F, int stage, int kk) {
    const uint8_t *st = lds + stage * STAGE;
    const int t0 = 4 * h + 2 * kk;
    F.w[kk][0] = *(const WV *)(st + boff + ((t0 ^ bsw) * 16) + wdw);
    F.w[kk][1] = *(const WV *)(st + boff + (((t0 + 1) ^ bsw) * 16) + wdw);
#pragma unroll
    for (int i = 0; i < RT; i++) {
      if constexpr (SPLIT) {
        F.a[kk][i][0] = *(const u32x4 *)(st + aoff[i] + ((t0 ^ asw[i]) * 16));
        F.a[kk][i][1] = *(const u32x4 *)(st + aoff[i] + (((t0 + 1) ^ asw[i]) * 16));
      } else {
        F.a[kk][i][0] = *(const u32x4 *)(st + aoff[i] + (2 * h + kk) * 256);
      }
    }
  };
  // The MFMAs of one slice (when `live`), column c outer: the conversion of
  // column c + 1 is placed before the MFMAs of column c, so it overlaps
  // them. After column c's MFMAs, hook(c) issues the ring loads scheduled
  // there: the loads of a step are spread over the MFMA groups instead of
  // leaving every wavefront at once after the barrier (a burst of DMA
  // instructions from all wavefronts stalls their issue together, and the
  // matrix cores with it).
  // RTL: the wavefront's live 32-row tiles (compile time); live: a runtime
  // switch for the whole slice (the split shapes keep one loop copy).
  auto mfma_slice = [&](const Frags &F, int kk, auto rtl, bool live, auto &&hook) {
    constexpr int RTL = decltype(rtl)::value;
    constexpr int PL = SPLIT ? 2 : 1;
    half8 af[RT][PL];
    half8 bf[CT];
    if (RTL > 0 && live) {
#pragma unroll
      for (int i = 0; i < RT; i++) {
        if constexpr (PAIRS) {
          const u32x4 c0 = F.a[kk][i][0], c1 = F.a[kk][i][1];
          af[i][0] = __builtin_bit_cast(half8, u32x4{c0[0], c0[2], c1[0], c1[2]});
          af[i][1] = __builtin_bit_cast(half8, u32x4{c0[1], c0[3], c1[1], c1[3]});
        } else if constexpr (SPLIT) {
          const floatx4 v0 = __builtin_bit_cast(floatx4, F.a[kk][i][0]);
          const floatx4 v1 = __builtin_bit_cast(floatx4, F.a[kk][i][1]);
#pragma unroll
          for (int j = 0; j < 8; j++) {
            const float x = j < 4 ? v0[j] : v1[j - 4];
            const _Float16 xh = (_Float16)x;
            af[i][0][j] = xh;
            af[i][PL - 1][j] = (_Float16)(x - (float)xh);
          }
        } else {
          af[i][0] = __builtin_bit_cast(half8, F.a[kk][i][0]);
        }
      }
      bf[0] = cvt_i8x8(F.w[kk][0][0], F.w[kk][1][0]);
    }
#pragma unroll
    for (int c = 0; c < CT; c++) {
      if (RTL > 0 && live) {
        if (c + 1 < CT) bf[c + 1] = cvt_i8x8(F.w[kk][0][c + 1], F.w[kk][1][c + 1]);
#pragma unroll
        for (int pl = 0; pl < PL; pl++)
#pragma unroll
          for (int i = 0; i < RTL; i++)
            acc[i][c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i][pl], bf[c], acc[i][c], 0, 0, 0);
      }
      hook(c);
    }
  };
  auto no_loads = [](int) {};

  // ---- epilogue of tile T from LDS buffer `sel`. acc[i][c][r]: row
  // 64wm + 32i + 8(r/4) + 4h + r%4, column cb + c of this lane's unit. Outputs go
  // through a buffer store whose offset is out of range for rows past the
  // tile (the store is dropped): no branches, so the stores queue back to
  // back. (Behind a per-row branch the compiler re-waits for every earlier
  // memory access, store included, at each branch.)
  const __amdgpu_buffer_rsrc_t orc =
      __builtin_amdgcn_make_buffer_rsrc(p.out, 0, p.out_bytes, BUF_DWORD3);
  // (m & x) | (~m & y) per bit: one v_bfi_b32, where a select of two
  // elements of one accumulator vector becomes a chain over all sixteen.
  auto pick = [](uint32_t m, float x, float y) {
    return __builtin_bit_cast(float, (m & __builtin_bit_cast(uint32_t, x)) |
                                         (~m & __builtin_bit_cast(uint32_t, y)));
  };
  // This lane's CT consecutive output columns of one row (offset past the
  // buffer: dropped).
  auto store_cols = [&](const float (&v)[CT], uint32_t off) {
    if constexpr (CT == 4)
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{__builtin_bit_cast(uint32_t, v[0]),
                                                   __builtin_bit_cast(uint32_t, v[1]),
                                                   __builtin_bit_cast(uint32_t, v[2]),
                                                   __builtin_bit_cast(uint32_t, v[3])},
                                             orc, off, 0, 0);
    else
      __builtin_amdgcn_raw_buffer_store_b64(u32x2{__builtin_bit_cast(uint32_t, v[0]),
                                                  __builtin_bit_cast(uint32_t, v[1])},
                                            orc, off, 0, 0);
  };
  // The same as f16 pairs (at the f32 values' offset).
  auto store_pairs = [&](const float (&v)[CT], uint32_t off) {
    uint32_t hl[CT];
#pragma unroll
    for (int c = 0; c < CT; c += 2) {
      const _Float16 h0 = (_Float16)v[c], h1 = (_Float16)v[c + 1];
      hl[c] = __builtin_bit_cast(uint32_t, half2v{h0, h1});
      hl[c + 1] = __builtin_bit_cast(
          uint32_t, half2v{(_Float16)(v[c] - (float)h0), (_Float16)(v[c + 1] - (float)h1)});
    }
    if constexpr (CT == 4)
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{hl[0], hl[1], hl[2], hl[3]}, orc, off, 0, 0);
    else
      __builtin_amdgcn_raw_buffer_store_b64(u32x2{hl[0], hl[1]}, orc, off, 0, 0);
  };
  auto epilogue = [&](const Tile &T, int wu, int sel) {
    // Up with sorted rows writes act at the dispatch position.
    const bool out_sorted = MODE == MODE_UP && p.sorted;
    auto row_off = [&](int row, int uo) -> uint32_t {
      const uint32_t orow = out_sorted ? (uint32_t)(T.r0 + row) : (uint32_t)rowmap[sel][row];
      return row < T.rows ? (orow * (uint32_t)p.N + 4u * uo) * 4u : 0x80000000u;
    };
    const float *cs = consts[sel];
    if (MODE == MODE_UP) {
      // Lane lm < 16 holds glu and lane lm + 16 lin of unit wu + usub: the
      // low lane finishes rows r < 8 and the high lane rows r ≥ 8, each
      // receiving the other projection's values for its rows from its
      // partner.
      const bool low = lm < 16;
      const uint32_t lowm = low ? ~0u : 0u;
      const int uo = wu + usub;
      const bool col_ok = uo < N4;
      const int q = 4 * (uo - T.U0);  // output index within the tile
      const floatx4 sg = *(const floatx4 *)&cs[q], sl = *(const floatx4 *)&cs[256 + q];
      const floatx4 bg = *(const floatx4 *)&cs[512 + q], bl = *(const floatx4 *)&cs[768 + q];
#pragma unroll
      for (int i = 0; i < RT; i++)
#pragma unroll
        for (int r = 0; r < 8; r++) {
          float v[CT];
#pragma unroll
          for (int c = 0; c < CT; c++) {
            const int cc = cb + c;
            const float a0 = acc[i][c][r], a8 = acc[i][c][r + 8];
            const float send = pick(lowm, a8, a0);
            // ds_swizzle, bit mode: lane ^ 16 within each 32 lanes.
            const float recv = __builtin_bit_cast(
                float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, send), 0x401F));
            const float g = pick(lowm, a0, recv);
            const float l = pick(lowm, recv, a8);
            v[c] = swiglu(g * sg[cc] + bg[cc], l * sl[cc] + bl[cc]);
          }
          const int rr = low ? r : r + 8;
          const int row = 64 * wm + 32 * i + 8 * (rr / 4) + 4 * h + (rr % 4);
          if constexpr (OPAIR)
            store_pairs(v, col_ok ? row_off(row, uo) + wdw : 0x80000000u);
          else
            store_cols(v, col_ok ? row_off(row, uo) + wdw : 0x80000000u);
        }
    } else {
      const int uo = wu + usub;
      const bool col_ok = uo < N4;
      const int q = 4 * (uo - T.U0);
      // The bias goes into part 0 only; every part carries its scale.
      const floatx4 sc = *(const floatx4 *)&cs[q];
      const floatx4 bb = *(const floatx4 *)&cs[512 + q] * (T.part == 0 ? 1.f : 0.f);
      const uint32_t pbase = (uint32_t)T.part * (uint32_t)p.part_floats * 4u;
#pragma unroll
      for (int i = 0; i < RT; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int row = 64 * wm + 32 * i + 8 * (r / 4) + 4 * h + (r % 4);
          float v[CT];
#pragma unroll
          for (int c = 0; c < CT; c++) v[c] = acc[i][c][r] * sc[cb + c] + bb[cb + c];
          store_cols(v, col_ok ? row_off(row, uo) + wdw + pbase : 0x80000000u);
        }
    }
  };

  // ---- the pipeline. Ring loads run STAGES steps ahead of the MFMAs,
  // across tile boundaries: the first steps of tile j + 1 load while tile j
  // finishes and stores. Each step: the MFMAs of its first 16-k slice from
  // registers; then (mid-step) wait for this wavefront's ring loads of the
  // next step and for its own LDS reads, barrier (every wavefront's loads
  // landed, every read of this step's slot done), load the step STAGES
  // ahead into this step's slot, read the next step's first-slice
  // fragments, run the second slice's MFMAs, and read the next step's
  // second-slice fragments (their latency hides behind the next step's
  // first slice). MFMAs issued before the barrier keep the matrix pipe busy
  // while the wavefront waits there.
  // The vmcnt threshold counts what was issued after the awaited loads: the
  // ring loads of STAGES − 2 steps, plus the previous tile's epilogue stores
  // in the first steps of a tile, plus the next tile's row map and constants
  // while those are younger. The row map and constants of tile j + 1 load
  // STAGES − 1 steps before the step whose wait covers them, where the next
  // tile's load parameters are made (the step before its first ring load).
  // Every step issues the same number of ring loads (past the last tile
  // they re-read its last step), so the counts hold.
  Tile cur = tile_at(start), nxt = cur;
  issue_tile(cur, 0);
  WAIT_VMCNT(0);
  block_barrier();
  Params pc = make_params(cur, 0), pn = pc;
  if (ntiles > 1) nxt = tile_at(start + bx);
  // PAIR: one barrier per two steps. At the barrier in the middle of an
  // even step ks every wavefront has read all of steps ks − 1 and ks (their
  // fragments are in registers or consumed), so those two slots take steps
  // ks + STAGES − 1 and ks + STAGES; the wait covers steps ks + 1 and
  // ks + 2, whose fragments are read before the next barrier. The prologue
  // loads STAGES − 1 steps.
  constexpr int PRO = PAIR ? STAGES - 1 : STAGES;
#pragma unroll
  for (int s = 0; s < PRO; s++) issue(pc, cur.kb + s, s);
  WAIT_VMCNT((PRO - 1) * LOADS);  // step 0
  block_barrier();
  Frags f;
  read_frags(f, 0, 0);
  read_frags(f, 0, 1);
  // Row map and constants of the next tile: loaded at tile_step, covered by
  // the wait of the barrier before param_step, where its load parameters are
  // made (the step of its first ring load). Both are even with PAIR.
  const int tile_step = PAIR ? ksteps - 2 * STAGES + 2 : ksteps - 2 * STAGES;
  const int param_step = PAIR ? ksteps - STAGES : ksteps - STAGES - 1;
  // Ring loads issued after the awaited ones at a barrier.
  constexpr int P_BASE = PAIR ? (STAGES - 4) * LOADS : BASE_WAIT;
  constexpr int P_STORE = P_BASE + STORES < 63 ? P_BASE + STORES : 63;
  int stage = 0;  // slot of the step being computed
  for (int j = 0; j < ntiles; j++) {
    const bool has_next = j + 1 < ntiles;
    const int sel = j & 1;
    // First unit of the wavefront's group (up: of each source).
    const int wu = MODE == MODE_UP ? cur.U0 + UPW * ug
                   : TALL          ? (wave < 4 ? cur.U0 : cur.U1) + 16 * (wave & 3)
                                   : (wn < 2 ? cur.U0 : cur.U1) + 32 * (wn & 1);
    // Uniform: the wavefront's 32-row tiles with a row of the tile (0 when
    // it has no unit below N); the MFMAs of the others are skipped (the
    // last M-tile of an expert is partial).
    const int rt_live = wu >= N4 ? 0 : min(RT, max(0, (cur.rows - 64 * wm + 31) >> 5));
    const bool live = TALL || rt_live > 0;
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
      for (int c = 0; c < CT; c++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][c][r] = 0.f;
    // Ring loads of step a ≥ ksteps are the next tile's, or re-read the last
    // step past the last tile, so every barrier issues the same count.
    // The loads a barrier frees slots for: steps a0 (slot s0) and, with
    // PAIR, a1 (slot s1), each resolved at the barrier to a step of the
    // current tile (nx false) or of the next (nx true). Load j of the NL =
    // LOADS (or 2·LOADS) goes after MFMA group j·NG / NL of the NG = CT (or
    // 2·CT) groups that follow the barrier: slice 1 of this step and, with
    // PAIR, slice 0 of the next.
    int k0 = 0, s0 = 0, k1 = 0, s1 = 0;
    bool nx0 = false, nx1 = false;
    auto resolve = [&](int a, int &kstep, bool &nx) {
      nx = a >= ksteps && has_next;
      kstep = a < ksteps ? cur.kb + a : has_next ? nxt.kb + a - ksteps : cur.kb + ksteps - 1;
    };
    auto issue_sel = [&](bool nx, int kstep, int slot, int q) {
      Params P;
      P.wr = nx ? pn.wr : pc.wr;
#pragma unroll
      for (int i = 0; i < 2; i++) P.woff[i] = nx ? pn.woff[i] : pc.woff[i];
#pragma unroll
      for (int i = 0; i < AI; i++) P.aoff[i] = nx ? pn.aoff[i] : pc.aoff[i];
      issue_q(P, kstep, slot, q);
    };
    constexpr int NL = PAIR ? 2 * LOADS : LOADS;
    constexpr int NG = PAIR ? 2 * CT : CT;
    auto loads_at = [&](int g) {
#pragma unroll
      for (int jl = 0; jl < NL; jl++)
        if (jl * NG / NL == g) {
          if (jl < LOADS) issue_sel(nx0, k0, s0, jl);
          else issue_sel(nx1, k1, s1, jl - LOADS);
        }
    };
    // One step; BAR: the step has the barrier (every step without PAIR,
    // the even ones with it).
    auto step = [&](int ks, auto bar, auto rtl) {
      constexpr bool BAR = decltype(bar)::value;
      if (PAIR && !BAR) mfma_slice(f, 0, rtl, live, [&](int c) { loads_at(CT + c); });
      else mfma_slice(f, 0, rtl, live, no_loads);
      __builtin_amdgcn_sched_barrier(0);
      // ---- mid-step
      if constexpr (!PAIR) {
        if (j > 0 && ks <= STAGES - 2) WAIT_VMCNT(STORE_WAIT);
        else if (has_next && ks > tile_step && ks <= tile_step + STAGES - 2) WAIT_VMCNT(BASE_WAIT + TILE_LOADS);
        else WAIT_VMCNT(BASE_WAIT);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this step's LDS reads done
        block_barrier();
        if (has_next && ks == tile_step) issue_tile(nxt, sel ^ 1);
        if (has_next && ks == param_step) pn = make_params(nxt, sel ^ 1);
        resolve(ks + STAGES, k0, nx0);
        s0 = stage;
      } else if constexpr (BAR) {
        // Younger than the awaited loads (issued after the barrier of step
        // ks + 2 − STAGES): the previous tile's stores while that barrier
        // was in the previous tile, the next tile's row map and constants
        // when they were loaded at a barrier between.
        if (j > 0 && ks <= STAGES - 4) WAIT_VMCNT(P_STORE);
        else if (has_next && ks >= tile_step + 2 && ks <= tile_step + STAGES - 4) WAIT_VMCNT(P_BASE + TILE_LOADS);
        else WAIT_VMCNT(P_BASE);
        __builtin_amdgcn_s_waitcnt(0xC07F);
        block_barrier();
        if (has_next && ks == tile_step) issue_tile(nxt, sel ^ 1);
        if (has_next && ks == param_step) pn = make_params(nxt, sel ^ 1);
        resolve(ks + STAGES - 1, k0, nx0);
        s0 = stage == 0 ? STAGES - 1 : stage - 1;
        resolve(ks + STAGES, k1, nx1);
        s1 = stage;
      }
      stage = stage + 1 == STAGES ? 0 : stage + 1;
      read_frags(f, stage, 0);  // next step (the next tile's first after a tile's last)
      __builtin_amdgcn_sched_barrier(0);
      if (BAR) mfma_slice(f, 1, rtl, live, loads_at);
      else mfma_slice(f, 1, rtl, live, no_loads);
      __builtin_amdgcn_sched_barrier(0);
      read_frags(f, stage, 1);
    };
    auto kloop = [&](auto rtl) {
      if constexpr (PAIR) {
        for (int ks = 0; ks < ksteps; ks += 2) {
          step(ks, std::true_type(), rtl);
          step(ks + 1, std::false_type(), rtl);
        }
      } else {
        for (int ks = 0; ks < ksteps; ks++) step(ks, std::true_type(), rtl);
      }
    };
    // TALL wavefronts (all 128 rows) skip the dead row tiles of a partial
    // tile; the 64-row wavefronts of the split shapes only skip a tile half
    // with no row (more loop copies spill their registers).
    if constexpr (TALL) {
      if (rt_live >= 4) kloop(std::integral_constant<int, 4>());
      else if (rt_live == 3) kloop(std::integral_constant<int, 3>());
      else if (rt_live == 2) kloop(std::integral_constant<int, 2>());
      else if (rt_live == 1) kloop(std::integral_constant<int, 1>());
      else kloop(std::integral_constant<int, 0>());
    } else {
      kloop(std::integral_constant<int, RT>());
    }
    epilogue(cur, wu, sel);
    if (has_next) {
      cur = nxt;
      pc = pn;
      if (j + 2 < ntiles) nxt = tile_at(start + (j + 2) * bx);
    }
  }
  // The last steps' ring loads (re-reads) still write LDS: let them land
  // before the workgroup's LDS is released.
  WAIT_VMCNT(0);
}


}  // namespace

static int gemm_stages(const ExpertArgs &ea) { return ea.a_dtype == MOE_F16 ? 6 : 4; }

bool gemm_eligible(const ExpertArgs &ea) {
  // One scale group per column, K in whole steps, 32-bit buffer offsets
  // (one expert's weights, the input, the scales and the outputs stay below
  // 2 GiB), and enough steps per tile for the ring: the next tile's row map
  // loads 2·STAGES − 2 steps before the end of a tile, after the previous
  // epilogue's stores have left the wait window.
  const int64_t a_bytes = (int64_t)(ea.A / ea.a_row_div) * ea.K * (ea.a_dtype == MOE_F16 ? 2 : 4);
  const int64_t out_bytes = (int64_t)ea.A * ea.N * 4 * (ea.mode == MODE_DOWN ? 2 : 1);
  return ea.bits == 8 && ea.g == ea.K && ea.K % BK == 0 && ea.N % 4 == 0 &&
         ea.K / BK >= 3 * gemm_stages(ea) && ea.E <= GEMM_MAX_E && out_bytes < (1ll << 31) &&
         (int64_t)ea.K * ea.N < (1ll << 31) && a_bytes < (1ll << 31) &&
         (int64_t)ea.E * ea.N * 4 < (1ll << 31) && (int64_t)ea.A * 4 < (1ll << 31);
}

static int gemm_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!cus[dev] && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  return cus[dev];
}

// Upper bound of the M-tiles over all experts: each active expert adds at
// most one partial tile.
static long gemm_mtiles(const ExpertArgs &ea) {
  return (ea.A + BM - 1) / BM + (ea.E < ea.A ? ea.E : ea.A);
}

int gemm_down_parts(const ExpertArgs &ea) {
  if (ea.mode != MODE_DOWN || !gemm_eligible(ea)) return 1;
  const int ksteps = ea.K / BK;
  if (ksteps % 2 || ksteps / 2 < 3 * gemm_stages(ea)) return 1;
  const long cus = gemm_cus();
  if (cus <= 0) return 1;
  // Rounds of whole tiles over the CUs against rounds of half tiles (each
  // half as long), from the upper bound of the tile count.
  const long tiles = gemm_mtiles(ea) * ((ea.N + 511) / 512);
  const long whole = (tiles + cus - 1) / cus;
  const long halves = (2 * tiles + cus - 1) / cus;
  return halves < 2 * whole ? 2 : 1;
}

int launch_expert_gemm(const ExpertArgs &ea, const DispatchBufs &db, hipStream_t s) {
  if (ea.calls != 1)
    return moe_fail(MOE_EXECUTION_FAILED, "expert gemm: one call per launch");
  if (ea.act_i8 && ea.mode == MODE_DOWN) {
    const int cus = gemm_cus();
    if (cus <= 0) return moe_fail(MOE_EXECUTION_FAILED, "expert gemm: no CU count for the device");
    return launch_gemm_down_i8(ea, db, cus, s);
  }
  GemmArgs p;
  p.a = ea.a;
  p.a_row_div = ea.a_row_div;
  p.a_bytes = (int)((int64_t)(ea.A / ea.a_row_div) * ea.K * (ea.a_dtype == MOE_F16 ? 2 : 4));
  p.w0 = ea.w0.w;
  p.s0 = ea.w0.scales;
  p.b0 = ea.w0.bias;
  // Down reads its one weight through both sources (units 0..63 and 64..127
  // of the tile).
  p.w1 = ea.mode == MODE_UP ? ea.w1.w : ea.w0.w;
  p.s1 = ea.mode == MODE_UP ? ea.w1.scales : ea.w0.scales;
  p.b1 = ea.mode == MODE_UP ? ea.w1.bias : ea.w0.bias;
  p.K = ea.K;
  p.N = ea.N;
  p.E = ea.E;
  p.out = ea.out;
  p.out_bytes = (int)((int64_t)ea.A * ea.N * 4 * (ea.mode == MODE_DOWN && ea.parts == 2 ? 2 : 1));
  p.perm = db.perm;
  p.perm_bytes = ea.A * 4;
  p.sorted = ea.dispatch_order;
  p.active = db.active;
  p.meta = db.meta;
  const int cols = ea.mode == MODE_UP ? 256 : 512;  // output columns per tile
  p.nt = (ea.N + cols - 1) / cols;
  p.parts = ea.mode == MODE_DOWN && ea.parts == 2 ? 2 : 1;
  p.kpart = ea.K / BK / p.parts;
  p.part_floats = ea.A * ea.N;
  p.act_i8 = ea.act_i8;
  p.act_npairs = ea.N / 64;
  if (ea.act_i8) {
    if (ea.mode != MODE_UP || !gemm_wide_eligible(ea) || ea.N % 64)
      return moe_fail(MOE_EXECUTION_FAILED, "expert gemm: int8-limb act needs the f16-x up GEMM");
    p.out_bytes = (int)gemm_i8_act_bytes(ea.A, ea.E, ea.N);
  }
  if (p.kpart < 3 * gemm_stages(ea))
    return moe_fail(MOE_EXECUTION_FAILED, "expert gemm: too few steps per K part");
  // Persistent blocks, one per CU (the LDS ring takes a CU), a multiple of 8
  // for the XCD split; blocks past the tile count exit at once.
  const int cus = gemm_cus();
  if (cus <= 0) return moe_fail(MOE_EXECUTION_FAILED, "expert gemm: no CU count for the device");
  long blocks = gemm_mtiles(ea) * p.nt * p.parts;
  if (blocks > cus) blocks = cus;
  blocks = (blocks + 7) / 8 * 8;
  dim3 grid((unsigned)blocks), block(512);
  // Dispatch-order act (the fused layer, both products here) is stored as
  // f16 pairs: up writes them, down reads them.
  const bool pairs = ea.dispatch_order != 0;
  // Paired steps (one barrier per 64 k) when each part has an even number
  // of steps.
  const bool pair = p.kpart % 2 == 0;
  // Up with f16 x: weights straight into registers (gemm_wide.hip).
  if (gemm_wide_eligible(ea))
    return launch_gemm_up_wide(p, (int)blocks, ea.act_i8 ? 2 : pairs ? 1 : 0, s);
#define LAUNCH_P(M_, AT_, OP_)                                                            \
  do {                                                                                    \
    if (pair) hipLaunchKernelGGL((k_expert_gemm<M_, AT_, OP_, true>), grid, block, 0, s, p); \
    else hipLaunchKernelGGL((k_expert_gemm<M_, AT_, OP_, false>), grid, block, 0, s, p);  \
  } while (0)
  if (ea.mode == MODE_UP) {
    if (ea.a_dtype == MOE_F16) {
      if (pairs) LAUNCH_P(MODE_UP, _Float16, true);
      else LAUNCH_P(MODE_UP, _Float16, false);
    } else {
      if (pairs) LAUNCH_P(MODE_UP, float, true);
      else LAUNCH_P(MODE_UP, float, false);
    }
  } else if (pairs) {
    if (ea.a_dtype != MOE_F32)
      return moe_fail(MOE_EXECUTION_FAILED, "expert gemm: dispatch-order act must be f32");
    LAUNCH_P(MODE_DOWN, f16pair, false);
  } else {
    if (ea.a_dtype == MOE_F16) LAUNCH_P(MODE_DOWN, _Float16, false);
    else LAUNCH_P(MODE_DOWN, float, false);
  }
#undef LAUNCH_P
  return 0;
}
