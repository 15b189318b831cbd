// Grouped gate/up GEMM for prefill shapes with f16 x: weights straight from
// global memory into registers, x through an LDS ring.
//
// Reference: src/core/kernels/matmul/moeQuantW.ts:122-175 (moeUp: glu and lin
// products of the routed rows, clamped SwiGLU); quantW layout
// src/core/kernels/quantCommon.ts:8-31. Same results as the up product of
// gemm.hip and expert.hip.
//
// Tiles, their order and the wavefront shape are those of gemm.hip's
// k_expert_gemm for f16 x: 128 rows of one expert × the same 64 units of
// glu and lin per block (expert → N-tile → M-tile, contiguous tile ranges per
// XCD); eight wavefronts, two per SIMD, each all 128 rows × 16 slots (8 glu
// units and the same 8 lin units) with two of each unit's four columns per
// lane: 4 × 2 v_mfma_f32_32x32x16_f16 tiles, so one converted weight
// fragment feeds four MFMAs.
//
// What differs is the weight path. No wavefront shares a weight unit with
// another, so weights skip LDS. Lane l = 32h + 16b + 2σ + s of a wavefront
// holds unit σ of source s (glu, lin), columns 2b and 2b + 1; its MFMA B
// operand for slice kk of a 32-k step is those columns' dwords of quantW
// tiles 4h + 2kk and 4h + 2kk + 1 (k = 16h + 8kk .. + 7). Per step the lane
// loads two whole tiles, 4h + 2b and 4h + 2b + 1 (32 contiguous bytes, two
// 16-byte loads): lanes with b = 0 hold slice 0's tiles, lanes with b = 1
// slice 1's, all four columns. v_permlane16_swap (lane l ↔ l ± 16) of
// dwords (0, 2) and (1, 3) then leaves every lane its own two columns of
// slice 0 in the first result and of slice 1 in the second, with no select.
// The loads run four steps ahead into a rotating set of four register
// buffers. Measured on config 4's up shape: weights through LDS (a
// direct-to-LDS load and a read per byte) took about a third of the
// kernel's time; 8-byte loads straight into registers kept the texture
// data path 88% busy; 16-byte loads halve its instructions. Loads that
// each cover whole lines (one source per instruction) need a DPP exchange
// and selects per step and measured 7% slower.
//
// x rows (shared by all eight wavefronts) come through LDS by direct buffer
// loads (buffer_load … lds), gathered through the dispatch permutation, in
// step pairs: 64 k of a row is 128 bytes, one whole cache line (one step's
// 64 bytes per row took 12-17% longer over the kernel, with a barrier per
// step); one workgroup barrier per pair. x's k order inside a step follows
// the weights': slice kk of lane half h reads 16-byte chunk 4q + 2h + kk of
// the pair's row (q: the step's place in the pair).
//
// Waits: the weight loads are ordinary loads whose waits the compiler places
// (it counts only its own loads, so it waits a little longer than needed).
// The x loads are asm (the compiler does not track loads that write LDS), so
// each step waits on an explicit vmcnt: the number of vector memory
// instructions issued after the awaited one, which the fixed issue order
// below determines (per step one x load, then two weight loads; at tile
// boundaries the row map, the epilogue constants and the epilogue stores).
#include "gemm_dev.h"

namespace {

constexpr int WD_WAVES = 8;
constexpr int WD_SP = 5;                 // x ring stages, two steps each
constexpr int WD_NB = 4;                 // weight register buffers (steps ahead)
constexpr int WD_P_STAGE = BM * 2 * BK * 2;  // 16 KB of f16 x per step pair
constexpr int WD_RT = 4;                 // 32-row MFMA tiles per wavefront
constexpr int WD_CT = 2;                 // columns of each unit per lane
constexpr int WD_WLOADS = 2;             // weight loads per lane and step
constexpr int WD_ALOADS = 2;             // x loads per lane and step pair
constexpr int WD_STORES = WD_RT * 8;     // epilogue stores per lane
constexpr int WD_TILE_LOADS = 2;         // row map + constants, per wavefront and tile
// Instructions younger than the x loads a barrier waits for (see the
// pipeline below): the weight loads of their step, then 2·SP − 3 steps,
// SP − 2 of them with x loads.
constexpr int WD_BASE_WAIT = WD_WLOADS + WD_WLOADS * (2 * WD_SP - 3) + WD_ALOADS * (WD_SP - 2);
static_assert(WD_BASE_WAIT + WD_TILE_LOADS < 64, "vmcnt range");
constexpr int wd_wait(int n) { return n < 63 ? n : 63; }

// The lane id, recomputed where it is used. The kernel runs at the 256-VGPR
// limit; a lane-derived value held across the loop gets spilled, and its
// reload (the youngest load) costs a wait for every load in flight, which
// drains the prefetch pipeline. The asm keeps the compiler from keeping or
// spilling it.
__device__ __forceinline__ int fresh_lane() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

template <int OMODE>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))
void k_gemm_up_direct(GemmArgs p) {
  __shared__ __align__(16) uint8_t aring[WD_SP * WD_P_STAGE];
  __shared__ __align__(16) uint8_t junk[1024];  // target of the placeholder loads
  __shared__ __align__(16) int32_t rowmap[2][BM];
  // Epilogue constants per tile: glu scales, lin scales, glu biases, lin
  // biases (256 each).
  __shared__ __align__(16) float consts[2][1024];
  __shared__ int4 descs[GEMM_MAX_E];

  // ---- this block's tiles (as in k_expert_gemm): 8 contiguous ranges of
  // the tile list, one per XCD, dealt round robin to the XCD's blocks.
  const int total = p.meta[META_TILES] * p.nt;
  const int n_active = p.meta[META_ACTIVE];
  const int bx = gridDim.x >> 3;
  const int xcd = blockIdx.x & 7, xb = blockIdx.x >> 3;
  const int per_x = (total + 7) >> 3;
  const int start = xcd * per_x + xb, end = min(total, (xcd + 1) * per_x);
  if (start >= end) return;
  const int ntiles = (end - start + bx - 1) / bx;

  const int tid = threadIdx.x;
  const int lane = tid & (WAVE - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
  const int lm = lane & 31, h = lane >> 5;
  const int src = lm & 1;          // weight source: 0 glu, 1 lin
  const int usub = (lm >> 1) & 7;  // unit within the wavefront's 8 (per source)
  const int cb = 2 * (lm >> 4);    // first of the lane's two columns
  const int N4 = p.N / 4;
  const int ksteps = p.kpart;

  for (int i = tid; i < n_active; i += blockDim.x) descs[i] = ((const int4 *)p.active)[i];
  __syncthreads();

  auto tile_at = [&](int L) {
    const int t = L / p.nt;
    int lo = 0, hi = n_active - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (descs[mid].w <= t) lo = mid; else hi = mid - 1;
    }
    const int4 d = descs[lo];
    const int mt = (d.z + BM - 1) / BM;
    const int local = L - d.w * p.nt;
    const int ntile = local / mt, mtile = local % mt;
    Tile T;
    T.e = __builtin_amdgcn_readfirstlane(d.x);
    T.r0 = __builtin_amdgcn_readfirstlane(d.y + mtile * BM);
    T.rows = __builtin_amdgcn_readfirstlane(min(BM, d.z - mtile * BM));
    T.U0 = T.U1 = __builtin_amdgcn_readfirstlane(ntile * 64);
    T.part = 0;
    T.kb = 0;
    T.mtg = __builtin_amdgcn_readfirstlane(d.w + mtile);
    return T;
  };

  const uint32_t aring0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)aring;
  const uint32_t junk0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)junk;
  const uint32_t rowmap0 =
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int32_t *)&rowmap[0][0];
  const uint32_t consts0 =
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float *)&consts[0][0];
  const uint64_t slab = (uint64_t)p.K * (uint64_t)p.N;  // weight bytes of one expert
  const i32x4 ar = buffer_rsrc(p.a, (uint32_t)p.a_bytes);
  const i32x4 pr = buffer_rsrc(p.perm, (uint32_t)p.perm_bytes);
  // Wavefronts 2a, 2a + 1 load constant array a (glu scales, lin scales,
  // glu biases, lin biases), halves wave & 1; a missing bias reads zeros
  // from an empty buffer.
  const float *cbase = wave < 2 ? p.s0 : wave < 4 ? p.s1 : wave < 6 ? p.b0 : p.b1;
  const i32x4 cr = buffer_rsrc(cbase, cbase ? (uint32_t)p.E * (uint32_t)p.N * 4u : 0u);

  // Row map (rows 16·wave + lane, lanes < 16; rows past the tile repeat its
  // last) and constants (128 floats per wavefront, lanes < 32) of tile T
  // into buffer sel: one load instruction each per wavefront.
  auto issue_tile = [&](const Tile &T, int sel) {
    const int ln = fresh_lane();
    if (ln < 16) {
      const int r = 16 * wave + ln;
      dma4(pr, (uint32_t)(T.r0 + min(r, T.rows - 1)) * 4u, 0, rowmap0 + sel * (BM * 4) + 64 * wave);
    }
    if (ln < 32) {
      const int col = 4 * T.U0 + (wave & 1) * 128 + 4 * ln;
      dma16(cr, ((uint32_t)T.e * (uint32_t)p.N + (uint32_t)col) * 4u, 0,
            consts0 + sel * 4096 + 512 * wave);
    }
  };

  // x loads of a step pair (64 k: 128 contiguous bytes, a whole cache line,
  // per row): wavefront w fills rows 16w .. 16w + 15, instruction i rows
  // 16w + 8i + (l >> 3), 8 lanes per row. Rows are 128 bytes in LDS, 16-byte
  // chunk c of row r at r·128 + (c ^ sw8(r))·16. A 16-byte fragment read is
  // served 16 lanes (16 rows) at a time; sw8 gives 16 consecutive rows 16
  // different 16-byte bank positions (r & 7 alone repeats after 8 rows and
  // measured 5e7 bank-conflict cycles per config-4 launch). Lane l loads the
  // chunk that belongs at its position, (l & 7) ^ sw8(r).
  struct AOff {
    uint32_t o[WD_ALOADS];
  };
  auto make_aoff = [&](int sel) {
    AOff A;
    const int ln = fresh_lane();
#pragma unroll
    for (int i = 0; i < WD_ALOADS; i++) {
      const int r = 16 * wave + 8 * i + (ln >> 3);
      const uint32_t srow = (uint32_t)(rowmap[sel][r] / p.a_row_div);
      A.o[i] = srow * (uint32_t)p.K * 2u + (uint32_t)((ln & 7) ^ sw8(r)) * 16u;
    }
    return A;
  };
  auto issue_a = [&](const AOff &A, int pair, int stage) {
#pragma unroll
    for (int i = 0; i < WD_ALOADS; i++)
      dma16(ar, A.o[i], pair * 2 * BK * 2, aring0 + stage * WD_P_STAGE + (2 * wave + i) * 1024);
  };
  auto issue_junk = [&]() {
#pragma unroll
    for (int i = 0; i < WD_WLOADS; i++) dma16(ar, 0u, 0, junk0);
  };

  // This lane's weight bytes: unit U0 + 8·wave + usub of its source, tiles
  // 4h + cb and 4h + cb + 1 of each step; a unit past N reads the last unit
  // (its outputs are never stored).
  auto wptr = [&](const Tile &T) -> const uint8_t * {
    const int ln = fresh_lane(), lmf = ln & 31;
    const int u = min(T.U0 + 8 * wave + ((lmf >> 1) & 7), N4 - 1);
    const uint8_t *w = (const uint8_t *)((lmf & 1) ? p.w1 : p.w0);
    return w + (uint64_t)T.e * slab + (uint64_t)u * (uint64_t)p.K * 4u + (uint32_t)(ln >> 5) * 64u +
           (uint32_t)(2 * (lmf >> 4)) * 16u;
  };

  u32x4 wr[WD_NB][2];  // two whole quantW tiles per step, four steps
  auto load_w = [&](u32x4 (&dst)[2], const uint8_t *base, int ks) {
    const uint8_t *q = base + (uint32_t)ks * (BK * 4);
#pragma unroll
    for (int t = 0; t < 2; t++) dst[t] = *(const u32x4 *)(q + 16 * t);
  };
  // The step's B operands from the two loaded tiles: b[kk][c][t] = column
  // cb + c of tile 4h + 2kk + t.
  struct StepB {
    uint32_t b[2][2][2];
  };
  auto unpack_w = [&](const u32x4 (&w)[2]) {
    StepB B;
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int c = 0; c < 2; c++) {
        const auto r = __builtin_amdgcn_permlane16_swap(w[t][c], w[t][c + 2], false, false);
        B.b[0][c][t] = r[0];
        B.b[1][c][t] = r[1];
      }
    return B;
  };

  floatx16 acc[WD_RT][WD_CT];

  // x fragments of one slice: rows 32i + lm, chunk 4q + 2h + kk of the
  // pair's row (q: the step's place in its pair). Row 32i + lm has swizzle
  // sw8(lm) ^ 4·(i & 1), and (4q + kk) ^ 2h ^ sw8(lm) splits into a
  // compile-time and a lane part: each (q, kk) has one offset per lane,
  // odd row tiles take (q ^ 1, kk)'s, and i adds 4096·i, an immediate.
  uint32_t aoff[4];
#pragma unroll
  for (int qk = 0; qk < 4; qk++)
    aoff[qk] = (uint32_t)lm * 128u + 16u * (uint32_t)((4 * (qk >> 1) + (qk & 1)) ^ (2 * h) ^ sw8(lm));
  auto read_a = [&](u32x4 (&F)[WD_RT], int stage, int q, int kk) {
    const uint8_t *st0 = aring + stage * WD_P_STAGE + aoff[2 * q + kk];
    const uint8_t *st1 = aring + stage * WD_P_STAGE + aoff[2 * (q ^ 1) + kk];
#pragma unroll
    for (int i = 0; i < WD_RT; i++) F[i] = *(const u32x4 *)(((i & 1) ? st1 : st0) + 4096 * i);
  };
  auto mfma_slice = [&](const u32x4 (&F)[WD_RT], const StepB &w, int kk) {
    half8 bf[WD_CT];
    bf[0] = cvt_i8x8(w.b[kk][0][0], w.b[kk][0][1]);
#pragma unroll
    for (int c = 0; c < WD_CT; c++) {
      if (c + 1 < WD_CT) bf[c + 1] = cvt_i8x8(w.b[kk][c + 1][0], w.b[kk][c + 1][1]);
#pragma unroll
      for (int i = 0; i < WD_RT; i++)
        acc[i][c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, F[i]), bf[c],
                                                           acc[i][c], 0, 0, 0);
    }
  };

  // ---- epilogue: an even lane holds glu and the odd lane after it lin of
  // the same unit and columns. The even lane finishes rows r < 8 of each
  // accumulator, the odd lane rows r ≥ 8, each taking the other projection's
  // values for its rows from its partner (a DPP swap of lanes 2j, 2j + 1). Outputs go through
  // buffer stores whose offset is out of range for rows or units past the
  // tile (the store is dropped), with no branch.
  const __amdgpu_buffer_rsrc_t orc =
      __builtin_amdgcn_make_buffer_rsrc(p.out, 0, p.out_bytes, BUF_DWORD3);
  auto pick = [](uint32_t m, float x, float y) {
    return __builtin_bit_cast(float, (m & __builtin_bit_cast(uint32_t, x)) |
                                         (~m & __builtin_bit_cast(uint32_t, y)));
  };
  auto epilogue = [&](const Tile &T, int sel) {
    const bool low = src == 0;
    const uint32_t lowm = low ? ~0u : 0u;
    const int uo = T.U0 + 8 * wave + usub;
    const bool col_ok = uo < N4;
    const int q = 4 * (uo - T.U0) + cb;
    const float *cs = consts[sel];
    const floatx2 sg = *(const floatx2 *)&cs[q], sl = *(const floatx2 *)&cs[256 + q];
    const floatx2 bg = *(const floatx2 *)&cs[512 + q], bl = *(const floatx2 *)&cs[768 + q];
#pragma unroll
    for (int i = 0; i < WD_RT; i++)
#pragma unroll
      for (int r = 0; r < 8; r++) {
        float v[WD_CT];
#pragma unroll
        for (int c = 0; c < WD_CT; c++) {
          const float a0 = acc[i][c][r], a8 = acc[i][c][r + 8];
          const float send = pick(lowm, a8, a0);
          const float recv = __builtin_bit_cast(
              float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, send), 0xB1, 0xF, 0xF, true));
          const float g = pick(lowm, a0, recv);
          const float l = pick(lowm, recv, a8);
          v[c] = swiglu(g * sg[c] + bg[c], l * sl[c] + bl[c]);
        }
        const int rr = low ? r : r + 8;
        const int row = 32 * i + 8 * (rr / 4) + 4 * h + (rr % 4);
        const bool ok = row < T.rows && col_ok;
        if constexpr (OMODE == 2) {
          // int8 limbs of V = rint(v·2^17) (gemm_i8.hip): padded row
          // P = 128·mtg + row, k = 4·uo + cb (even) and k + 1.
          const uint32_t P = 128u * (uint32_t)T.mtg + (uint32_t)row;
          const uint32_t k = 4u * (uint32_t)uo + (uint32_t)cb;
          const uint32_t base =
              ((P >> 6) * (uint32_t)p.act_npairs + (k >> 6)) * 12288u + ((k >> 5) & 1u) * 2048u +
              ((k >> 4) & 1u) * 1024u + (P & 63u) * 16u + (k & 15u);
          uint32_t w[WD_CT];
#pragma unroll
          for (int c = 0; c < WD_CT; c++)
            w[c] = (uint32_t)((int)__builtin_rintf(fminf(fmaxf(v[c], -63.5f), 63.5f) * 131072.0f) +
                              32896);
          // limbs h = b2, m = b1 ^ 0x80, l = b0 ^ 0x80, at L·4096.
          const uint32_t hh = ((w[0] >> 16) & 0xffu) | (((w[1] >> 16) & 0xffu) << 8);
          const uint32_t mm = (((w[0] >> 8) & 0xffu) | (((w[1] >> 8) & 0xffu) << 8)) ^ 0x8080u;
          const uint32_t ll = ((w[0] & 0xffu) | ((w[1] & 0xffu) << 8)) ^ 0x8080u;
          const uint32_t o0 = ok ? base : 0x80000000u;
          __builtin_amdgcn_raw_buffer_store_b16((unsigned short)hh, orc, o0, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b16((unsigned short)mm, orc, ok ? base + 4096u : o0, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b16((unsigned short)ll, orc, ok ? base + 8192u : o0, 0, 0);
        } else {
          const uint32_t orow = p.sorted ? (uint32_t)(T.r0 + row) : (uint32_t)rowmap[sel][row];
          const uint32_t off = ok ? (orow * (uint32_t)p.N + 4u * uo + (uint32_t)cb) * 4u
                                  : 0x80000000u;
          u32x2 o;
          if constexpr (OMODE == 1) {
            // The f32 pair's 8 bytes as hi(n), hi(n + 1), lo(n), lo(n + 1).
            const _Float16 h0 = (_Float16)v[0], h1 = (_Float16)v[1];
            o[0] = __builtin_bit_cast(uint32_t, half2v{h0, h1});
            o[1] = __builtin_bit_cast(
                uint32_t, half2v{(_Float16)(v[0] - (float)h0), (_Float16)(v[1] - (float)h1)});
          } else {
            o[0] = __builtin_bit_cast(uint32_t, v[0]);
            o[1] = __builtin_bit_cast(uint32_t, v[1]);
          }
          __builtin_amdgcn_raw_buffer_store_b64(o, orc, off, 0, 0);
        }
      }
  };

  // ---- the pipeline. x comes in step pairs P = (2P, 2P + 1), pair P in
  // ring slot P mod SP; weights step by step. Step ks (x fragments of both
  // slices already in registers, weights of step ks in buffer ks % 4):
  //   slice 0 MFMAs;
  //   odd ks only: wait for this wavefront's x loads of the next pair and
  //   its LDS reads, barrier (the next pair landed, every read of this
  //   pair's slot done), [next tile's row map and constants at tile_step],
  //   x loads of pair (ks + 1)/2 + SP − 1 into this pair's slot;
  //   read step ks + 1's slice-0 fragments; slice 1 MFMAs; weight loads of
  //   step ks + 4 into buffer ks % 4; read step ks + 1's slice-1 fragments.
  // The x loads of a pair go out 2·SP − 2 steps before the barrier that
  // waits for them. Loads past a tile's end belong to the next tile; past
  // the last tile they re-read its last pair / step, so every step issues
  // the same instructions. The prologue issues pairs 0 .. SP − 1 as 2·SP
  // virtual steps of the same pattern (the weights of steps 0-3 in the last
  // four, placeholder loads into LDS before them), so the counts hold from
  // step 0.
  Tile cur = tile_at(start), nxt = cur;
  issue_tile(cur, 0);
  WAIT_VMCNT(0);
  block_barrier();
  AOff pa = make_aoff(0), pan = pa;
  if (ntiles > 1) nxt = tile_at(start + bx);
  const uint8_t *wp = wptr(cur);
  const uint8_t *wpn = ntiles > 1 ? wptr(nxt) : wp;
#pragma unroll
  for (int v = 0; v < 2 * WD_SP; v++) {
    if (v & 1) issue_a(pa, v >> 1, v >> 1);
    const int b = v - (2 * WD_SP - WD_NB);  // weight step loaded by this virtual step
    if (b < 0) issue_junk();
    else if (b == 0) load_w(wr[0], wp, 0);
    else if (b == 1) load_w(wr[1], wp, 1);
    else if (b == 2) load_w(wr[2], wp, 2);
    else load_w(wr[3], wp, 3);
  }
  // Pair 0: issued at virtual step 1, then 2·SP − 2 more steps.
  WAIT_VMCNT(WD_WLOADS * (2 * WD_SP - 1) + WD_ALOADS * (WD_SP - 1));
  block_barrier();
  u32x4 F0[WD_RT], F1[WD_RT];
  read_a(F0, 0, 0, 0);
  read_a(F1, 0, 0, 1);

  const int npairs = ksteps / 2;
  // Barrier steps are odd. The next tile's first x loads go out at
  // param_step; its row map and constants at tile_step, early enough that
  // the barrier of param_step has waited for them.
  const int param_step = 2 * (npairs - WD_SP) + 1;
  const int tile_step = param_step - 2 * WD_SP + 2;
  int stage = 0;  // ring slot of the current pair
  for (int j = 0; j < ntiles; j++) {
    const bool has_next = j + 1 < ntiles;
    const int sel = j & 1;
#pragma unroll
    for (int i = 0; i < WD_RT; i++)
#pragma unroll
      for (int c = 0; c < WD_CT; c++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][c][r] = 0.f;

    auto step = [&](int ks, auto bi) {
      constexpr int BI = decltype(bi)::value;  // ks % 4: odd for odd ks
      const StepB wb = unpack_w(wr[BI]);
      mfma_slice(F0, wb, 0);
      int nstage = stage, nq = 1;
      if constexpr ((BI & 1) != 0) {
        // The awaited x loads went out at step ks − 2·SP + 2 (a barrier
        // step, before its weight loads): the previous tile's epilogue
        // stores are younger when that step was in the previous tile, the
        // next tile's row map and constants when they went out later.
        const bool stores_younger = j > 0 && ks < 2 * WD_SP - 2;
        const bool tile_younger = has_next && ks > tile_step && tile_step > ks - 2 * WD_SP + 2;
        if (stores_younger) WAIT_VMCNT(wd_wait(WD_BASE_WAIT + WD_STORES));
        else if (tile_younger) WAIT_VMCNT(WD_BASE_WAIT + WD_TILE_LOADS);
        else WAIT_VMCNT(WD_BASE_WAIT);
        // This wavefront's LDS reads of the pair done (asm: the compiler
        // drops a builtin wait it considers redundant).
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        block_barrier();
        if (has_next && ks == tile_step) issue_tile(nxt, sel ^ 1);
        if (has_next && ks == param_step) pan = make_aoff(sel ^ 1);
        {
          // Selects, not branches: a load under a branch makes the compiler
          // wait for every load in flight where the paths join.
          const int a = (ks >> 1) + WD_SP;
          const bool an = a >= npairs && has_next;
          AOff A;
#pragma unroll
          for (int i = 0; i < WD_ALOADS; i++) A.o[i] = an ? pan.o[i] : pa.o[i];
          issue_a(A, a < npairs ? a : has_next ? a - npairs : npairs - 1, stage);
        }
        stage = stage + 1 == WD_SP ? 0 : stage + 1;
        nstage = stage;
        nq = 0;
      }
      read_a(F0, nstage, nq, 0);
      mfma_slice(F1, wb, 1);
      {
        const int b = ks + WD_NB;
        load_w(wr[BI], b >= ksteps && has_next ? wpn : wp,
               b < ksteps ? b : has_next ? b - ksteps : ksteps - 1);
      }
      read_a(F1, nstage, nq, 1);
    };
    for (int ks = 0; ks < ksteps; ks += WD_NB) {
      step(ks, std::integral_constant<int, 0>());
      step(ks + 1, std::integral_constant<int, 1>());
      step(ks + 2, std::integral_constant<int, 2>());
      step(ks + 3, std::integral_constant<int, 3>());
    }
    epilogue(cur, sel);
    if (has_next) {
      cur = nxt;
      pa = pan;
      wp = wpn;
      if (j + 2 < ntiles) {
        nxt = tile_at(start + (j + 2) * bx);
        wpn = wptr(nxt);
      }
    }
  }
  // The last steps' x loads (re-reads) still write LDS.
  WAIT_VMCNT(0);
}

}  // namespace

bool gemm_wide_eligible(const ExpertArgs &ea) {
  return ea.mode == MODE_UP && ea.a_dtype == MOE_F16 && gemm_eligible(ea) &&
         ea.K / BK >= 4 * WD_SP && (ea.K / BK) % WD_NB == 0;
}

int launch_gemm_up_wide(const GemmArgs &p, int blocks, int omode, hipStream_t s) {
  dim3 grid((unsigned)blocks), block(WD_WAVES * WAVE);
  if (omode == 2) hipLaunchKernelGGL((k_gemm_up_direct<2>), grid, block, 0, s, p);
  else if (omode == 1) hipLaunchKernelGGL((k_gemm_up_direct<1>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((k_gemm_up_direct<0>), grid, block, 0, s, p);
  return 0;
}
