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
#include <stdlib.h>

#include "moe_internal.h"
#include "norm_dev.h"
#include "router_dev.h"

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
  int rc;  // rows staged per chunk (skinny kernel)
  // act in dispatch order (fused layer): up writes row p of the sorted
  // order, down reads it there, so neither waits on perm for those rows.
  int sorted;
  DispatchBufs db;
  const float *a_inv;   // moe_block's pre-norm (up, skinny kernel), or NULL
  const void *a_normw;
  // Up of single-token calls: the router's fold, top-k and dispatch in the
  // prologue (fused_route), from the chunk sums; NULL otherwise.
  const float *fr_partial;
  const float *fr_b;
  int64_t fr_b_cs;
  int fr_J, fr_tile_m;
};

// Dynamic LDS fused_route borrows before the staging (int32 words).
__host__ __device__ constexpr int fused_route_words(int E) { return 96 + 2 * E + 1; }

// Single-token calls (p.fr_partial): the router's fold (chunk order, then
// + b), top-k and the call's dispatch, recomputed by every block of the
// call from its J·E chunk sums, so that no separate kernel sits between the
// router's chunk kernel and this product. The fold and top-k are the
// router's own (router_dev.h, bit for bit); block (0, 0) writes the route
// row, perm and the dispatch buffers (offsets, M-tiles, active experts,
// meta) as the router's fused dispatch kernel does. Returns this block's
// {expert, first sorted row, rows, 0}, expert −1 past the call's distinct
// experts. Every thread calls it; `lds` (fused_route_words(E) words of the
// dynamic LDS) is free again on return. Requires E ≤ 256, k ≤ 16, J ≤ 16.
__device__ int4 fused_route(const ExpertKArgs &p, int call, int32_t *lds) {
  const int lane = threadIdx.x & (WAVE - 1);
  const int E = p.E, k = p.k, J = p.fr_J;
  int32_t *ev = lds;                     // [16] distinct experts, ascending
  int32_t *pv = lds + 16;                // [16] first sorted row of each
  int32_t *cv = lds + 32;                // [16] rows of each
  int32_t *nd = lds + 48;                // distinct count
  float *rowbuf = (float *)(lds + 64);   // [2k] route row of the other blocks
  int32_t *hist = lds + 96;              // [E]
  int32_t *cur = hist + E;               // [E + 1]
  const bool writer = blockIdx.x == 0 && blockIdx.y == 0;
  if (threadIdx.x < WAVE) {
    const float *part = p.fr_partial + (int64_t)call * J * E;
    const float *b = p.fr_b ? p.fr_b + call * p.fr_b_cs : nullptr;
    // Every chunk sum of the lane's experts loaded before the first add.
    float v[4][16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int e = min(lane + WAVE * i, E - 1);
#pragma unroll
      for (int u = 0; u < 16; u++) v[i][u] = part[(int64_t)min(u, J - 1) * E + e];
    }
    float vals[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int e = lane + WAVE * i;
      float sum = v[i][0];
#pragma unroll
      for (int u = 1; u < 16; u++)
        if (u < J) sum = sum + v[i][u];
      if (b && e < E) sum = sum + b[e];
      vals[i] = e < E ? sum : -INFINITY;
    }
    // The route buffer is the layer's own (written here, read by the combine).
    float *row = writer ? const_cast<float *>(p.route) + call * p.route_cs : rowbuf;
    const int id = moe_dev::wave_topk_route<4>(vals, E, k, lane, row);
    // The stable counting sort of the k slots: slot s goes to row
    // (ids below its id) + (earlier slots with its id).
    const int my = lane < k ? id : 0x7fffffff;
    int less = 0, eqb = 0, cnt = 0;
    for (int j = 0; j < k; j++) {
      const int o = __shfl(my, j);
      less += o < my;
      eqb += (j < lane) && (o == my);
      cnt += o == my;
    }
    const bool first = lane < k && eqb == 0;
    int drank = 0;
    for (int j = 0; j < k; j++) {
      const int o = __shfl(my, j);
      const int of = __shfl((int)first, j);
      drank += of && o < my;
    }
    if (first) {
      ev[drank] = my;
      pv[drank] = less;
      cv[drank] = cnt;
    }
    const int ndist = __popcll(__ballot(first));  // every lane votes: outside the branch
    if (lane == 0) *nd = ndist;
    if (writer) {
      int32_t *perm = p.db.perm + call * p.db.perm_cs();
      if (lane < k) perm[less + eqb] = lane;
      for (int e = lane; e < E; e += WAVE) hist[e] = 0;
      if (first) hist[my] = cnt;
      moe_dev::wave_scan_experts(hist, E, p.fr_tile_m, lane, p.db.offsets + call * p.db.off_cs(),
                                 p.db.tile_off + call * p.db.off_cs(),
                                 p.db.active + call * p.db.act_cs(),
                                 p.db.meta + call * p.db.meta_cs(), cur);
    }
  }
  __syncthreads();
  const int y = blockIdx.y;
  int4 d = {-1, 0, 0, 0};
  if (y < *nd) d = int4{ev[y], pv[y], cv[y], 0};
  __syncthreads();
  return d;
}

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

// A rows staged in LDS as f16: row r, k at rows[r·kp + k] (kp = K rounded
// up to whole 32-wide K steps — the fragments of the last step read that far,
// and the staging writes zeros there — plus 8 halves of padding that shifts
// each row by 4 banks), and
// for f32 input a second plane with the low parts: v = hi + lo to ~2^-22.
template <typename AT>
struct AStage {
  static constexpr bool SPLIT = sizeof(AT) == 4;
  static constexpr int PLANES = SPLIT ? 2 : 1;
};

__host__ __device__ __forceinline__ int a_stage_kp(int K) { return ((K + 31) & ~31) + 8; }

// Rows per chunk that keep the staged A within 64 KB of LDS.
__host__ __device__ __forceinline__ int a_stage_rows(int K, bool split) {
  const int bytes_per_row = a_stage_kp(K) * 2 * (split ? 2 : 1);
  int r = 16;
  while (r > 1 && r * bytes_per_row > 65536) r >>= 1;
  return r;
}

typedef _Float16 half4 __attribute__((ext_vector_type(4)));

// Lane group kq of a 32-wide K step holds k = 8kq .. 8kq+7 of its row: the
// same k as the lane's B tiles (2kq and 2kq + 1 of the step).
__device__ __forceinline__ half8 a_frag(const _Float16 *plane, int kp, int row, int step, int kq) {
  return *(const half8 *)(plane + row * kp + step * 32 + 8 * kq);
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Weight tiles of one K step of one wavefront, as loaded: t0 from the
// wavefront's units 0-7, t1 from units 8-15 (see the load mapping below).
struct WStep {
  u32x4 t0, t1;
};

// Weight loads. A step's two load instructions each cover whole 128-byte
// lines (8 units × the step's 8 tiles), so a nontemporal load fetches every
// line once; the lanes then trade tiles (row_ror:8) into the MFMA layout.
// Nontemporal loads stream from HBM at ~7.1 TB/s on MI355X against ~6.3 TB/s
// for plain loads (same access pattern, measured). They are buffer loads
// with no branch around them: an offset past the buffer reads zeros, so a
// tile past K or a unit past N costs no divergent code, and the compiler's
// wait counts stay exact (a load under a branch makes it wait for every
// load in flight at the join, which empties the pipeline).
constexpr uint32_t OOB = 0x80000000u;
constexpr int BUF_DWORD3 = 0x00020000;  // raw buffer, 32-bit data format
__device__ __forceinline__ u32x4 load_stream(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2 /* nt */));
}

// Lane L of a 16-lane row receives the value of lane L ^ 8 (DPP row_ror:8).
__device__ __forceinline__ uint32_t swap8(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xf, 0xf, false);
}

// k_expert_skinny: one block = one active expert × NW·(column groups per
// wavefront) groups of 64 output columns (16 quantW units each). The
// expert's rows are taken RC at a time (RC ≤ 16 keeps them in LDS); for each
// chunk the NW wavefronts stage the rows' A in LDS once, then each wavefront
// streams its segments — up: glu then lin of one column group; down: NS
// column groups — as one continuous stream over K through a 4-stage register
// pipeline: the loads of steps g+1..g+3 are in flight while step g converts
// and multiplies. A comes from LDS, so its reads never wait behind the weight
// stream; scales and biases are fetched before the stream starts. The glu
// sums wait in LDS for the SwiGLU epilogue.
// GROUPED: scales change along K (groupSize < K), so partial sums are
// scaled per group; otherwise one scale per column is applied at the end.
// KS = 2 or 4 splits every stream over KS wavefronts, each taking a
// contiguous 1/KS of K (more wavefronts, and more of each stream's loads in
// flight at once, when few experts and columns are active); at each segment
// end the later parts' sums meet the first's in LDS, added in part order,
// before the scales, biases and SwiGLU.
// NWS streams per block; the block has NW = NWS·KS wavefronts.
// Weight stream buffers per wavefront (loads SK_PD − 1 steps ahead). 6 and 8
// measured slower at configs 2 and 3 (fewer wavefronts fit), up to 25%.
constexpr int SK_PD = 4;
#ifndef SKINNY_KS4_STREAMS
#define SKINNY_KS4_STREAMS 256
#endif
// NORM: gate/up of moe_block with the pre-norm applied while staging
// (a_inv, a_normw); a template flag, so that the instances without it keep
// their registers.
template <int MODE, typename AT, bool GROUPED, int NWS, int NS, int KS, bool NORM = false>
__global__ __launch_bounds__(64 * NWS * KS) __attribute__((amdgpu_waves_per_eu(NS == 1 ? 3 : 4))) void k_expert_skinny(
    ExpertKArgs p) {
  constexpr int NW = NWS * KS;
  static_assert(KS == 1 || ((KS == 2 || KS == 4) && !GROUPED),
                "K split only with one scale per column");
  // Up with NS = 2: one wavefront streams glu then lin of its column group.
  // Up with NS = 1: glu and lin on paired wavefronts (2w, 2w+1), which meet
  // in LDS after the stream. Down: NS column groups per wavefront.
  constexpr bool PAIRED = MODE == MODE_UP && NS == 1;
  static_assert(!PAIRED || NWS % 2 == 0, "paired up needs an even stream count");
  constexpr int GPW = (MODE == MODE_UP) ? 1 : NS;  // column groups per wavefront
  constexpr bool SPLIT = AStage<AT>::SPLIT;
  // LDS: the staged A rows, then each wavefront's parked glu sums
  // [NW][4][64] floatx4 (up only).
  extern __shared__ __align__(16) unsigned char smem[];
  _Float16 *ahi = (_Float16 *)smem;

  const int call = blockIdx.z;
  int4 desc;
  if (MODE == MODE_UP && p.fr_partial) {
    desc = fused_route(p, call, (int32_t *)smem);
  } else {
    desc = ((const int4 *)(p.db.active + call * p.db.act_cs()))[blockIdx.y];
  }
  const int e = desc.x;
  if (e < 0) return;
  const int p0 = desc.y, cnt = desc.z;
  const int32_t *perm = p.db.perm + call * p.db.perm_cs();
  const AT *abase = (const AT *)p.a + call * p.a_cs;
  float *out = p.out + call * p.out_cs;

  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = threadIdx.x / WAVE;
  const int sw = wave / KS;     // stream of this wavefront
  const int kpart = wave % KS;  // its part of K when split
  const int N4 = p.N / 4, K4 = p.K / 4;
  const int arr = PAIRED ? (sw & 1) : 0;  // weight array of a paired stream
  const int cg0 = PAIRED ? blockIdx.x * (NWS / 2) + (sw >> 1)
                         : (blockIdx.x * NWS + sw) * GPW;  // first column group
  int useg[NS];
  bool uok[NS];
#pragma unroll
  for (int j = 0; j < NS; j++) {
    useg[j] = (cg0 + (MODE == MODE_UP ? 0 : j)) * 16 + (lane & 15);
    uok[j] = useg[j] < N4;
  }
  const int kq = lane >> 4;
  const int m = lane & 15;
  const int steps = (p.K + 31) / 32;
  const int lsteps = steps / KS;  // steps of this wavefront per segment (KS divides steps)
  const int kbeg = kpart * lsteps;
  const int gsteps = NS * lsteps;
  const int kg = p.K / p.g;
  const int kp = a_stage_kp(p.K);
  const int RC = p.rc;
  const int planes = SPLIT ? 2 : 1;
  _Float16 *alo = ahi + RC * kp;
  floatx4 *park0 = (floatx4 *)(smem + (size_t)RC * kp * 2 * planes);
  floatx4 *park = park0 + (PAIRED ? (sw >> 1) : sw) * 4 * WAVE;
  // K-split partial sums, KS − 1 [4][64] floatx4 slots per stream, after the
  // parks.
  floatx4 *red = park0 + (MODE == MODE_UP ? (PAIRED ? NWS / 2 : NWS) : 0) * 4 * WAVE +
                 sw * (KS - 1) * 4 * WAVE;

  // Loaded units: instruction 0 takes unit 16·cg + (lane & 7), instruction 1
  // unit 16·cg + 8 + (lane & 7); tile (lane >> 3) of the step, ^ 1 for
  // instruction 1. After the row_ror:8 trade every lane holds tiles 2kq and
  // 2kq + 1 of its own unit 16·cg + (lane & 15).
  __amdgpu_buffer_rsrc_t wr[NS];
  uint32_t wl[NS][2];  // byte offset of the lane's unit in the expert's slab, or OOB
  const float *sc[NS];
  floatx4 sone[NS], bias[NS];
#pragma unroll
  for (int j = 0; j < NS; j++) {
    const bool second = MODE == MODE_UP && (PAIRED ? arr == 1 : j == 1);
    const uint32_t *w = second ? p.w1 + call * p.w1_cs : p.w0 + call * p.w0_cs;
    sc[j] = second ? p.s1 + call * p.s1_cs : p.s0 + call * p.s0_cs;
    const float *b = second ? (p.b1 ? p.b1 + call * p.b1_cs : nullptr)
                            : (p.b0 ? p.b0 + call * p.b0_cs : nullptr);
    const uint32_t slab = (uint32_t)p.K * (uint32_t)p.N * (uint32_t)p.bits / 8u;
    wr[j] = __builtin_amdgcn_make_buffer_rsrc((void *)((const char *)w + (int64_t)e * slab), 0,
                                              (int)slab, BUF_DWORD3);
#pragma unroll
    for (int h2 = 0; h2 < 2; h2++) {
      const int u = (useg[j] & ~15) + 8 * h2 + (lane & 7);
      wl[j][h2] = u < N4 ? (uint32_t)u * (uint32_t)K4 * 16u : OOB;
    }
    // This segment's 4 columns: scales (one group) and biases, fetched early.
    sone[j] = (!GROUPED && uok[j]) ? *(const floatx4 *)(sc[j] + (int64_t)e * p.N + 4 * useg[j])
                                   : floatx4{0.f, 0.f, 0.f, 0.f};
    bias[j] = (b && uok[j]) ? *(const floatx4 *)(b + (int64_t)e * p.N + 4 * useg[j])
                            : floatx4{0.f, 0.f, 0.f, 0.f};
  }

  // Stream step g = seg·steps + s: per instruction, 8 lanes read one unit's
  // 8 tiles of the step (128 contiguous bytes).
  const int lt = lane >> 3;
  const bool odd = (lane & 8) != 0;
  // Steps past the stream load zeros (out-of-range offsets), so every
  // phase of the pipeline issues its loads unconditionally.
  auto issue = [&](int g, WStep &d) {
    const int seg = NS == 1 ? 0 : (g >= lsteps ? 1 : 0);
    const int s = kbeg + g - seg * lsteps;
    const bool live = g < gsteps;
    const int ka = s * 8 + lt, kb = s * 8 + (lt ^ 1);
    const uint32_t o0 = (live && ka < K4) ? wl[seg][0] + (uint32_t)ka * 16u : OOB;
    const uint32_t o1 = (live && kb < K4) ? wl[seg][1] + (uint32_t)kb * 16u : OOB;
    d.t0 = load_stream(wr[seg], o0);
    d.t1 = load_stream(wr[seg], o1);
  };
  for (int c0 = 0; c0 < cnt; c0 += RC) {
    const int rows = min(RC, cnt - c0);
    WStep wb[SK_PD];
    // The weight stream does not depend on the rows: start it first.
#pragma unroll
    for (int j = 0; j < SK_PD - 1; j++) issue(j, wb[j]);

    // Stage this chunk's A rows (gathered through perm) in LDS. Each thread
    // moves 16-byte pieces (8 halves or 4 floats), 8 pieces in flight at
    // once; each wavefront reads the rows' sources once (lane r: row r) and
    // passes them by shuffle. (Loading element by element, one row at a time,
    // cost several memory latencies per block before the weights streamed.)
    {
      constexpr int EPC = 16 / (int)sizeof(AT);  // elements per piece
      constexpr int NT = 64 * NW;
      const int cpr = kp / EPC;  // pieces per staged row (kp is a multiple of 8)
      const int total = RC * cpr;
      const int srcv = lane >= rows ? 0
                       : (MODE == MODE_DOWN && p.sorted) ? p0 + c0 + lane
                       : (MODE == MODE_UP && p.fr_partial) ? 0  // the call's one token
                                                           : perm[p0 + c0 + lane] / p.a_row_div;
      const bool vec = p.K % EPC == 0 && (((uintptr_t)abase) & 15) == 0;
      const AT *nw = (const AT *)p.a_normw;
      const bool nvec = vec && (((uintptr_t)nw) & 15) == 0;
      // Pieces per batch: 8, or 4 with the norm's weights and inverse RMS
      // loaded alongside.
      constexpr int PB = NORM ? 4 : 8;
      for (int b0 = threadIdx.x; b0 < total; b0 += PB * NT) {
        u32x4 v[PB], nwv[NORM ? PB : 1];
        float invv[NORM ? PB : 1];
#pragma unroll
        for (int u = 0; u < PB; u++) {
          const int c = b0 + u * NT;
          const int r = c < total ? c / cpr : 0;
          const int k = (c - r * cpr) * EPC;
          const int src = __shfl(srcv, r);
          const bool ok = c < total && r < rows;
          const AT *xr = abase + (int64_t)src * p.K;
          if (vec) {
            v[u] = (ok && k < p.K) ? *(const u32x4 *)(xr + k) : u32x4{0, 0, 0, 0};
          } else {
            AT e[EPC];
#pragma unroll
            for (int j = 0; j < EPC; j++) e[j] = (ok && k + j < p.K) ? xr[k + j] : (AT)0;
            v[u] = __builtin_bit_cast(u32x4, e);
          }
          if constexpr (NORM) {
            // The norm's weights and the row's inverse RMS, loaded with x.
            invv[u] = ok ? p.a_inv[src] : 0.f;
            if (nvec) {
              nwv[u] = (ok && k < p.K) ? *(const u32x4 *)(nw + k) : u32x4{0, 0, 0, 0};
            } else {
              AT e[EPC];
#pragma unroll
              for (int j = 0; j < EPC; j++) e[j] = (ok && k + j < p.K) ? nw[k + j] : (AT)0;
              nwv[u] = __builtin_bit_cast(u32x4, e);
            }
          }
        }
        if constexpr (NORM) {
          // moe_block's pre-norm while staging: x·inv·w in f32, rounded to
          // x's dtype, as the standalone norm stores it (after every load of
          // the batch is out).
#pragma unroll
          for (int u = 0; u < PB; u++) {
            const int c = b0 + u * NT;
            const int r = c < total ? c / cpr : 0;
            const int k = (c - r * cpr) * EPC;
            const bool ok = c < total && r < rows;
            AT e[EPC], wn[EPC];
            __builtin_memcpy(e, &v[u], sizeof(e));
            __builtin_memcpy(wn, &nwv[u], sizeof(wn));
#pragma unroll
            for (int j = 0; j < EPC; j++)
              if (ok && k + j < p.K) e[j] = (AT)moe_dev::norm_value<AT>((float)e[j], invv[u], (float)wn[j]);
            v[u] = __builtin_bit_cast(u32x4, e);
          }
        }
#pragma unroll
        for (int u = 0; u < PB; u++) {
          const int c = b0 + u * NT;
          if (c >= total) break;
          const int r = c / cpr, k = (c - r * cpr) * EPC;
          if constexpr (SPLIT) {
            const floatx4 f = __builtin_bit_cast(floatx4, v[u]);
            half4 h, l;
#pragma unroll
            for (int j = 0; j < 4; j++) {
              const _Float16 hv = (_Float16)f[j];
              h[j] = hv;
              l[j] = (_Float16)(f[j] - (float)hv);
            }
            *(half4 *)(ahi + r * kp + k) = h;
            *(half4 *)(alo + r * kp + k) = l;
          } else {
            *(u32x4 *)(ahi + r * kp + k) = v[u];
          }
        }
      }
    }
    // Output rows of this lane's sums (rows 4·kq + q of the chunk), fetched
    // before the stream so that no load waits inside it.
    int orow_i[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int mm = kq * 4 + q;
      orow_i[q] = mm >= rows ? 0 : (MODE == MODE_UP && p.sorted) ? p0 + c0 + mm : perm[p0 + c0 + mm];
    }
    __syncthreads();

    floatx4 tot[4], tmp[GROUPED ? 4 : 1];
#pragma unroll
    for (int i = 0; i < 4; i++) tot[i] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < (GROUPED ? 4 : 1); i++) tmp[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int ar = m < rows ? m : 0;  // rows past the chunk read row 0, masked below
    const bool rok = m < rows;

    // tot[i][q]: row 4·kq + q of the chunk, column 4·useg + i.
    auto finish = [&](int seg) {
      if (KS > 1) {
        // The later parts park their sums; the first adds them in part
        // order ((first + second) + third) + ….
        if (kpart > 0) {
#pragma unroll
          for (int i = 0; i < 4; i++) red[((kpart - 1) * 4 + i) * WAVE + lane] = tot[i];
        }
        __syncthreads();
        if (kpart == 0) {
#pragma unroll
          for (int j = 0; j < KS - 1; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) tot[i] = tot[i] + red[(j * 4 + i) * WAVE + lane];
        }
        __syncthreads();
        if (kpart > 0) {
#pragma unroll
          for (int i = 0; i < 4; i++) tot[i] = floatx4{0.f, 0.f, 0.f, 0.f};
          return;
        }
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        if (!GROUPED) tot[i] = tot[i] * sone[seg][i];
        tot[i] += bias[seg][i];
      }
      if (PAIRED) return;  // the SwiGLU runs after the stream, with the partner
      if (MODE == MODE_UP && seg == 0) {
        // Park glu; the wavefront reads its own lanes back, no barrier.
#pragma unroll
        for (int i = 0; i < 4; i++) {
          park[i * WAVE + lane] = tot[i];
          tot[i] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
        return;
      }
      if (uok[seg]) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int mm = kq * 4 + q;
          if (mm >= rows) continue;
          float *orow = out + (int64_t)orow_i[q] * p.N + 4 * useg[seg];
          floatx4 v;
          if (MODE == MODE_UP) {
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = swiglu(park[i * WAVE + lane][q], tot[i][q]);
          } else {
            v = floatx4{tot[0][q], tot[1][q], tot[2][q], tot[3][q]};
          }
          *(floatx4 *)orow = v;
        }
      }
#pragma unroll
      for (int i = 0; i < 4; i++) tot[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    };

    auto compute = [&](int g, const WStep &d) {
      const int seg = NS == 1 ? 0 : (g >= lsteps ? 1 : 0);
      const int s = kbeg + g - seg * lsteps;
      half8 a_hi = a_frag(ahi, kp, ar, s, kq);
      half8 a_lo;
      if (SPLIT) a_lo = a_frag(alo, kp, ar, s, kq);
      if (!rok) {
        a_hi = half8{};
        if (SPLIT) a_lo = half8{};
      }
      floatx4 *acc = GROUPED ? tmp : tot;
      // Own tile 2kq (t0 on even lanes, t1 on odd), tile 2kq + 1 from lane ^ 8.
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t own = odd ? d.t1[i] : d.t0[i];
        const uint32_t other = swap8(odd ? d.t0[i] : d.t1[i]);
        const half8 bv = cvt_i8x8(own, other);
        acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_hi, bv, acc[i], 0, 0, 0);
        if (SPLIT) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_lo, bv, acc[i], 0, 0, 0);
      }
      if (GROUPED) {
        // Fold the group's partial sums with its scales at each group end.
        const int kend = min(p.K, (s + 1) * 32);
        if (kend % p.g == 0 || s == steps - 1) {
          const int grp = (s * 32) / p.g;
          floatx4 s4 = uok[seg] ? *(const floatx4 *)(sc[seg] + ((int64_t)e * kg + grp) * p.N +
                                                      4 * useg[seg])
                                : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int i = 0; i < 4; i++) {
            tot[i] += tmp[i] * s4[i];
            tmp[i] = floatx4{0.f, 0.f, 0.f, 0.f};
          }
        }
      }
      if (s == kbeg + lsteps - 1) finish(seg);
    };

    // SK_PD buffers in rotation (loads SK_PD − 1 steps ahead). The loads
    // are unconditional (past the stream they read zeros); only the
    // computes are guarded.
    for (int g = 0; g < gsteps; g += SK_PD) {
#pragma unroll
      for (int j = 0; j < SK_PD; j++) {
        issue(g + j + SK_PD - 1, wb[(j + SK_PD - 1) % SK_PD]);
        if (j == 0 || g + j < gsteps) compute(g + j, wb[j]);
      }
    }
    if (PAIRED) {
      // lin wavefront parks its sums; glu wavefront applies the SwiGLU (the
      // first K half of each when split: it holds the whole sums).
      if (arr == 1 && kpart == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++) park[i * WAVE + lane] = tot[i];
      }
      __syncthreads();
      if (arr == 0 && kpart == 0 && uok[0]) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int mm = kq * 4 + q;
          if (mm >= rows) continue;
          float *orow = out + (int64_t)orow_i[q] * p.N + 4 * useg[0];
          floatx4 v;
#pragma unroll
          for (int i = 0; i < 4; i++) v[i] = swiglu(tot[i][q], park[i * WAVE + lane][q]);
          *(floatx4 *)orow = v;
        }
      }
    }
    __syncthreads();  // the next chunk restages A
  }
}

// Rows staged per chunk: no more than the rows an expert can get from T
// tokens with distinct ids per token (more rows only take more chunks), and
// at most what 64 KB of LDS holds.
int skinny_rows(int K, bool split, int T) {
  int r = 1;
  while (r < T && r < 16) r <<= 1;
  const int cap = a_stage_rows(K, split);
  return r < cap ? r : cap;
}

// LDS bytes of k_expert_skinny: the staged A, (up) the parked glu sums and
// (K split) one partial-sum slot per stream.
size_t skinny_lds_bytes(int K, bool split, int rc, int parks, int reds) {
  return (size_t)rc * a_stage_kp(K) * 2 * (split ? 2 : 1) +
         (size_t)(parks + reds) * 4 * WAVE * sizeof(floatx4);
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
  // Sorted act: down reads, up writes, the row at the dispatch position.
  const int64_t arow = (MODE == MODE_DOWN && p.sorted) ? pos : asg / p.a_row_div;
  const int64_t orow = (MODE == MODE_UP && p.sorted) ? pos : asg;
  const AT *x = (const AT *)p.a + call * p.a_cs + arow * p.K;
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
  p.out[call * p.out_cs + orow * p.N + n] = v;
}

// out[t] = residual[t] + Σ_s gate_s · y[t·k + s], slots in order; rows of
// ids that are not experts contribute nothing. Reads, never scatters.
template <typename RT>
__global__ __launch_bounds__(256) void k_combine(const float *__restrict__ y, int64_t y_cs,
                                                 int parts, int64_t part_cs,
                                                 const float *__restrict__ route, int64_t route_cs,
                                                 const RT *__restrict__ residual, int64_t res_cs,
                                                 int T, int N, int E, int k,
                                                 float *__restrict__ out, int64_t out_cs) {
  const int call = blockIdx.z;
  const int t = blockIdx.x;
  const int n = blockIdx.y * 256 + threadIdx.x;
  if (n >= N) return;
  y += call * y_cs;
  route += call * route_cs;
  float acc = residual ? (float)residual[call * res_cs + (int64_t)t * N + n] : 0.f;
  for (int s = 0; s < k; s++) {
    const int64_t asg = (int64_t)t * k + s;
    if (route_expert(route, asg, k, E) < 0) continue;
    const float gate = route[(int64_t)t * 2 * k + k + s];
    float v = y[asg * N + n];
    for (int q = 1; q < parts; q++) v += y[q * part_cs + asg * N + n];
    acc = fmaf(gate, v, acc);
  }
  out[call * out_cs + (int64_t)t * N + n] = acc;
}

// The same for N % 4 == 0: four columns per thread, the slot count a
// template parameter so every slot's loads are in flight together (a
// runtime count leaves the slot array in scratch memory, one load at a
// time); the same order of operations per column.
// Four residual values as f32.
__device__ __forceinline__ float4 load4(const float *p) { return *(const float4 *)p; }
// y is read once: nontemporal 16-byte loads (config 5's combine 60 → 52 µs).
typedef float floatx4_nt __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 load4_nt(const float *p) {
  const floatx4_nt v = __builtin_nontemporal_load((const floatx4_nt *)p);
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ float4 load4(const _Float16 *p) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  const h4 v = *(const h4 *)p;
  return make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
}

template <int KK, typename RT>
__global__ __launch_bounds__(256) void k_combine4(const float *__restrict__ y, int64_t y_cs,
                                                  int parts, int64_t part_cs,
                                                  const float *__restrict__ route, int64_t route_cs,
                                                  const RT *__restrict__ residual, int64_t res_cs,
                                                  int T, int N, int E,
                                                  float *__restrict__ out, int64_t out_cs) {
  const int call = blockIdx.z;
  const int t = blockIdx.x;
  const int n = (blockIdx.y * 256 + threadIdx.x) * 4;
  if (n >= N) return;
  y += call * y_cs;
  route += call * route_cs;
  float4 v[KK];
  bool ok[KK];
  float gate[KK];
#pragma unroll
  for (int s = 0; s < KK; s++) {
    const int64_t asg = (int64_t)t * KK + s;
    ok[s] = route_expert(route, asg, KK, E) >= 0;
    gate[s] = route[(int64_t)t * 2 * KK + KK + s];
    v[s] = load4_nt(&y[asg * N + n]);
  }
  // The residual after the slot loads, so they all wait together.
  float4 acc = residual ? load4(&residual[call * res_cs + (int64_t)t * N + n])
                        : make_float4(0.f, 0.f, 0.f, 0.f);
  for (int q = 1; q < parts; q++) {
#pragma unroll
    for (int s = 0; s < KK; s++) {
      const float4 u = *(const float4 *)&y[q * part_cs + ((int64_t)t * KK + s) * N + n];
      v[s].x += u.x;
      v[s].y += u.y;
      v[s].z += u.z;
      v[s].w += u.w;
    }
  }
#pragma unroll
  for (int s = 0; s < KK; s++) {
    if (!ok[s]) continue;
    acc.x = fmaf(gate[s], v[s].x, acc.x);
    acc.y = fmaf(gate[s], v[s].y, acc.y);
    acc.z = fmaf(gate[s], v[s].z, acc.z);
    acc.w = fmaf(gate[s], v[s].w, acc.w);
  }
  *(float4 *)&out[call * out_cs + (int64_t)t * N + n] = acc;
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
    ExpertKArgs q = p;
    const bool split = ea.a_dtype != MOE_F16;
    const bool grouped = ea.g != ea.K;
    q.rc = skinny_rows(ea.K, split, ea.A / ea.k);
    // Wavefronts per block: enough to share the staged A so it costs at most
    // ~8 KB of LDS per wavefront. Column groups per wavefront (down): 2 for
    // longer weight streams when that still leaves ≥ 2 wavefronts per SIMD.
    const size_t a_bytes = (size_t)q.rc * a_stage_kp(ea.K) * 2 * (split ? 2 : 1);
    int nw = a_bytes <= 8192 ? 1 : a_bytes <= 16384 ? 2 : 4;
    const int ncg = (ea.N / 4 + 15) / 16;
    // Longer streams (NS = 2) for short units (K < 1024: a 4-column unit
    // under 4 KB) while they still give ≥ 2 wavefronts per SIMD. Units of
    // 4 KB and more already stream long enough: batched config-3 calls
    // (K = 2048 and 1408) measured NS = 1 faster at 2-16 calls per launch
    // (up 64-78% against 54-74% of HBM).
    const long waves_ns2 = (long)ea.calls * max_active * (MODE == MODE_UP ? ncg : (ncg + 1) / 2);
    const int ns = (waves_ns2 >= 2048 && ea.K < 1024) ? 2 : 1;
    if (MODE == MODE_UP && ns == 1 && nw == 1) nw = 2;  // glu/lin pairs
    const int gpw = (MODE == MODE_UP) ? 1 : ns;
    const int cg_per_block = (MODE == MODE_UP && ns == 1) ? nw / 2 : nw * gpw;
    // Split K over two wavefronts per stream when the unsplit launch has
    // only a few wavefronts per CU (few active experts and columns: config 1
    // measured 628k → 712k tokens/s). At ~7 wavefronts per CU (config 3) the
    // split measured slower (up 53 → 60 µs): shorter streams pay the per-
    // wavefront start-up twice.
    const long streams = (long)ea.calls * max_active *
                         ((ncg + cg_per_block - 1) / cg_per_block) * nw;
    const int steps = (ea.K + 31) / 32;
    int ks = (!grouped && steps % 2 == 0 && streams < 1024) ? 2 : 1;
    // Very few streams (one single-token call): four wavefronts per stream,
    // so that each one's loads are nearly all in flight at once.
    if (ks == 2 && steps % 4 == 0 && streams < SKINNY_KS4_STREAMS && nw <= 2) ks = 4;
    dim3 grid((ncg + cg_per_block - 1) / cg_per_block, max_active, ea.calls), block(64 * nw * ks);
    // Up parks one [4][64] floatx4 per stream (per pair when paired).
    const int parks = MODE == MODE_UP ? (ns == 1 ? nw / 2 : nw) : 0;
    size_t lds = skinny_lds_bytes(ea.K, split, q.rc, parks, nw * (ks - 1));
    if (q.fr_partial) lds = std::max(lds, (size_t)fused_route_words(ea.E) * 4);
#define SKINNY(AT_, GR_, NW_, NS_, KS_)                                                   \
  do {                                                                                    \
    if constexpr (MODE == MODE_UP) {                                                      \
      if (q.a_normw) {                                                                    \
        hipLaunchKernelGGL((k_expert_skinny<MODE, AT_, GR_, NW_, NS_, KS_, true>), grid, block, lds, s, q); \
        break;                                                                            \
      }                                                                                   \
    }                                                                                     \
    hipLaunchKernelGGL((k_expert_skinny<MODE, AT_, GR_, NW_, NS_, KS_>), grid, block, lds, s, q); \
  } while (0)
#define SKINNY_KS(AT_, GR_, NW_, NS_)                                                     \
  if constexpr (!GR_) {                                                                   \
    if (ks == 4) { if constexpr (NW_ <= 2) { SKINNY(AT_, GR_, NW_, NS_, 4); } }             \
    else if (ks == 2) { SKINNY(AT_, GR_, NW_, NS_, 2); } else { SKINNY(AT_, GR_, NW_, NS_, 1); } \
  } else { SKINNY(AT_, GR_, NW_, NS_, 1); }
#define SKINNY_NS(AT_, GR_, NW_)                                                          \
  if (ns == 2) { SKINNY_KS(AT_, GR_, NW_, 2); }                                           \
  else if constexpr (MODE == MODE_DOWN || NW_ % 2 == 0) { SKINNY_KS(AT_, GR_, NW_, 1); }
#define SKINNY_NW(AT_, GR_)                                                               \
  if (nw == 1) { SKINNY_NS(AT_, GR_, 1); } else if (nw == 2) { SKINNY_NS(AT_, GR_, 2); }  \
  else { SKINNY_NS(AT_, GR_, 4); }
    if (!split) {
      if (grouped) { SKINNY_NW(_Float16, true); } else { SKINNY_NW(_Float16, false); }
    } else {
      if (grouped) { SKINNY_NW(float, true); } else { SKINNY_NW(float, false); }
    }
#undef SKINNY_NW
#undef SKINNY_NS
#undef SKINNY_KS
#undef SKINNY
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

bool expert_uses_gemm(const ExpertArgs &ea) {
  // Prefill shapes (≥ 64 rows per expert on average): the grouped GEMM.
  const int max_active = ea.E < ea.A ? ea.E : ea.A;
  const bool want_gemm = ea.A >= 64 * max_active;
  return ea.calls == 1 && want_gemm && gemm_eligible(ea);
}

bool expert_stages_norm(const ExpertArgs &ea) {
  return ea.mode == MODE_UP && !expert_uses_gemm(ea) && ea.bits == 8 &&
         (ea.g == ea.K || ea.g % 32 == 0);
}

bool expert_fuses_route(const ExpertArgs &up, int J) {
  return expert_stages_norm(up) && up.A == up.k && up.a_row_div == up.k && up.E <= 256 &&
         up.k <= 16 && J >= 1 && J <= 16;
}

int launch_expert(const ExpertArgs &ea, const DispatchBufs &db, hipStream_t s) {
  if (ea.a_normw && (!expert_stages_norm(ea) || !ea.a_inv))
    return moe_fail(MOE_EXECUTION_FAILED, "expert: the staged pre-norm needs the skinny gate/up kernel");
  if (ea.mode == MODE_UP && ea.fr_partial && !expert_fuses_route(ea, ea.fr_J))
    return moe_fail(MOE_EXECUTION_FAILED, "expert: the fused route needs a single-token call on the skinny gate/up kernel");
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
  if (expert_uses_gemm(ea)) return launch_expert_gemm(ea, db, s);
  ExpertKArgs p;
  p.sorted = ea.dispatch_order;
  p.fr_partial = ea.mode == MODE_UP ? ea.fr_partial : nullptr;
  p.fr_b = ea.fr_b;
  p.fr_b_cs = ea.fr_b_cs;
  p.fr_J = ea.fr_J;
  p.fr_tile_m = ea.fr_tile_m;
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
  p.a_inv = ea.a_inv;
  p.a_normw = ea.a_normw;
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

template <typename RT>
static int combine_typed(const float *y, int64_t y_cs, int parts, int64_t part_cs,
                         const float *route, int64_t route_cs, const RT *residual, int64_t res_cs,
                         int T, int N, int E, int k, float *out, int64_t out_cs, int calls,
                         hipStream_t s) {
  auto a16 = [](const void *q) { return ((uintptr_t)q & 15) == 0; };
  const int pp = parts < 1 ? 1 : parts;
  if (N % 4 == 0 && (k <= 8 || k == 16) && a16(y) && a16(out) && (!residual || a16(residual)) &&
      y_cs % 4 == 0 && part_cs % 4 == 0 && out_cs % 4 == 0 && res_cs % 4 == 0) {
    dim3 grid(T, (N / 4 + 255) / 256, calls), block(256);
#define COMBINE4(KK_)                                                                        \
  case KK_:                                                                                  \
    hipLaunchKernelGGL((k_combine4<KK_, RT>), grid, block, 0, s, y, y_cs, pp, part_cs, route, \
                       route_cs, residual, res_cs, T, N, E, out, out_cs);                    \
    return 0;
    switch (k) {
      COMBINE4(1) COMBINE4(2) COMBINE4(3) COMBINE4(4) COMBINE4(5) COMBINE4(6) COMBINE4(7)
      COMBINE4(8) COMBINE4(16)
    }
#undef COMBINE4
  }
  dim3 grid(T, (N + 255) / 256, calls), block(256);
  hipLaunchKernelGGL(k_combine<RT>, grid, block, 0, s, y, y_cs, pp, part_cs, route, route_cs,
                     residual, res_cs, T, N, E, k, out, out_cs);
  return 0;
}

int launch_combine(const float *y, int64_t y_cs, int parts, int64_t part_cs, const float *route,
                   int64_t route_cs, const void *residual, moe_dtype res_dtype, int64_t res_cs,
                   int T, int N, int E, int k, float *out, int64_t out_cs, int calls,
                   hipStream_t s) {
  MOE_NONNULL(y);
  MOE_NONNULL(route);
  MOE_NONNULL(out);
  if (res_dtype == MOE_F16)
    return combine_typed(y, y_cs, parts, part_cs, route, route_cs, (const _Float16 *)residual,
                         res_cs, T, N, E, k, out, out_cs, calls, s);
  return combine_typed(y, y_cs, parts, part_cs, route, route_cs, (const float *)residual, res_cs,
                       T, N, E, k, out, out_cs, calls, s);
}

int launch_zero(float *p, size_t n, hipStream_t s) {
  MOE_NONNULL(p);
  size_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks == 0) return 0;
  hipLaunchKernelGGL(k_zero, dim3((unsigned)blocks), dim3(256), 0, s, p, n);
  return 0;
}
