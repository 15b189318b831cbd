// Grouped down GEMM of the fused prefill layer on the int8 matrix cores.
//
// Reference: src/core/kernels/matmul/moeQuantW.ts:188-237 (moeDown: the
// routed act rows times the expert's int8 down weights, per-column scale and
// bias); quantW layout src/core/kernels/quantCommon.ts:8-31.
//
// act between the two products is private to the layer. The gate/up GEMM
// writes every f32 act value v as the 24-bit fixed-point integer
// V = rint(v · 2^17) (|act| ≤ 56 by the clamped SwiGLU, so |V| < 2^23),
// stored as three signed bytes with V = 65536·h + 256·m + l. The rounding
// error is at most 2^-18 per act value; through K = 5632 weights of
// |q·scale| ~ 0.09 it moves an output by ~1.5e-5 (rms), far inside the
// 2e-3 bar, where f16 act alone (11 bits) would move it by ~7e-3. Down runs
// three exact v_mfma_i32_32x32x32_i8 per product (limbs h, m, l against the
// int8 weights, i32 accumulation: |Σ| ≤ 128·128·K, below 2^31 for
// K < 131,072) and adds the limbs exactly in the epilogue (int64), rounding
// once to f32. Against the f16 hi + lo form this is 3 int8 MFMAs (each half
// an f16 MFMA's time) instead of 4 f16 per 32 k, and the weights feed the
// matrix cores as loaded: no int8 → f16 conversion at all.
//
// The limbs: W = V + 32896 as a 24-bit two's complement integer has bytes
// b0, b1, b2; l = b0 ^ 0x80 and m = b1 ^ 0x80 read as signed bytes are
// b0 − 128 and b1 − 128, and h = b2 (signed), so l + 256·m + 65536·h =
// W − 32896 = V.
//
// act layout (bytes), over padded rows: the sorted row p of expert e sits
// at padded row P = 128·(first M-tile of e) + (p − first row of e), so each
// 64-row block of P holds rows of one expert. Block b, pair of steps j
// (64 k), limb L, step q of the pair, 16-k half hf: a 1 KB chunk of 64 rows
// × 16 bytes (k = 64j + 32q + 16hf + 0..15, in order) at
//   ((b·(K/64) + j)·12 + (2L + q)·2 + hf)·1024 + (P mod 64)·16.
// A pair of a block is one contiguous 12 KB run: its direct-to-LDS loads
// are whole lines, and its LDS image is the MFMA A fragments as they are
// read (16 lanes read 256 contiguous bytes).
//
// Tiles: 64 rows (one act block) × 128 units (512 columns) per block of
// eight wavefronts, two per SIMD. Wavefront w takes rows 32·(w >> 2) ..
// + 31 and units 32·(w & 3) .. + 31: 4 column tiles × 3 limbs = 12 MFMAs
// per 32 k and 192 i32 accumulators, so two wavefronts fit a SIMD and each
// hides the other's waits (one wavefront per SIMD with 64 rows × 32 units
// needs 384 accumulators and measured 15-25% slower). Lane l = 32hf + u
// holds unit u of the group for k half hf: per step it reads the unit's 64
// bytes for its half (four quantW tiles of 4 columns × 4 k), and column c's
// dwords of the four tiles are the B operand of column tile c (columns
// 4u + c): no exchange between lanes. act and the weights both come through
// LDS rings of step pairs filled by direct-to-LDS loads of whole lines.
//
// Measured at config 4 (per launch, on one box): the loads alone (no
// MFMAs) take 0.87 M cycles at 2.24 GHz, the MFMAs and LDS reads alone
// 0.82 M cycles at 2.06 GHz, the kernel 1.1 M cycles at 1.81 GHz: under the
// full load the clock drops (power), which is most of what separates the
// kernel from its parts.
//
// Order of tiles: expert, then N-tile, then 64-row block, cut into 8
// contiguous ranges, one per XCD (block b runs on XCD b mod 8), so the
// blocks of an (expert, N-tile) — which share its weights — and the N-tiles
// of a row block — which share its act — run at once on one L2.
#include "gemm_dev.h"


namespace {

typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

constexpr int I8_WAVES = 8;
constexpr int I8_BM = 64;                        // rows per tile (one act block)
constexpr int I8_UNITS = 128;                    // weight units per tile
constexpr int I8_SPA = 4;                        // act ring stages (step pairs)
constexpr int I8_SPW = 3;                        // weight ring stages (step pairs)
constexpr int I8_PAIR = I8_BM * 64 * 3;          // act bytes of one pair: 12 KB
constexpr int I8_LOADS = 6;                      // loads per wavefront and pair (2 act, 4 weights)
constexpr int I8_WPAIR = 4 * 2 * 32 * 128;        // weights of one pair: 32 KB
constexpr int I8_MAX_E = GEMM_MAX_E;
// Offset past every buffer: a load there fetches nothing (the range check
// drops it) and lands zeros in the junk area; keeps each wavefront's load
// count fixed without moving bytes.
constexpr uint32_t I8_NOFETCH = 0x80000000u;

struct I8Args {
  const uint8_t *act;      // limbs, layout above
  uint32_t act_bytes;
  const uint8_t *w;        // quantW words of the down weight [E·K, N]
  const float *scales;     // [E, N]
  const float *bias;       // [E, N] or NULL
  float *y;                // [A, N] f32, row = assignment
  uint32_t y_bytes;
  const int32_t *perm;     // sorted position → assignment
  const int32_t *active;   // [E][4] {e, first row, rows, first M-tile}
  const int32_t *meta;
  int K, N, E;
  int nt;                  // N-tiles (512 columns each)
};

__device__ __forceinline__ int fresh_lane_i8() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_gemm_down_i8(I8Args p) {
  __shared__ __align__(16) uint8_t aring[I8_SPA * I8_PAIR];   // 48 KB
  __shared__ __align__(16) uint8_t wring[I8_SPW * I8_WPAIR];  // 96 KB
  __shared__ __align__(16) uint8_t junk[1024];
  __shared__ int32_t rowmap[2][I8_BM];  // this tile's and the next one's
  __shared__ int4 descs[I8_MAX_E];
  __shared__ int c64[I8_MAX_E + 1];  // cumulative 64-row blocks per active expert

  const int n_active = p.meta[META_ACTIVE];
  const int tid = threadIdx.x;
  for (int i = tid; i < n_active; i += blockDim.x) descs[i] = ((const int4 *)p.active)[i];
  __syncthreads();
  if (tid < 64) {
    // One wavefront scans the per-expert block counts (ceil(rows / 64)).
    int carry = 0;
    for (int base = 0; base < n_active; base += 64) {
      const int i = base + tid;
      int v = i < n_active ? (descs[i].z + I8_BM - 1) / I8_BM : 0;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(v, o, 64);
        if (tid >= o) v += t;
      }
      if (i < n_active) c64[i + 1] = carry + v;
      carry += __shfl(v, 63, 64);
    }
    if (tid == 0) c64[0] = 0;
  }
  __syncthreads();
  const int total = c64[n_active] * p.nt;
  const int bx = gridDim.x >> 3;
  const int xcd = blockIdx.x & 7, xb = blockIdx.x >> 3;
  const int per_x = (total + 7) >> 3;
  const int start = xcd * per_x + xb, end = min(total, (xcd + 1) * per_x);

  const int lane = tid & (WAVE - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
  const int rg = wave >> 2, cg = wave & 3;  // row half, unit group of the wavefront
  const int hf = lane >> 5, u = lane & 31;
  const int N4 = p.N / 4;
  const int ksteps = p.K / BK, npairs = ksteps / 2;
  const uint64_t slab = (uint64_t)p.K * (uint64_t)p.N;
  const i32x4 ar = buffer_rsrc(p.act, p.act_bytes);
  const uint32_t aring0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)aring;
  const uint32_t wring0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)wring;
  const uint32_t junk0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)junk;
  const __amdgpu_buffer_rsrc_t yrc = __builtin_amdgcn_make_buffer_rsrc(p.y, 0, p.y_bytes, BUF_DWORD3);
  const int swu = sw8(u);

  // ---- a tile: expert (binary search over the block counts), N-tile, row
  // block. Tiles of active expert i: c64[i]·nt .. c64[i + 1]·nt. Past the
  // block's range a tile is invalid and only its loads' validity is read.
  struct TileP {
    int e, r0, rows, U0;
    uint32_t a_base;  // act bytes of the tile's row block
    bool valid;
  };
  auto decode = [&](int L) {
    TileP T{0, 0, 1, 0, 0u, false};
    if (L >= end) return T;
    int lo = 0, hi = n_active - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (c64[mid] * p.nt <= L) lo = mid; else hi = mid - 1;
    }
    const int4 d = descs[lo];
    const int nb = c64[lo + 1] - c64[lo];
    const int local = L - c64[lo] * p.nt;
    const int ntile = local / nb, jb = local % nb;
    T.e = __builtin_amdgcn_readfirstlane(d.x);
    T.r0 = __builtin_amdgcn_readfirstlane(d.y + jb * I8_BM);  // first sorted row
    T.rows = __builtin_amdgcn_readfirstlane(min(I8_BM, d.z - jb * I8_BM));
    T.U0 = ntile * I8_UNITS;
    const int blk = __builtin_amdgcn_readfirstlane(2 * d.w + jb);  // act block
    T.a_base = (uint32_t)blk * (uint32_t)npairs * (uint32_t)I8_PAIR;
    T.valid = true;
    return T;
  };

  // Loads of a pair, 6 per wavefront: act chunks 2w, 2w + 1 (12 chunks of
  // 1 KB over wavefronts 0-5; wavefronts 6 and 7 issue fetch-free loads into
  // the junk area, so that every wavefront issues the same count), then the
  // weights of step rg of the pair for units 32·cg .. 32·cg + 31:
  // instruction i loads units 8i .. 8i + 7 of the group, lane l the 16-byte
  // chunk (l & 7) ^ sw8(unit) of unit 8i + (l >> 3)'s 128 bytes, so that
  // chunk c of unit u sits at u·128 + (c ^ sw8(u))·16 (the 16 lanes reading
  // one tile of 16 units hit 16 different bank groups). A unit past N loads
  // from past the buffer (zeros, no fetch; its outputs are not stored).
  // Pairs past a tile's last are the next tile's first (the ring runs on
  // across the block's tiles); past the block's last tile every load goes
  // to the junk area, fetch-free. Branch-free: a load under a branch makes
  // the compiler wait for every load in flight where the paths join.
  auto woffs = [&](const TileP &T, uint32_t (&wo)[4]) {
    const int ln = fresh_lane_i8();
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int uu = 8 * i + (ln >> 3);
      const int ug = T.U0 + 32 * cg + uu;
      wo[i] = ug < N4 ? (uint32_t)ug * (uint32_t)p.K * 4u + (uint32_t)((ln & 7) ^ sw8(uu)) * 16u
                      : I8_NOFETCH;
    }
  };
  TileP T = decode(start), Tn = decode(start + bx);  // this tile, the next
  uint32_t woff[4], woffn[4];
  woffs(T, woff);
  woffs(Tn, woffn);
  i32x4 wr = buffer_rsrc(p.w + (uint64_t)T.e * slab, (uint32_t)slab);
  i32x4 wrn = buffer_rsrc(p.w + (uint64_t)Tn.e * slab, (uint32_t)slab);

  // Pair ja of act, jw of the weights, counted from this tile's first
  // (≥ npairs: the next tile's).
  auto issue_one = [&](int n, int ja, int sa_, int jw, int sw_) {
    if (n < 2) {
      const int c = 2 * wave + n;
      const bool nx = ja >= npairs;
      const int jj = nx ? ja - npairs : ja;
      const bool ok = (nx ? Tn.valid : T.valid) && c < 12;
      const uint32_t at = (nx ? Tn.a_base : T.a_base) + (uint32_t)jj * I8_PAIR +
                          (uint32_t)c * 1024u + (uint32_t)fresh_lane_i8() * 16u;
      dma16(ar, ok ? at : I8_NOFETCH, 0, ok ? aring0 + sa_ * I8_PAIR + c * 1024 : junk0);
    } else {
      const int i = n - 2;
      const bool nx = jw >= npairs;
      const int jj = nx ? jw - npairs : jw;
      const bool ok = (nx ? Tn.valid : T.valid) && jj >= 0;
      dma16(nx ? wrn : wr, ok ? (nx ? woffn[i] : woff[i]) : I8_NOFETCH,
            ok ? (2 * jj + rg) * (BK * 4) : 0,
            ok ? wring0 + sw_ * I8_WPAIR + cg * 8192 + rg * 4096 + i * 1024 : junk0);
    }
  };
  auto issue_pair = [&](int ja, int sa_, int jw, int sw_) {
#pragma unroll
    for (int n = 0; n < I8_LOADS; n++) issue_one(n, ja, sa_, jw, sw_);
  };

  // The pipeline: after the barrier of pair j (its loads landed, every read
  // of pair j − 1 done), the act loads of pair j + SPA − 1 and the weight
  // loads of pair j + SPW − 1 go into pair j − 1's stages, spread between
  // the MFMA groups of step 2j (all wavefronts issuing them in one burst
  // stalls the matrix cores together). At the wait of pair j, its weights
  // (issued one pair after its act) are followed by exactly one pair's
  // I8_LOADS younger instructions. The stages rotate over the block's whole
  // run of pairs; only its first tile has a prologue, which issues virtual
  // pairs −(SPA − 1) .. −1 of the same pattern.
  static_assert(I8_SPA == I8_SPW + 1, "act runs one pair ahead of the weights");
  if (T.valid) {
#pragma unroll
    for (int v = 0; v < I8_SPA - 1; v++) issue_pair(v, v, v - 1, v - 1);
  }

  // Fragments of step q of the pair: act rows 32·rg + u, limb l3, half hf;
  // the unit's four quantW tiles for half hf (tile t = columns 0..3 × k
  // 4t .. 4t + 3).
  struct Frags {
    u32x4 a[3];
    u32x4 w[4];
  };
  auto read_frags = [&](Frags &F, int sa, int sw, int q) {
    const uint8_t *s = aring + sa * I8_PAIR + hf * 1024 + (32 * rg + u) * 16 + q * 2048;
#pragma unroll
    for (int l3 = 0; l3 < 3; l3++) F.a[l3] = *(const u32x4 *)(s + l3 * 4096);
    const uint8_t *t = wring + sw * I8_WPAIR + cg * 8192 + q * 4096 + u * 128;
#pragma unroll
    for (int j4 = 0; j4 < 4; j4++) F.w[j4] = *(const u32x4 *)(t + ((hf * 4 + j4) ^ swu) * 16);
  };

  int sa = 0, sw = 0, rb = 0;
  for (int L = start; L < end; L += bx) {
    // ---- tile start: its row map and epilogue constants. Their one wait
    // (the compiler's, for every load in flight) also covers this tile's
    // first pairs, issued under the previous tile, and that tile's stores.
    const int uo = T.U0 + 32 * cg + u;
    const bool col_ok = uo < N4;
    const int col = 4 * min(uo, N4 - 1);
    const int rmv = tid < I8_BM ? p.perm[T.r0 + min(tid, T.rows - 1)] : 0;
    const floatx4 sc = *(const floatx4 *)(p.scales + (size_t)T.e * p.N + col) * (1.0f / 131072.0f);
    floatx4 bs = {0.f, 0.f, 0.f, 0.f};
    if (p.bias) bs = *(const floatx4 *)(p.bias + (size_t)T.e * p.N + col);
    if (tid < I8_BM) rowmap[rb][tid] = rmv;
    asm volatile("" ::"v"(sc), "v"(bs));

    i32x16 acc[4][3];
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
      for (int l3 = 0; l3 < 3; l3++) acc[c][l3] = i32x16{};
    // The 12 MFMAs of a step; hook(c) runs after column tile c's three.
    auto mfmas = [&](const Frags &F, auto hook) {
#pragma unroll
      for (int c = 0; c < 4; c++) {
        // Column c's dwords of the four quantW tiles: 16 k of column 4u + c.
        const i32x4 B = {(int)F.w[0][c], (int)F.w[1][c], (int)F.w[2][c], (int)F.w[3][c]};
#pragma unroll
        for (int l3 = 0; l3 < 3; l3++)
          acc[c][l3] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, F.a[l3]), B,
                                                             acc[c][l3], 0, 0, 0);
        hook(c);
      }
    };

    for (int j = 0; j < npairs; j++) {
      WAIT_VMCNT(I8_LOADS);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      block_barrier();
      const int ja = j + I8_SPA - 1, jw = j + I8_SPW - 1;
      const int na = sa == 0 ? I8_SPA - 1 : sa - 1, nw = sw == 0 ? I8_SPW - 1 : sw - 1;
      Frags F;
      read_frags(F, sa, sw, 0);
      mfmas(F, [&](int c) {
        issue_one(c, ja, na, jw, nw);
        if (c < 2) issue_one(c + 4, ja, na, jw, nw);
      });
      read_frags(F, sa, sw, 1);
      mfmas(F, [](int) {});
      sa = sa + 1 == I8_SPA ? 0 : sa + 1;
      sw = sw + 1 == I8_SPW ? 0 : sw + 1;
    }

    // ---- epilogue: y[assignment][col .. col + 3] = scale · V-sum · 2^-17
    // + bias, for columns 4·unit' + 0..3 of the lane. The row map was
    // written before this tile's first barrier.
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int row = 32 * rg + 8 * (r / 4) + 4 * hf + (r % 4);
      // the exact sum 65536·h + 256·m + l (int64), rounded once to f32
      floatx4 o;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const int64_t v = ((int64_t)acc[c][0][r] << 16) + ((int64_t)acc[c][1][r] << 8) +
                          (int64_t)acc[c][2][r];
        o[c] = __builtin_fmaf((float)v, sc[c], bs[c]);
      }
      const uint32_t off = (row < T.rows && col_ok)
                               ? ((uint32_t)rowmap[rb][row] * (uint32_t)p.N + (uint32_t)col) * 4u
                               : 0x80000000u;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), yrc, off, 0, 0);
    }
    // ---- the next tile (its first pairs are in flight); the one after.
    T = Tn;
#pragma unroll
    for (int i = 0; i < 4; i++) woff[i] = woffn[i];
    wr = wrn;
    Tn = decode(L + 2 * bx);
    woffs(Tn, woffn);
    wrn = buffer_rsrc(p.w + (uint64_t)Tn.e * slab, (uint32_t)slab);
    rb ^= 1;
  }
  // Loads past the last tile (fetch-free) still land in the junk area: wait
  // for them before the workgroup's LDS goes away.
  WAIT_VMCNT(0);
}

}  // namespace

bool gemm_i8_down_eligible(const ExpertArgs &dn) {
  // 8-bit weights with one scale group per column, K in whole step pairs
  // with at least a ring's worth of them, 32-bit buffer offsets, and i32
  // limb sums that cannot overflow (|limb · q| ≤ 128 · 128 per k).
  const int64_t mt = (dn.A + BM - 1) / BM + (dn.E < dn.A ? dn.E : dn.A);
  return dn.mode == MODE_DOWN && dn.bits == 8 && dn.g == dn.K && dn.K % 64 == 0 &&
         dn.K / 64 >= I8_SPA && dn.K < (1 << 17) && dn.N % 4 == 0 && dn.E <= I8_MAX_E &&
         dn.calls == 1 &&
         gemm_i8_act_bytes(dn.A, dn.E, dn.K) < (1ll << 31) &&
         (int64_t)dn.A * dn.N * 4 < (1ll << 31) && (int64_t)dn.K * dn.N < (1ll << 31) &&
         mt > 0;
}

int64_t gemm_i8_act_bytes(int A, int E, int K) {
  const int64_t mt = (A + BM - 1) / BM + (E < A ? E : A);
  return mt * BM * (int64_t)K * 3;
}

int launch_gemm_down_i8(const ExpertArgs &dn, const DispatchBufs &db, int cus, hipStream_t s) {
  I8Args p;
  p.act = (const uint8_t *)dn.a;
  p.act_bytes = (uint32_t)gemm_i8_act_bytes(dn.A, dn.E, dn.K);
  p.w = (const uint8_t *)dn.w0.w;
  p.scales = dn.w0.scales;
  p.bias = dn.w0.bias;
  p.y = dn.out;
  p.y_bytes = (uint32_t)((int64_t)dn.A * dn.N * 4);
  p.perm = db.perm;
  p.active = db.active;
  p.meta = db.meta;
  p.K = dn.K;
  p.N = dn.N;
  p.E = dn.E;
  p.nt = (dn.N + 511) / 512;
  long blocks = ((long)(dn.A + I8_BM - 1) / I8_BM + dn.E) * p.nt;
  if (blocks > cus) blocks = cus;
  blocks = (blocks + 7) / 8 * 8;
  hipLaunchKernelGGL(k_gemm_down_i8, dim3((unsigned)blocks), dim3(I8_WAVES * WAVE), 0, s, p);
  return 0;
}
