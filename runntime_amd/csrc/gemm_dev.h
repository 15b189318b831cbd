// Device helpers shared by the grouped-GEMM kernels (gemm.hip, gemm_wide.hip):
// operand types, the int8 → f16 conversion, direct-to-LDS buffer loads,
// explicit vmcnt waits and the kernel argument block.
#pragma once
#include "moe_internal.h"

// Arguments of the grouped-GEMM kernels (shared by both translation units).
struct GemmArgs {
  const void *a;
  int a_bytes;  // size of a (bounds of its buffer loads)
  int a_row_div;
  const uint32_t *w0;  // glu (up) or down
  const float *s0;
  const float *b0;
  const uint32_t *w1;  // lin (up); down: w0 again
  const float *s1;
  const float *b1;
  int K, N, E;         // N: output columns (up: I, per projection)
  float *out;
  int out_bytes;  // size of out (bounds of its buffer stores)
  const int32_t *perm;
  int perm_bytes;
  const int32_t *active;  // [E][4] {e, first row, rows, first M-tile}
  const int32_t *meta;
  int nt;                 // N-tiles
  int sorted;             // act in dispatch order: up writes row r0 + row, down reads it
  int parts;              // K parts (down); part q writes out + q·A·N
  int kpart;              // steps per part
  int part_floats;        // A·N
  int act_i8;             // up: write act as int8 limbs (gemm_i8.hip's layout)
  int act_npairs;         // up with act_i8: N / 64
};

// The wide up kernel (gemm_wide.hip): f16 x, K in whole groups of four
// steps and at least 16 steps.
bool gemm_wide_eligible(const ExpertArgs &ea);
// omode: 0 f32 act, 1 f16 hi + lo pairs, 2 int8 limbs (gemm_i8.hip).
int launch_gemm_up_wide(const GemmArgs &p, int blocks, int omode, hipStream_t s);
// The down product of the fused layer on the int8 matrix cores (gemm_i8.hip).
int launch_gemm_down_i8(const ExpertArgs &dn, const DispatchBufs &db, int cus, hipStream_t s);

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// act between the two products of the fused layer (dispatch order): each
// f32 value v as its f16 split hi = f16(v), lo = f16(v − hi), per pair of
// columns n, n + 1 (n even): hi(n), hi(n + 1), lo(n), lo(n + 1), 8 bytes at
// the f32 pair's place. Up stores exactly where the f32 values would go;
// down takes its hi and lo operands from dwords 0, 2 and 1, 3 of the
// 16-byte chunks it reads, with no conversion.
struct f16pair {
  _Float16 hi, lo;
};

constexpr int WAVE = 64;
constexpr int BM = GEMM_TILE_M;  // 128 rows
constexpr int BK = 32;           // k per step
constexpr int TPS = BK / 4;      // quantW tiles per unit per step
constexpr int SLOTS = 128;       // weight units per block (2 sources × 64)
constexpr int W_BYTES = SLOTS * TPS * 16;  // weights of one step: 16 KB
// Largest active-expert count (descriptors cached in LDS).
constexpr int GEMM_MAX_E = 256;
// Word 3 of a raw buffer resource on gfx9-family parts (32-bit data format).
constexpr int BUF_DWORD3 = 0x00020000;



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

// 8 int8 q (k order, little-endian in two words) → 8 f16 q. Flipping the
// sign bit gives u = q + 128; placing u under the exponent byte 0x64 gives
// the f16 1024 + u; minus 1152 leaves q exactly.
__device__ __forceinline__ uint32_t u8x2_to_h2(uint32_t x, uint32_t sel) {
  const half2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  return __builtin_bit_cast(
      uint32_t, __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, x, sel)) - bias);
}
__device__ __forceinline__ half8 cvt_i8x8(uint32_t x0, uint32_t x1) {
  x0 ^= 0x80808080u;
  x1 ^= 0x80808080u;
  const u32x4 r = {u8x2_to_h2(x0, 0x04010400u), u8x2_to_h2(x0, 0x04030402u),
                   u8x2_to_h2(x1, 0x04010400u), u8x2_to_h2(x1, 0x04030402u)};
  return __builtin_bit_cast(half8, r);
}

__device__ __forceinline__ int sw8(int r) { return (r ^ (r >> 3)) & 7; }
// Weight slots: sw8, with slots 64-127 (up: lin) moved to the other bank
// groups (bit 0 flipped) when TALL wavefronts read both sources' tiles at
// the same 8-byte half in one 32-lane group.
template <bool TALL>
__device__ __forceinline__ int sw8w(int s) { return sw8(s) ^ (TALL ? (s >> 6) & 1 : 0); }

// One buffer_load_dwordx4 … lds: 16 bytes per lane from rsrc at voff + soff
// into LDS at lds_addr + 16·lane. Written as asm so that the compiler, which
// does not track these loads, adds no waits for them; the loop's explicit
// vmcnt waits order them. (The compiler's own waits for other vector loads
// only count its own loads and so can only wait longer with these in
// flight.) M0 holds the LDS address; nothing else in this kernel uses M0.
__device__ __forceinline__ i32x4 uniform4(i32x4 v) {
  return i32x4{__builtin_amdgcn_readfirstlane(v[0]), __builtin_amdgcn_readfirstlane(v[1]),
               __builtin_amdgcn_readfirstlane(v[2]), __builtin_amdgcn_readfirstlane(v[3])};
}
__device__ __forceinline__ void dma16(i32x4 rsrc, uint32_t voff, int soff, uint32_t lds_addr) {
  rsrc = uniform4(rsrc);
  soff = __builtin_amdgcn_readfirstlane(soff);
  lds_addr = __builtin_amdgcn_readfirstlane(lds_addr);
  asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :: "v"(voff), "s"(rsrc), "s"(soff), "s"(lds_addr) : "memory");
}
__device__ __forceinline__ i32x4 buffer_rsrc(const void *base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  return i32x4{(int)(uint32_t)a, (int)(uint32_t)(a >> 32), (int)bytes, BUF_DWORD3};
}

// The same for 4 bytes per lane (LDS at lds_addr + 4·lane).
__device__ __forceinline__ void dma4(i32x4 rsrc, uint32_t voff, int soff, uint32_t lds_addr) {
  rsrc = uniform4(rsrc);
  soff = __builtin_amdgcn_readfirstlane(soff);
  lds_addr = __builtin_amdgcn_readfirstlane(lds_addr);
  asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dword %0, %1, %2 offen lds"
               :: "v"(voff), "s"(rsrc), "s"(soff), "s"(lds_addr) : "memory");
}

// s_waitcnt with vmcnt = n (< 64) and no wait on the other counters.
#define WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

// Workgroup barrier without a memory fence (a fence would wait for every
// load in flight); the asm statements keep the compiler from moving LDS
// accesses across it.
__device__ __forceinline__ void block_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// One tile of the grouped GEMM, uniform across the block.
struct Tile {
  int e;     // expert
  int r0;    // first sorted row (dispatch order) of the tile
  int rows;  // rows of the tile (≤ BM)
  int U0, U1;  // first unit of each weight source
  int part;  // K part
  int kb;    // first step of the part
  int mtg;   // global index of the M-tile (padded rows 128·mtg ..)
};


}  // namespace
