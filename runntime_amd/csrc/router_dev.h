// Top-k gating of one token by one wavefront, shared by the router kernels
// of router.hip (the chunk fold with and without the fused dispatch, and the
// standalone topk), which must pick the same ids and gates bit for bit.
//
// Reference: src/core/kernels/reduce/topkSelect.ts:21-92 (selection) and
// :142-156 (softmax over the selected logits). Each lane owns experts lane,
// lane + 64, …; k rounds of a butterfly arg-max (ties → lower id) pick the
// winners: the reference's bubble insertion restated for a wavefront. A
// logit is a candidate only if it is strictly above the reference's
// −3.4e38 start value (so NaN never enters), and a slot no candidate fills
// keeps (−3.4e38, id 0), as the reference's does. Both including files are
// compiled with -ffp-contract=off.
#pragma once
#include "dispatch_dev.h"

namespace moe_dev {

constexpr float NEG_START = -3.4e38f;

// (v, e) arg-max over the wavefront; larger v wins, equal v → lower e. The
// order is total, so every lane ends with the same winner whatever the
// tree. Within 16 lanes the partners come from DPP (quad xor 1, quad xor
// 2, half-row mirror, row mirror: register moves, no LDS trip); across the
// rows from two xor shuffles.
template <int CTRL>
__device__ __forceinline__ void argmax_dpp(float &v, int &e) {
  const float ov = __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
  const int oe = __builtin_amdgcn_mov_dpp(e, CTRL, 0xf, 0xf, false);
  const bool take = (ov > v) || (ov == v && oe < e);
  v = take ? ov : v;
  e = take ? oe : e;
}
__device__ __forceinline__ void wave_argmax(float &v, int &e) {
  argmax_dpp<0xB1>(v, e);   // quad_perm [1, 0, 3, 2]
  argmax_dpp<0x4E>(v, e);   // quad_perm [2, 3, 0, 1]
  argmax_dpp<0x141>(v, e);  // row_half_mirror
  argmax_dpp<0x140>(v, e);  // row_mirror
#pragma unroll
  for (int m = 16; m < WAVE; m <<= 1) {
    float ov = __shfl_xor(v, m);
    int oe = __shfl_xor(e, m);
    bool take = (ov > v) || (ov == v && oe < e);
    v = take ? ov : v;
    e = take ? oe : e;
  }
}

// Selects the top k of the wavefront's logits and writes the route row.
// vals[i] is expert lane + 64·i (i < NI). Round r's winner is kept by lane r.
// Then w_i = exp(v_i − v_0) / Σ_j exp(v_j − v_0), the sum taken left to right
// (topkSelect.ts:142-156); lane i < k writes slot i.
template <int NI>
__device__ __forceinline__ int wave_topk_route(const float (&vals)[NI], int E, int k, int lane,
                                               float *row) {
  uint64_t taken = 0;
  float my_v = NEG_START;
  int my_id = 0;
#pragma unroll 1
  for (int r = 0; r < k; r++) {
    float bv = -INFINITY;
    int be = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < NI; i++) {
      int e = lane + WAVE * i;
      float v = vals[i];
      bool cand = (e < E) && !((taken >> i) & 1ull) && (v > NEG_START);
      if (cand && v > bv) {  // ascending e and strict > keep the lower id
        bv = v;
        be = e;
      }
    }
    wave_argmax(bv, be);
    float sv = NEG_START;  // no candidate left: the reference's untouched slot
    int si = 0;
    if (be != 0x7fffffff) {
      sv = bv;
      si = be;
      if ((be & (WAVE - 1)) == lane) taken |= 1ull << (be / WAVE);
    }
    if (lane == r) {
      my_v = sv;
      my_id = si;
    }
  }
  // Lane reads go through readlane (a register read, no LDS trip).
  auto lane_f = [](float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
  };
  float m = lane_f(my_v, 0);
  float ex = expf(my_v - m);
  float z = lane_f(ex, 0);
#pragma unroll 1
  for (int i = 1; i < k; i++) z = z + lane_f(ex, i);
  if (lane < k) {
    row[lane] = (float)my_id;
    row[k + lane] = ex / z;
  }
  return my_id;
}

}  // namespace moe_dev
