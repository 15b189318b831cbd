// RMSNorm's canonical inverse RMS of one row, for kernels that normalise
// their input while staging it (the router chunks and the gate/up product of
// moe_block) instead of reading a normalised copy from memory.
//
// Reference: src/core/kernels/reduce/rmsNorm.ts:84-140 (f32 sums, then
// v = x·inv·w stored in the input dtype). The order is norm.hip's canonical
// one, so a fused kernel sees the same bits the standalone norm writes:
// lane l sums the quads q ≡ l (mod 64) of the row in ascending q, each
// quad's elements in ascending order (s = s + x·x, no fused multiply-add:
// including files are compiled with -ffp-contract=off); the 64 lane sums
// meet in an xor butterfly, strides 32 … 1; inv = 1 / sqrt(s / n + eps).
#pragma once
#include "moe_internal.h"

namespace moe_dev {

template <typename T>
__device__ __forceinline__ float wave_row_inv(const T *x, int n, float eps, int lane) {
  float s = 0.f;
  for (int q = lane; 4 * q < n; q += 64) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int i = 4 * q + j;
      if (i < n) {
        const float v = (float)x[i];
        s = s + v * v;
      }
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) s = s + __shfl_xor(s, m);
  return 1.0f / sqrtf(s / (float)n + eps);
}

// The normalised value as the standalone norm stores it: x·inv·w in f32,
// left to right, rounded to the input dtype. The f32 product is rounded
// before the conversion: the empty asm keeps the compiler from merging the
// last multiply and the conversion to f16 into one mixed-precision fma
// (v_fma_mixlo_f16), which rounds once and so differs in the last f16 bit.
template <typename T>
__device__ __forceinline__ float norm_value(float x, float inv, float w) {
  float v = x * inv * w;
  __asm__ volatile("" : "+v"(v));
  return (float)(T)v;
}

}  // namespace moe_dev
